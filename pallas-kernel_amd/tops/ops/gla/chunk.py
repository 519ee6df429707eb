"""Chunked GLA on the MI355X HIP kernels, mirroring ``tops/ops/gla/chunk.py``.

Public names, argument meanings and return conventions follow the reference (cited per
function); arrays are torch tensors on a ROCm device instead of jax arrays, and the
reference's missing autodiff rule is provided by ``torch.autograd.Function`` (the role
``jax.custom_vjp`` plays in the JAX API): ``chunk_gla`` is differentiable w.r.t. q, k, v,
g (or g_gamma) and initial_state.

Kernels compute the chunk-local cumsum of the gates in-kernel, handle a partial last chunk
and varlen sequences natively (no padding copies on the hot path), and keep every
accumulation in float32. bfloat16 inputs feed bf16 MFMA; float32 inputs feed f32 MFMA.
"""

from __future__ import annotations

import math

import torch

from ... import _lib
from ..._lib import SeqLayout, call, check_device, dtype_code, ptr, require, stream_of
from ...utils import pad_to_multiple

__all__ = [
    "chunk_gla",
    "chunk_local_cumsum",
    "chunk_local_cumsum_vector",
    "chunk_local_cumsum_ref",
    "chunk_fwd_h",
    "chunk_fwd_h_ref",
    "chunk_gla_fwd_intra_gk",
    "chunk_gla_fwd_o_gk",
    "chunk_gla_fwd",
    "chunk_gla_bwd",
    "chunk_gla_bwd_with_pl",
    "chunk_gla_bwd_dA_ref",
    "chunk_gla_bwd_dv_ref",
    "chunk_gla_bwd_dqk_intra_ref",
    "chunk_gla_bwd_dqkg_ref",
]

# chunk sizes of the per-chunk kernels (4 and 8 on the small-chunk vector kernels)
_KERNEL_CHUNKS = (4, 8, 16, 32, 64)


def _kernel_chunk(chunk_size: int) -> int:
    """Chunk size used by the kernels for chunk-size-independent results (o, ht, grads).

    The outputs are mathematically independent of the chunk size, so every power of two
    runs on 64-row chunks: the full-head kernels' size, and the most work per chunk for
    the others.
    """
    c = int(chunk_size)
    require(c > 0 and c & (c - 1) == 0, "chunk_size must be power of 2")
    return 64


def _compute_dtype(*xs):
    """bf16 if every given tensor is bf16, else float32 (f16 / mixed are upcast)."""
    dts = {x.dtype for x in xs if x is not None}
    return torch.bfloat16 if dts == {torch.bfloat16} else torch.float32


def _c(x, dt=None):
    if x is None:
        return None
    if dt is not None and x.dtype != dt:
        x = x.to(dt)
    return x.contiguous()


def _full_head(K, V, C, dtype, backward, *tensors):
    """The full-head kernels will run (shape and 16-byte aligned buffers): state
    workspaces they do not use need not be allocated."""
    if any(t is not None and t.data_ptr() % 16 for t in tensors):
        return False
    return _lib.full_head(K, V, C, dtype, backward)


def _out_like(x, cu_list):
    """Output buffer shaped like x; tokens after the last sequence (cu_seqlens[-1] < T) belong
    to no sequence and stay zero, as in the reference's varlen outputs (``naive.py:52``)."""
    if cu_list is not None and cu_list[-1] < x.shape[1]:
        return torch.zeros_like(x)
    return torch.empty_like(x)


def _default_scale(scale, K):
    return K ** -0.5 if scale is None else float(scale)


def _shape_check(q, k=None, v=None, g=None, h0=None, N=None, name="initial_state"):
    """Shape consistency the kernels rely on (they index every tensor with q's B, T, H)."""
    B, T, H, K = q.shape
    if k is not None:
        require(tuple(k.shape) == (B, T, H, K),
                f"Expected k shape {(B, T, H, K)}, got {tuple(k.shape)}")
    if g is not None:
        require(tuple(g.shape) == (B, T, H, K),
                f"Expected g shape {(B, T, H, K)}, got {tuple(g.shape)}")
    if v is not None:
        require(v.dim() == 4 and tuple(v.shape[:3]) == (B, T, H),
                f"Expected v shape {(B, T, H)} + (V,), got {tuple(v.shape)}")
    if h0 is not None:
        V = v.shape[-1] if v is not None else h0.shape[-1]
        require(tuple(h0.shape) == (N, H, K, V),
                f"Expected {name} shape {(N, H, K, V)}, got {tuple(h0.shape)}")


def _gates(g, g_gamma, q):
    """The per-element gate tensor: g, or g_gamma broadcast (kept in float32, as the
    reference computes its ramp ``g_gamma * pos`` in float32, ``chunk.py:1134-1143``), or
    zeros."""
    if g is not None:
        return g
    if g_gamma is not None:
        return g_gamma.to(torch.float32).expand(q.shape)
    return torch.zeros_like(q)


def _per_head(g_gamma, H):
    """g_gamma as a float32 ``[H]`` vector when it is constant over batch, time and key
    columns (the scalar-gate kernels' per-head form), else None."""
    if g_gamma.dim() > 4:
        return None
    shape = [1] * (4 - g_gamma.dim()) + list(g_gamma.shape)
    if shape[0] != 1 or shape[1] != 1 or shape[3] != 1 or shape[2] not in (1, H):
        return None
    return g_gamma.reshape(shape[2]).to(torch.float32).expand(H)


# ---------------------------------------------------------------------------
# autograd core
# ---------------------------------------------------------------------------


class _ChunkGLAFunction(torch.autograd.Function):
    """o, ht = chunk_gla(q, k, v, g, h0); backward = reference chunk_gla_bwd semantics."""

    @staticmethod
    def forward(ctx, q, k, v, g, h0, scale, output_final_state, cu_list, chunk):
        B, T, H, K = q.shape
        V = v.shape[-1]
        dev = check_device(q, k, v, g, h0)
        seq = SeqLayout(B, T, chunk, cu_list, dev)
        dt = dtype_code(q.dtype)
        o = _out_like(v, cu_list)
        ht = (torch.empty(seq.N, H, K, V, dtype=torch.float32, device=dev)
              if output_final_state else None)
        # the states are the backward's residual: not kept when no gradient is wanted (the
        # full-head path then stores none; the other paths read them back themselves)
        keep = any(ctx.needs_input_grad[:5])
        h_ws = (torch.empty(seq.NC, H, K, V, dtype=q.dtype, device=dev)
                if keep or not _full_head(K, V, chunk, q.dtype, False, q, k, v, g, h0) else None)
        ws, nws = _lib.seg_workspace(B, T, H, K, V, chunk, cu_list, q.dtype, dev)
        call("tops_gla_chunk_fwd", ptr(q), ptr(k), ptr(v), ptr(g), ptr(h0), ptr(o), ptr(ht),
             ptr(h_ws), ptr(ws), nws, scale, B, T, H, K, V, chunk, *seq.args(), dt,
             stream_of(dev))
        ctx.save_for_backward(q, k, v, g, h0, h_ws)
        ctx.meta = (scale, cu_list, chunk)
        if ht is None:
            return o, None
        return o, ht

    @staticmethod
    def backward(ctx, do, dht):
        q, k, v, g, h0, h_ws = ctx.saved_tensors
        scale, cu_list, chunk = ctx.meta
        B, T, H, K = q.shape
        V = v.shape[-1]
        dev = q.device
        seq = SeqLayout(B, T, chunk, cu_list, dev)
        do = torch.zeros_like(v) if do is None else _c(do, v.dtype)
        dht = None if dht is None else _c(dht, torch.float32)
        dq, dk, dv, dg = (_out_like(x, cu_list) for x in (q, k, v, g))
        need_dh0 = h0 is not None and ctx.needs_input_grad[4]
        dh0 = torch.empty(seq.N, H, K, V, dtype=torch.float32, device=dev) if need_dh0 else None
        dh_ws = (None if _full_head(K, V, chunk, q.dtype, True, q, k, v, g, h0, h_ws, do, dht,
                                    dq, dk, dv, dg, dh0)
                 else torch.empty(seq.NC, H, K, V, dtype=q.dtype, device=dev))
        ws, nws = _lib.seg_workspace(B, T, H, K, V, chunk, cu_list, q.dtype, dev,
                                     backward=True)
        call("tops_gla_chunk_bwd", ptr(q), ptr(k), ptr(v), ptr(g), ptr(h0), ptr(h_ws), ptr(do),
             ptr(dht), ptr(dq), ptr(dk), ptr(dv), ptr(dg), ptr(dh0), None, ptr(dh_ws), ptr(ws),
             nws, scale, B, T, H, K, V, chunk, *seq.args(), dtype_code(q.dtype),
             stream_of(dev))
        return dq, dk, dv, dg, dh0, None, None, None, None


class _ScalarGateGLAFunction(torch.autograd.Function):
    """GLA with scalar gates on the full-head kernels (``tops_gla_simple_chunk_fwd / _bwd``):
    the log-decay of token t and head h is ``gs[t, h]`` (gs ``[B * T, H]``) or ``gs[h]`` (gs
    ``[H]``) for every key column. Differentiable w.r.t. q, k, v, gs and h0."""

    @staticmethod
    def forward(ctx, q, k, v, gs, h0, scale, output_final_state, cu_list):
        B, T, H, K = q.shape
        V = v.shape[-1]
        C = 64
        dev = check_device(q, k, v, gs, h0)
        seq = SeqLayout(B, T, C, cu_list, dev)
        ts = 0 if gs.dim() == 1 else H
        o = _out_like(v, cu_list)
        ht = (torch.empty(seq.N, H, K, V, dtype=torch.float32, device=dev)
              if output_final_state else None)
        keep = any(ctx.needs_input_grad[:5])
        h_ws = torch.empty(seq.NC, H, K, V, dtype=q.dtype, device=dev) if keep else None
        ws, nws = _lib.seg_workspace(B, T, H, K, V, C, cu_list, q.dtype, dev)
        call("tops_gla_simple_chunk_fwd", ptr(q), ptr(k), ptr(v), ptr(gs), ts, ptr(h0), ptr(o),
             ptr(ht), ptr(h_ws), ptr(ws), nws, scale, B, T, H, K, V, C, *seq.args(),
             dtype_code(q.dtype), stream_of(dev))
        ctx.save_for_backward(q, k, v, gs, h0, h_ws)
        ctx.meta = (scale, cu_list)
        return o, ht

    @staticmethod
    def backward(ctx, do, dht):
        q, k, v, gs, h0, h_ws = ctx.saved_tensors
        scale, cu_list = ctx.meta
        B, T, H, K = q.shape
        V = v.shape[-1]
        C = 64
        dev = q.device
        seq = SeqLayout(B, T, C, cu_list, dev)
        ts = 0 if gs.dim() == 1 else H
        do = torch.zeros_like(v) if do is None else _c(do, v.dtype)
        dht = None if dht is None else _c(dht, torch.float32)
        dq, dk, dv = (_out_like(x, cu_list) for x in (q, k, v))
        want_dg = ctx.needs_input_grad[3]
        dg = _out_like(q, cu_list) if want_dg else None
        need_dh0 = h0 is not None and ctx.needs_input_grad[4]
        dh0 = torch.empty(seq.N, H, K, V, dtype=torch.float32, device=dev) if need_dh0 else None
        ws, nws = _lib.seg_workspace(B, T, H, K, V, C, cu_list, q.dtype, dev)
        call("tops_gla_simple_chunk_bwd", ptr(q), ptr(k), ptr(v), ptr(gs), ts, ptr(h0),
             ptr(h_ws), ptr(do), ptr(dht), ptr(dq), ptr(dk), ptr(dv), ptr(dg), ptr(dh0), None,
             ptr(ws), nws, scale, B, T, H, K, V, C, *seq.args(), dtype_code(q.dtype),
             stream_of(dev))
        dgs = None
        if want_dg:   # a scalar gate's gradient sums its key columns' gradients
            d = dg.to(torch.float32).sum(-1)
            dgs = d.reshape(B * T, H) if gs.dim() == 2 else d.sum((0, 1))
        return dq, dk, dv, dgs, dh0, None, None, None


def scalar_gate_gla(q, k, v, gs, initial_state, scale, output_final_state, cu_list):
    """GLA whose log-decay is the same for every key column: ``gs`` float32 ``[B, T, H]``
    (per-token raw gates) or ``[H]`` (a per-head constant). bf16 inputs of full-head shapes
    run the scalar-gate chunk kernels; anything else the recurrent kernel on the gate
    broadcast over K, in float32 (exact for any decay strength, as the scalar-gate kernels
    are). Returns (o in the compute dtype, ht or None)."""
    from .fused_recurrent import fused_recurrent_gla

    B, T, H, K = q.shape
    V = v.shape[-1]
    cdt = _compute_dtype(q, k, v)
    if cu_list is not None:
        cu_kept, keep = _lib.drop_empty(cu_list)
        if keep is not None:   # empty sequences: run the others, keep their initial states
            o, ht = (torch.zeros(v.shape, dtype=cdt, device=v.device), None) if not keep else \
                scalar_gate_gla(q, k, v, gs, _lib.gather_states(initial_state, keep), scale,
                                output_final_state, cu_kept)
            if output_final_state:
                ht = _lib.scatter_states(ht, initial_state, keep, (len(cu_list) - 1, H, K, V),
                                         v.device)
            return o, ht
    q, k, v = _c(q, cdt), _c(k, cdt), _c(v, cdt)
    h0 = _c(initial_state, torch.float32)
    grad = torch.is_grad_enabled() and any(
        t is not None and t.requires_grad for t in (q, k, v, gs, h0))
    if _full_head(K, V, 64, cdt, grad, q, k, v, h0):
        gflat = gs.reshape(B * T, H) if gs.dim() == 3 else gs
        return _ScalarGateGLAFunction.apply(q, k, v, _c(gflat, torch.float32), h0, float(scale),
                                            bool(output_final_state), cu_list)
    f32 = torch.float32
    g = (gs[..., None] if gs.dim() == 3 else gs[None, None, :, None]).to(f32)
    g = g.expand(B, T, H, K).contiguous()
    o, ht = fused_recurrent_gla(q.to(f32), k.to(f32), v.to(f32), gk=g, scale=float(scale),
                                initial_state=h0, output_final_state=bool(output_final_state),
                                cu_seqlens=cu_list)
    return o, ht


def chunk_gla(q, k, v, g=None, g_gamma=None, scale=None, initial_state=None,
              output_final_state=False, cu_seqlens=None, chunk_size=16):
    """Chunked GLA forward (differentiable). Reference: ``tops/ops/gla/chunk.py:1187-1251``.

    Args mirror the reference: q, k ``[B, T, H, K]``, v ``[B, T, H, V]``, g ``[B, T, H, K]``
    log-gates or ``g_gamma`` broadcastable to it (used only when g is None; neither means no
    decay), ``scale`` (default ``K ** -0.5``), ``initial_state [N, H, K, V]``,
    ``output_final_state``, ``cu_seqlens [N + 1]`` (B must be 1) and ``chunk_size``.

    Returns ``(o, final_state)``: o ``[B, T, H, V]`` in q's dtype, final_state float32
    ``[N, H, K, V]`` or None.
    """
    dtype = q.dtype
    B, T, H, K = q.shape
    V = v.shape[-1]
    require(k.shape == (B, T, H, K), f"Expected k shape {(B, T, H, K)}, got {tuple(k.shape)}")
    require(v.shape[:3] == (B, T, H), f"Expected v shape {(B, T, H, V)}, got {tuple(v.shape)}")
    cu_list = None if cu_seqlens is None else _lib.to_list(cu_seqlens)
    N = B if cu_list is None else len(cu_list) - 1
    if initial_state is not None:
        require(initial_state.shape == (N, H, K, V),
                f"Expected initial_state shape {(N, H, K, V)}, got {tuple(initial_state.shape)}")
    if cu_list is not None:
        cu_kept, keep = _lib.drop_empty(cu_list)
        if keep is not None:   # empty sequences: run the others, keep their initial states
            o, ht = (None, None) if not keep else chunk_gla(
                q, k, v, g, g_gamma, scale, _lib.gather_states(initial_state, keep),
                output_final_state, cu_kept, chunk_size)
            if o is None:
                o = torch.zeros(v.shape, dtype=dtype, device=v.device)
            if not output_final_state:
                return o, None
            return o, _lib.scatter_states(ht, initial_state, keep, (N, H, K, V), v.device)
    gh = _per_head(g_gamma, H) if g is None and g_gamma is not None else None
    if gh is not None:   # a per-head constant decay: the scalar-gate kernels, gate in float32
        o, ht = scalar_gate_gla(q, k, v, gh, initial_state, _default_scale(scale, K),
                                output_final_state, cu_list)
        return o.to(dtype), (ht if output_final_state else None)
    g = _gates(g, g_gamma, q)
    require(g.shape == (B, T, H, K), f"Expected g shape {(B, T, H, K)}, got {tuple(g.shape)}")
    cdt = _compute_dtype(q, k, v, g)
    o, ht = _ChunkGLAFunction.apply(_c(q, cdt), _c(k, cdt), _c(v, cdt), _c(g, cdt),
                                    _c(initial_state, torch.float32),
                                    _default_scale(scale, K), bool(output_final_state),
                                    cu_list, _kernel_chunk(chunk_size))
    return o.to(dtype), (ht if output_final_state else None)


# ---------------------------------------------------------------------------
# sub-functions (reference exports)
# ---------------------------------------------------------------------------


def chunk_local_cumsum_vector(g, chunk_size, reverse=False, scale=None, cu_seqlens=None,
                              head_first=False, output_dtype=torch.float32, chunk_indices=None):
    """Chunk-local cumsum of gates. Reference: ``tops/ops/gla/chunk.py:110-198``.

    ``chunk_indices`` is accepted for API parity; the kernel derives the same map from
    ``cu_seqlens``.
    """
    del chunk_indices
    require(chunk_size == 2 ** (chunk_size.bit_length() - 1), "chunk_size must be power of 2")
    if head_first:
        B, H, T, S = g.shape
    else:
        B, T, H, S = g.shape
    dev = check_device(g)
    gin = _c(g, g.dtype if g.dtype in (torch.float32, torch.bfloat16) else torch.float32)
    odt = output_dtype or g.dtype
    if odt not in (torch.float32, torch.bfloat16):
        odt = torch.float32
    out = torch.empty(g.shape, dtype=odt, device=dev)
    seq = SeqLayout(B, T, chunk_size, cu_seqlens, dev)
    call("tops_gla_chunk_local_cumsum", ptr(gin), ptr(out), B, T, H, S, chunk_size,
         int(reverse), int(scale is not None), float(scale or 1.0), int(head_first),
         *seq.args(), dtype_code(gin.dtype), dtype_code(odt), stream_of(dev))
    if output_dtype is not None and out.dtype != output_dtype:
        out = out.to(output_dtype)
    return out


chunk_local_cumsum = chunk_local_cumsum_vector


def chunk_local_cumsum_ref(g, chunk_size, scale=None, reverse=False, cu_seqlens_cpu=None):
    """``chunk_local_cumsum_ref`` (``tops/ops/gla/chunk.py:20-52``): T and cu_seqlens must be
    chunk-aligned, no reverse; computed by the same kernel."""
    require(reverse is False, "Reverse mode not supported in chunk_local_cumsum")
    require(g.shape[1] % chunk_size == 0,
            "T must be a multiple of chunk_size for chunk_local_cumsum")
    if cu_seqlens_cpu is not None:
        require(all(c % chunk_size == 0 for c in _lib.to_list(cu_seqlens_cpu)),
                "cu_seqlens must be multiples of chunk_size for chunk_local_cumsum")
    return chunk_local_cumsum_vector(g, chunk_size, scale=scale, cu_seqlens=cu_seqlens_cpu)


def chunk_fwd_h(k, v, gk=None, h0=None, output_final_state=False, cu_seqlens_cpu=None,
                chunk_size=64):
    """State at the start of every chunk. Reference (exported ``chunk_fwd_h``):
    ``chunk_fwd_h_ref``, ``tops/ops/gla/chunk.py:206-292``.

    ``gk`` is the chunk-local cumsum of the gates. Returns ``h [B, NT, H, K, V]`` in k's
    dtype and ``ht [N, H, K, V]`` float32 (zeros unless ``output_final_state``).
    """
    B, T, H, K = k.shape
    V = v.shape[-1]
    C = chunk_size
    require(T % C == 0, "T must be a multiple of chunk_size for chunk_fwd_h")
    if cu_seqlens_cpu is not None:
        require(all(c % C == 0 for c in _lib.to_list(cu_seqlens_cpu)),
                "cu_seqlens must be multiples of chunk_size for chunk_fwd_h")
    if C not in _KERNEL_CHUNKS:
        raise NotImplementedError(f"chunk_fwd_h: chunk_size {C} (kernels take 4, 8, 16, 32, 64)")
    N = B if cu_seqlens_cpu is None else len(_lib.to_list(cu_seqlens_cpu)) - 1
    _shape_check(k, v=v, g=gk, h0=h0, N=N)
    dev = check_device(k, v, gk, h0)
    cdt = _compute_dtype(k, v) if gk is None or gk.dtype == k.dtype else torch.float32
    kk, vv = _c(k, cdt), _c(v, cdt)
    gg = torch.zeros_like(kk) if gk is None else _c(gk, cdt)
    seq = SeqLayout(B, T, C, cu_seqlens_cpu, dev)
    h = torch.empty(B, seq.NC // B, H, K, V, dtype=cdt, device=dev)
    ht = torch.empty(seq.N, H, K, V, dtype=torch.float32, device=dev)
    call("tops_gla_chunk_fwd_h", ptr(kk), ptr(vv), ptr(gg), 1, ptr(_c(h0, torch.float32)),
         ptr(h), ptr(ht), None, 0, B, T, H, K, V, C, *seq.args(), dtype_code(cdt),
         stream_of(dev))
    if not output_final_state:
        ht.zero_()
    return h.to(k.dtype), ht


chunk_fwd_h_ref = chunk_fwd_h


def chunk_gla_fwd_intra_gk(q, k, g, scale, chunk_size=64):
    """Unmasked intra-chunk matrix ``A [B, T, H, C]`` float32 from the gate cumsum ``g``.
    Reference: ``tops/ops/gla/chunk.py:386-433`` (body ``:350-383``, jnp ref ``:300-342``).
    """
    B, T, H, K = q.shape
    C = chunk_size
    require(T % C == 0)
    if C not in _KERNEL_CHUNKS:
        raise NotImplementedError(f"chunk_gla_fwd_intra_gk: chunk_size {C}")
    _shape_check(q, k=k, g=g)
    dev = check_device(q, k, g)
    cdt = _compute_dtype(q, k) if g.dtype == q.dtype else torch.float32
    seq = SeqLayout(B, T, C, None, dev)
    A = torch.empty(B, T, H, C, dtype=torch.float32, device=dev)
    call("tops_gla_chunk_fwd_o", ptr(_c(q, cdt)), ptr(_c(k, cdt)), None, ptr(_c(g, cdt)), 1,
         None, None, ptr(A), None, float(scale), B, T, H, K, 1, C, *seq.args(),
         dtype_code(cdt), stream_of(dev))
    return A


def chunk_gla_fwd_o_gk(q, v, g, A, h, scale, cu_seqlens=None, chunk_indices=None,
                       chunk_size=64, use_exp2=False):
    """``o = scale (q exp(g)) h + tril(A) v`` per chunk, with ``g`` the gate cumsum.
    Reference: ``tops/ops/gla/chunk.py:1387-1416`` (launcher ``:1315-1384``, body
    ``:1259-1312``, jnp ref ``:441-496``). ``use_exp2`` reads g in base 2."""
    del chunk_indices, cu_seqlens  # chunk-aligned layout: the per-chunk view is the same
    B, T, H, K = q.shape
    V = v.shape[-1]
    C = chunk_size
    require(T % C == 0)
    if C not in _KERNEL_CHUNKS:
        raise NotImplementedError(f"chunk_gla_fwd_o_gk: chunk_size {C}")
    _shape_check(q, v=v, g=g)
    require(tuple(A.shape) == (B, T, H, C),
            f"Expected A shape {(B, T, H, C)}, got {tuple(A.shape)}")
    require(tuple(h.shape) == (B, T // C, H, K, V),
            f"Expected h shape {(B, T // C, H, K, V)}, got {tuple(h.shape)}")
    dev = check_device(q, v, g, A, h)
    cdt = _compute_dtype(q, v) if g.dtype == q.dtype else torch.float32
    gg = g * math.log(2.0) if use_exp2 else g
    seq = SeqLayout(B, T, C, None, dev)
    o = torch.empty(B, T, H, V, dtype=cdt, device=dev)
    call("tops_gla_chunk_fwd_o", ptr(_c(q, cdt)), None, ptr(_c(v, cdt)), ptr(_c(gg, cdt)), 1,
         ptr(_c(h, cdt)), ptr(_c(A, torch.float32)), None, ptr(o), float(scale), B, T, H, K,
         V, C, *seq.args(), dtype_code(cdt), stream_of(dev))
    return o.to(v.dtype)


def _pad_like_reference(tensors, B, T, cu_list, C):
    """Zero-pad T (or each varlen segment) to a multiple of C, as ``chunk.py:751-793``.

    Returns ``(padded, padded_cu or None, unpad)``. Host-side glue for the sub-function API
    (the kernels themselves take partial chunks natively).
    """
    if cu_list is None:
        Tp = -(-T // C) * C
        if Tp == T:
            return tensors, None, (lambda x: x)
        return [pad_to_multiple(x, C, 1, 0) for x in tensors], None, (lambda x: x[:, :T])
    lens = [b - a for a, b in zip(cu_list, cu_list[1:])]
    plens = [-(-L // C) * C for L in lens]
    new_cu = [0]
    for pl in plens:
        new_cu.append(new_cu[-1] + pl)
    if lens == plens:
        return tensors, new_cu, (lambda x: x)
    out = []
    for x in tensors:
        parts = []
        for i, L in enumerate(lens):
            seg = x[:, cu_list[i]:cu_list[i + 1]]
            parts.append(pad_to_multiple(seg, C, 1, 0) if L % C else seg)
        out.append(torch.cat(parts, 1))

    def unpad(x):
        return torch.cat([x[:, new_cu[i]:new_cu[i] + L] for i, L in enumerate(lens)], 1)

    return out, new_cu, unpad


def chunk_gla_fwd(q, k, v, g, g_gamma, g_cumsum, scale, initial_state, output_final_state,
                  cu_seqlens=None, chunk_size=64):
    """Forward orchestrator returning ``(g_cumsum, A, h, ht, o)``.
    Reference: ``tops/ops/gla/chunk.py:1083-1179``.

    As in the reference, g_cumsum, A and h come back in the padded chunk layout (T, or each
    varlen segment, padded to a multiple of the chunk size) and o unpadded; ht is None
    unless requested. A given ``g_cumsum`` is used as the gates' cumsum.
    """
    B, T, H, K = q.shape
    V = v.shape[-1]
    C = chunk_size
    if C not in _KERNEL_CHUNKS:
        raise NotImplementedError(f"chunk_gla_fwd: chunk_size {C} (kernels take 4, 8, 16, 32, 64)")
    g = _gates(g, g_gamma, q)
    cu_list = None if cu_seqlens is None else _lib.to_list(cu_seqlens)
    N = B if cu_list is None else len(cu_list) - 1
    _shape_check(q, k=k, v=v, g=g, h0=initial_state, N=N)
    dev = check_device(q, k, v, g, initial_state)
    cdt = _compute_dtype(q, k, v, g) if g_cumsum is None else torch.float32
    (qp, kp, vp, gp), new_cu, unpad = _pad_like_reference(
        [_c(q, cdt), _c(k, cdt), _c(v, cdt), _c(g, cdt)], B, T, cu_list, C)
    Tp = qp.shape[1]
    seq = SeqLayout(B, Tp, C, new_cu, dev)
    if g_cumsum is None:
        g_cumsum = chunk_local_cumsum_vector(gp, C, cu_seqlens=new_cu)
        g_in, g_is_cumsum = gp, 0
    else:
        require(tuple(g_cumsum.shape) == tuple(qp.shape),
                f"g_cumsum must be in the padded layout {tuple(qp.shape)}, got "
                f"{tuple(g_cumsum.shape)}")
        g_in, g_is_cumsum = _c(g_cumsum, cdt), 1
    dt = dtype_code(cdt)
    st = stream_of(dev)
    h = torch.empty(B, seq.NC // B, H, K, V, dtype=cdt, device=dev)
    ht = torch.empty(seq.N, H, K, V, dtype=torch.float32, device=dev) if output_final_state \
        else None
    ws, nws = (None, 0) if g_is_cumsum else _lib.seg_workspace(B, Tp, H, K, V, C, new_cu,
                                                                cdt, dev)
    call("tops_gla_chunk_fwd_h", ptr(kp), ptr(vp), ptr(g_in), g_is_cumsum,
         ptr(_c(initial_state, torch.float32)), ptr(h), ptr(ht), ptr(ws), nws, B, Tp, H, K, V,
         C, *seq.args(), dt, st)
    A = torch.empty(B, Tp, H, C, dtype=torch.float32, device=dev)
    o = torch.empty(B, Tp, H, V, dtype=cdt, device=dev)
    call("tops_gla_chunk_fwd_o", ptr(qp), ptr(kp), ptr(vp), ptr(g_in), g_is_cumsum, ptr(h),
         None, ptr(A), ptr(o), float(scale), B, Tp, H, K, V, C, *seq.args(), dt, st)
    return g_cumsum, A, h.to(k.dtype), ht, unpad(o).to(q.dtype)


def chunk_gla_bwd(q, k, v, g, g_gamma, g_cumsum, scale, initial_state, h, A, do, dht,
                  cu_seqlens=None, chunk_size=64):
    """Backward orchestrator returning ``(dq, dk, dv, dg, dh0)``.
    Reference: ``tops/ops/gla/chunk.py:815-977``.

    ``h`` (forward states, padded chunk layout) is reused when given; ``g_cumsum`` and ``A``
    are recomputed in-kernel from g, q, k (the same values the reference would pass).
    ``dh0`` is returned when ``initial_state`` or ``dht`` is given, else None; with only
    ``g_gamma`` given, dg is sum-reduced to its shape (``chunk.py:967-975``).
    """
    del g_cumsum, A
    B, T, H, K = q.shape
    V = v.shape[-1]
    C = _kernel_chunk(chunk_size)
    if C != chunk_size:
        h = None  # states of another chunk size cannot be reused
    g_orig = g
    g = _gates(g, g_gamma, q)
    cu_list = None if cu_seqlens is None else _lib.to_list(cu_seqlens)
    N = B if cu_list is None else len(cu_list) - 1
    _shape_check(q, k=k, v=v, g=g, h0=initial_state, N=N)
    _shape_check(q, v=do, h0=dht, N=N, name="dht")
    dev = check_device(q, k, v, g, do, initial_state, dht, h)
    cdt = _compute_dtype(q, k, v, g, do)
    qq, kk, vv, gg, dd = (_c(x, cdt) for x in (q, k, v, g, do))
    seq = SeqLayout(B, T, C, cu_list, dev)
    if h is not None:
        require(h.numel() == seq.NC * H * K * V, "h does not match the chunk layout")
        h = _c(h, cdt)
    dq, dk, dv, dg = (torch.empty_like(x) for x in (qq, kk, vv, gg))
    want_dh0 = initial_state is not None or dht is not None
    dh0 = torch.empty(seq.N, H, K, V, dtype=torch.float32, device=dev) if want_dh0 else None
    h_ws = None if h is not None else torch.empty(seq.NC, H, K, V, dtype=cdt, device=dev)
    dh_ws = (None if _full_head(K, V, C, cdt, True, qq, kk, vv, gg, dd, h, dht, initial_state)
             else torch.empty(seq.NC, H, K, V, dtype=cdt, device=dev))
    ws, nws = _lib.seg_workspace(B, T, H, K, V, C, cu_list, cdt, dev, backward=True)
    call("tops_gla_chunk_bwd", ptr(qq), ptr(kk), ptr(vv), ptr(gg),
         ptr(_c(initial_state, torch.float32)), ptr(h), ptr(dd), ptr(_c(dht, torch.float32)),
         ptr(dq), ptr(dk), ptr(dv), ptr(dg), ptr(dh0), ptr(h_ws), ptr(dh_ws), ptr(ws), nws,
         float(scale), B, T, H, K, V, C, *seq.args(), dtype_code(cdt), stream_of(dev))
    dq, dk, dv, dg = dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), dg.to(g.dtype)
    if g_orig is None and g_gamma is not None:
        gg_shape = tuple(g_gamma.shape)
        extra = dg.dim() - len(gg_shape)
        if extra > 0:
            dg = dg.sum(dim=tuple(range(extra)))
        for ax, n in enumerate(gg_shape):
            if n == 1 and dg.shape[ax] != 1:
                dg = dg.sum(dim=ax, keepdim=True)
        dg = dg.reshape(gg_shape)
    return dq, dk, dv, dg, dh0


chunk_gla_bwd_with_pl = chunk_gla_bwd


# ---------------------------------------------------------------------------
# the backward's per-chunk parts over given intermediates (reference jnp exports)
# ---------------------------------------------------------------------------


def _parts_prep(C, T, *xs):
    """float32 contiguous copies; result dtype = the inputs' promoted dtype (jnp's rule)."""
    require(T % C == 0, f"T ({T}) must be a multiple of chunk_size ({C})")
    dev = check_device(*xs)
    rdt = xs[0].dtype
    for x in xs[1:]:
        rdt = torch.promote_types(rdt, x.dtype)
    return dev, rdt, [x.to(torch.float32).contiguous() for x in xs]


def chunk_gla_bwd_dA_ref(v, do, scale, cu_seqlens_cpu=None, chunk_size=64):
    """``dA = scale tril(do v^T)`` per chunk, ``[B, T, H, C]``. Reference:
    ``tops/ops/gla/chunk.py:504-539`` (which, like this, groups tokens as B * T / C chunks
    and does not read ``cu_seqlens_cpu``)."""
    del cu_seqlens_cpu
    B, T, H, V = v.shape
    C = chunk_size
    dev, rdt, (vf, dof) = _parts_prep(C, T, v, do)
    dA = torch.empty(B, T, H, C, dtype=torch.float32, device=dev)
    call("tops_gla_bwd_part_dA", ptr(vf), ptr(dof), ptr(dA), float(scale), B, T, H, V, C,
         stream_of(dev))
    return dA.to(rdt)


def chunk_gla_bwd_dv_ref(k, g_cumsum, A, do, dh, cu_seqlens_cpu=None, chunk_size=64):
    """``dv = tril(A)^T do + (k e^{gn - g~}) dh``. Reference: ``tops/ops/gla/chunk.py:547-595``.
    ``dh`` is ``[B, NT, H, K, V]`` (or ``[B * NT, H, K, V]``)."""
    del cu_seqlens_cpu
    B, T, H, K = k.shape
    V = do.shape[-1]
    C = chunk_size
    dev, rdt, (kf, gf, Af, dof, dhf) = _parts_prep(C, T, k, g_cumsum, A, do, dh)
    dv = torch.empty(B, T, H, V, dtype=torch.float32, device=dev)
    call("tops_gla_bwd_part_dv", ptr(kf), ptr(gf), ptr(Af), ptr(dof), ptr(dhf), ptr(dv), B, T,
         H, K, V, C, stream_of(dev))
    return dv.to(rdt)


def chunk_gla_bwd_dqk_intra_ref(q, k, g_cumsum, dA, cu_seqlens_cpu=None, chunk_size=64):
    """Intra-chunk ``dq = e^{g~} (dA (k e^{-g~}))``, ``dk = e^{-g~} (dA^T (q e^{g~}))``.
    Reference: ``tops/ops/gla/chunk.py:603-648``."""
    del cu_seqlens_cpu
    B, T, H, K = q.shape
    C = chunk_size
    dev, rdt, (qf, kf, gf, dAf) = _parts_prep(C, T, q, k, g_cumsum, dA)
    dq = torch.empty(B, T, H, K, dtype=torch.float32, device=dev)
    dk = torch.empty_like(dq)
    call("tops_gla_bwd_part_dqk_intra", ptr(qf), ptr(kf), ptr(gf), ptr(dAf), ptr(dq), ptr(dk),
         B, T, H, K, C, stream_of(dev))
    return dq.to(rdt), dk.to(rdt)


def chunk_gla_bwd_dqkg_ref(q, k, v, h, g_cumsum, do, dh, dq, dk, scale, cu_seqlens_cpu=None,
                           chunk_size=64):
    """Inter-chunk dq, dk added to the given intra ones, and the gate gradient
    ``dg = revcumsum_chunk(q dq - k dk) + e^{gn} sum_v h dh + sum_c dk_inter k``.
    Reference: ``tops/ops/gla/chunk.py:656-743``. Returns ``(dq, dk, dg)``."""
    del cu_seqlens_cpu
    B, T, H, K = q.shape
    V = v.shape[-1]
    C = chunk_size
    dev, rdt, xs = _parts_prep(C, T, q, k, v, h, g_cumsum, do, dh, dq, dk)
    qf, kf, vf, hf, gf, dof, dhf, dqf, dkf = xs
    dq_out = torch.empty(B, T, H, K, dtype=torch.float32, device=dev)
    dk_out = torch.empty_like(dq_out)
    dg = torch.empty_like(dq_out)
    call("tops_gla_bwd_part_dqkg", ptr(qf), ptr(kf), ptr(vf), ptr(hf), ptr(gf), ptr(dof),
         ptr(dhf), ptr(dqf), ptr(dkf), ptr(dq_out), ptr(dk_out), ptr(dg), float(scale), B, T, H,
         K, V, C, stream_of(dev))
    return dq_out.to(rdt), dk_out.to(rdt), dg.to(rdt)
