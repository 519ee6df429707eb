"""Chunked simple GLA on the MI355X kernels, mirroring ``tops/ops/simple_gla/chunk.py``.

Simple GLA is GLA whose log-decay is one scalar per token and head: a per-head constant
``g_gamma [H]``, a per-token ``g [B, T, H]`` (given, as in the reference, as its chunk-local
cumsum), or their sum. bf16 inputs of full-head shapes (K <= 256 forward, K, V <= 128
backward) run the scalar-gate kernels (``tops_gla_simple_chunk_fwd / _bwd``: the gate is read
as one float per token and head, never as a ``[B, T, H, K]`` tensor); other shapes and
float32 run the per-element GLA kernels on the gate broadcast over K, in float32.
"""

from __future__ import annotations

import torch

from ... import _lib
from ..._lib import require
from ..gla.chunk import chunk_gla_fwd_intra_gk, chunk_gla_fwd_o_gk, scalar_gate_gla

__all__ = [
    "chunk_simple_gla_fwd",
    "chunk_simple_gla_bwd",
    "chunk_simple_gla_fwd_ref",
    "chunk_simple_gla_fwd_intra_ref",
    "chunk_simple_gla_fwd_o_ref",
]


def _raw_from_cumsum(g, C):
    """Per-token raw gates from their chunk-local cumsum ``[B, T, H]`` (T % C == 0)."""
    gf = g.to(torch.float32)
    raw = gf.clone()
    raw[:, 1:] -= gf[:, :-1]
    raw[:, 0::C] = gf[:, 0::C]   # first row of every chunk
    return raw


def _scalar_gates(g, g_gamma, B, T, H, C, device):
    """float32 ``[B, T, H]`` raw per-token gates (g given), else the ``[H]`` constant."""
    gh = None if g_gamma is None else g_gamma.reshape(H).to(torch.float32)
    if g is not None:
        raw = _raw_from_cumsum(g, C)
        return raw + gh if gh is not None else raw
    if gh is not None:
        return gh
    return torch.zeros(H, dtype=torch.float32, device=device)


def _ramp(g_gamma, B, T, H, K, C, device):
    """The chunk-local cumsum of a per-head constant gate, ``g_h (row + 1)``, as a float32
    ``[B, T, H, K]`` tensor (``chunk.py:150-153``)."""
    pos = (torch.arange(T, device=device) % C + 1).to(torch.float32)
    gh = g_gamma.reshape(H).to(torch.float32)
    return (pos[:, None] * gh[None, :])[None, :, :, None].expand(B, T, H, K).contiguous()


def chunk_simple_gla_fwd(q, k, v, *, g=None, g_gamma=None, scale=None, h0=None, use_ht=False,
                         cu_seqlens=None, chunk_size=64):
    """Simple GLA forward. Reference: ``tops/ops/simple_gla/chunk.py:471-519``.

    q, k ``[B, T, H, K]``, v ``[B, T, H, V]``; ``g`` ``[B, T, H]`` the chunk-local cumsum
    of per-token scalar log-decays (chunks of ``chunk_size``), ``g_gamma`` ``[H]``;
    ``h0 [B, H, K, V]``; ``cu_seqlens [B + 1]`` splits the flattened ``[B * T]`` token axis
    into B sequences. Returns (o ``[B, T, H, V]`` in v's dtype, ht float32 or None).
    """
    B, T, H, K, V = *q.shape, v.shape[-1]
    require((B, T, H, K) == tuple(k.shape))
    require((B, T, H, V) == tuple(v.shape))
    require((g is None) or ((B, T, H) == tuple(g.shape)))
    require((g_gamma is None) or ((H,) == tuple(g_gamma.shape)))
    require((h0 is None) or ((B, H, K, V) == tuple(h0.shape)))
    require((cu_seqlens is None) or ((B + 1,) == tuple(cu_seqlens.shape)))
    require(T % chunk_size == 0)
    cu = None if cu_seqlens is None else _lib.to_list(cu_seqlens)
    require((cu is None) or all(c % chunk_size == 0 for c in cu))
    require((K % 128 == 0) and (V % 128 == 0))
    scale = K ** -0.5 if scale is None else float(scale)
    gs = _scalar_gates(g, g_gamma, B, T, H, chunk_size, q.device)
    if cu is not None:   # one row of B * T tokens
        q, k = (x.reshape(1, B * T, H, K) for x in (q, k))
        v = v.reshape(1, B * T, H, V)
        gs = gs.reshape(1, B * T, H) if gs.dim() == 3 else gs
    o, ht = scalar_gate_gla(q, k, v, gs, h0, scale, use_ht, cu)
    return o.reshape(B, T, H, V).to(v.dtype), (ht if use_ht else None)


def chunk_simple_gla_bwd(q, k, v, g_gamma, scale, initial_state, do, dht, chunk_size=64):
    """Simple GLA backward with a per-head constant decay. Reference:
    ``tops/ops/simple_gla/chunk.py:538-615``.

    Recomputes the forward states, then the state-gradient scan and the per-chunk gradients.
    Returns ``(dq, dk, dv, dh0)`` (dh0 float32 ``[B, H, K, V]`` when initial_state is given,
    else None).
    """
    B, T, H, K = q.shape
    V = v.shape[-1]
    for name, x, shp in (("q", q, (B, T, H, K)), ("k", k, (B, T, H, K)),
                         ("v", v, (B, T, H, V)), ("do", do, (B, T, H, V))):
        require(tuple(x.shape) == shp, f"{name}: expected shape {shp}, got {tuple(x.shape)}")
    require(K % 128 == 0 and V % 128 == 0)
    require(T % chunk_size == 0)
    with torch.enable_grad():
        qq, kk, vv = (x.detach().requires_grad_(True) for x in (q, k, v))
        h0 = None if initial_state is None else \
            initial_state.detach().to(torch.float32).requires_grad_(True)
        gs = g_gamma.detach().reshape(H).to(torch.float32)
        o, ht = scalar_gate_gla(qq, kk, vv, gs, h0, float(scale), dht is not None, None)
        outs, grads = [o], [do.to(o.dtype)]
        if dht is not None:
            outs.append(ht)
            grads.append(dht.to(torch.float32))
        wrt = [qq, kk, vv] + ([h0] if h0 is not None else [])
        res = torch.autograd.grad(outs, wrt, grads, allow_unused=True)
    dq, dk, dv = (r.to(x.dtype) for r, x in zip(res[:3], (q, k, v)))
    dh0 = res[3] if h0 is not None else None
    return dq, dk, dv, dh0


def chunk_simple_gla_fwd_ref(q, k, v, g_gamma, scale, initial_state=None,
                             output_final_state=False, chunk_size=64):
    """Simple GLA forward by sub-steps. Reference: ``tops/ops/simple_gla/chunk.py:126-170``.

    T is zero-padded to a multiple of ``chunk_size`` as in the reference, so the padded rows'
    decay reaches the final state. Returns ``(ht or None, o)``.
    """
    B, T, H, K = q.shape
    C = chunk_size
    gh = g_gamma.reshape(-1)
    require(gh.shape[0] == H)
    Tp = -(-T // C) * C
    if Tp != T:
        q, k, v = (torch.nn.functional.pad(x, (0, 0, 0, 0, 0, Tp - T)) for x in (q, k, v))
    o, ht = scalar_gate_gla(q, k, v, gh.to(torch.float32), initial_state, float(scale),
                            output_final_state, None)
    return (ht if output_final_state else None), o[:, :T].to(v.dtype)


def chunk_simple_gla_fwd_intra_ref(q, k, g_gamma, scale, chunk_size=64):
    """Unmasked intra-chunk matrix ``A [B, T, H, C]`` float32 with the Toeplitz decay
    ``scale (q_i . k_j) exp(g_h (i - j))``. Reference: ``tops/ops/simple_gla/chunk.py:27-70``.
    """
    B, T, H, K = q.shape
    C = chunk_size
    require(T % C == 0)
    g = _ramp(g_gamma, B, T, H, K, C, q.device)
    return chunk_gla_fwd_intra_gk(q.to(torch.float32), k.to(torch.float32), g, scale, C)


def chunk_simple_gla_fwd_o_ref(q, v, g_gamma, A, h, scale, chunk_size=64):
    """``o = scale (q exp(g_h (row + 1))) h_n + tril(A) v`` per chunk. Reference:
    ``tops/ops/simple_gla/chunk.py:73-123``. h ``[B, T / C, H, K, V]``."""
    B, T, H, K = q.shape
    C = chunk_size
    require(T % C == 0)
    g = _ramp(g_gamma, B, T, H, K, C, q.device)
    f32 = torch.float32
    return chunk_gla_fwd_o_gk(q.to(f32), v.to(f32), g, A.to(f32), h.to(f32), scale,
                              chunk_size=C)
