"""Fused recurrent GLA on the MI355X HIP kernel, mirroring
``tops/ops/gla/fused_recurrent.py``.

The state update is element-wise (no matrix product), so the kernel streams the sequence
once, keeps the K x V state in VGPRs and uses only fp32 VALU work plus LDS broadcasts.
"""

from __future__ import annotations

import torch

from ... import _lib
from ..._lib import SeqLayout, call, check_device, dtype_code, ptr, require, stream_of

__all__ = ["fused_recurrent_gla", "fused_recurrent_gla_fwd", "fused_recurrent_gla_bwd"]


def _out(B, T, H, D, dtype, dev, cu):
    """Output buffer; tokens after the last sequence stay zero (reference :186-194)."""
    if cu is not None and cu[-1] < T:
        return torch.zeros(B, T, H, D, dtype=dtype, device=dev)
    return torch.empty(B, T, H, D, dtype=dtype, device=dev)


def _compute_dtype(*xs):
    xs = [x for x in xs if x is not None]
    return torch.bfloat16 if {x.dtype for x in xs} == {torch.bfloat16} else torch.float32


def _run(q, k, v, gk, gv, scale, initial_state, output_final_state, reverse, cu_seqlens,
         out_dtype):
    B, T, H, K = q.shape
    V = v.shape[-1]
    dev = check_device(q, k, v, gk, gv, initial_state)
    cdt = _compute_dtype(q, k, v, gk, gv)
    c = lambda x: None if x is None else x.to(cdt).contiguous()  # noqa: E731
    odt = torch.float32 if out_dtype == torch.float32 or cdt == torch.float32 else cdt
    if cu_seqlens is not None:
        kept, keep = _lib.drop_empty(cu_seqlens)
        if keep is not None:   # empty sequences: run the others, keep their initial states
            o, ht = (torch.zeros(B, T, H, V, dtype=odt, device=dev), None) if not keep else \
                _run(q, k, v, gk, gv, scale, _lib.gather_states(initial_state, keep),
                     output_final_state, reverse, kept, out_dtype)
            if output_final_state:
                ht = _lib.scatter_states(ht, initial_state, keep,
                                         (len(cu_seqlens) - 1, H, K, V), dev)
            return o, ht
    seq = SeqLayout(B, T, 1, cu_seqlens, dev)
    o = _out(B, T, H, V, odt, dev, cu_seqlens)
    ht = torch.empty(seq.N, H, K, V, dtype=torch.float32, device=dev) if output_final_state \
        else None
    h0 = None if initial_state is None else initial_state.to(torch.float32).contiguous()
    call("tops_gla_fused_recurrent_fwd", ptr(c(q)), ptr(c(k)), ptr(c(v)), ptr(c(gk)),
         ptr(c(gv)), ptr(h0), ptr(o), ptr(ht), float(scale), int(bool(reverse)), B, T, H, K, V,
         ptr(seq.cu), seq.N, dtype_code(cdt), dtype_code(odt), stream_of(dev))
    return o, ht


def fused_recurrent_gla_fwd(q, k, v, gk=None, gv=None, scale=None, initial_state=None,
                            output_final_state=False, reverse=False, cu_seqlens=None):
    """Validation + dispatch. Reference: ``tops/ops/gla/fused_recurrent.py:379-430``.

    Returns ``(o, ht)``: o ``[B, T, H, V]`` float32 (as the reference, ``:262,369``), ht
    float32 ``[N, H, K, V]`` or None.
    """
    B, T, H, K = q.shape
    V = v.shape[-1]
    cu = None if cu_seqlens is None else _lib.to_list(cu_seqlens)
    N = len(cu) - 1 if cu is not None else B
    scale = scale if scale is not None else K ** -0.5
    require(tuple(k.shape) == (B, T, H, K), f"Expected k shape {(B, T, H, K)}, got {k.shape}")
    require(tuple(v.shape) == (B, T, H, V), f"Expected v shape {(B, T, H, V)}, got {v.shape}")
    require((gk is None) or (tuple(gk.shape) == (B, T, H, K)),
            f"Expected gk shape {(B, T, H, K)}, got {getattr(gk, 'shape', None)}")
    require((gv is None) or (tuple(gv.shape) == (B, T, H, V)),
            f"Expected gv shape {(B, T, H, V)}, got {getattr(gv, 'shape', None)}")
    require((initial_state is None) or (tuple(initial_state.shape) == (N, H, K, V)),
            f"Expected initial_state shape {(N, H, K, V)}, got "
            f"{getattr(initial_state, 'shape', None)}")
    require((cu_seqlens is None) or (B == 1),
            f"Batch size must be 1 when using cu_seqlens, got {B}")
    return _run(q, k, v, gk, gv, scale, initial_state, output_final_state, reverse, cu,
                torch.float32)


class _FusedRecurrentGLAFunction(torch.autograd.Function):
    """o, ht = fused_recurrent_gla(...); backward = ``fused_recurrent_gla_bwd``.

    The reference defines no autodiff rule for ``fused_recurrent_gla``; its backward entry
    point (``tops/ops/gla/fused_recurrent.py:879-956``) is what this rule calls.
    """

    @staticmethod
    def forward(ctx, q, k, v, gk, gv, h0, scale, output_final_state, reverse, cu):
        o, ht = _run(q, k, v, gk, gv, scale, h0, output_final_state, reverse, cu,
                     torch.float32)
        ctx.save_for_backward(q, k, v, gk, gv, h0, o if gv is not None else None)
        ctx.meta = (scale, reverse, cu)
        return o, ht

    @staticmethod
    def backward(ctx, do, dht):
        q, k, v, gk, gv, h0, o = ctx.saved_tensors
        scale, reverse, cu = ctx.meta
        if do is None:
            do = torch.zeros(*v.shape, dtype=torch.float32, device=v.device)
        dq, dk, dv, dgk, dgv, dh0 = _bwd(q, k, v, gk, gv, o, do, dht, scale, h0, reverse, cu)
        cast = lambda g, x: None if g is None or x is None else g.to(x.dtype)  # noqa: E731
        return (cast(dq, q), cast(dk, k), cast(dv, v), cast(dgk, gk), cast(dgv, gv),
                cast(dh0, h0), None, None, None, None)


def fused_recurrent_gla(q, k, v, gk=None, gv=None, scale=None, initial_state=None,
                        output_final_state=False, reverse=False, cu_seqlens=None):
    """Fused recurrent GLA, public API. Reference: ``tops/ops/gla/fused_recurrent.py:438-481``.

    Differentiable: gradients flow to q, k, v, gk, gv and initial_state through
    ``fused_recurrent_gla_bwd``.
    """
    if not torch.is_grad_enabled() or not any(
            x is not None and x.requires_grad for x in (q, k, v, gk, gv, initial_state)):
        return fused_recurrent_gla_fwd(q, k, v, gk=gk, gv=gv, scale=scale,
                                       initial_state=initial_state,
                                       output_final_state=output_final_state,
                                       reverse=reverse, cu_seqlens=cu_seqlens)
    B, T, H, K = q.shape
    V = v.shape[-1]
    cu = None if cu_seqlens is None else _lib.to_list(cu_seqlens)
    N = len(cu) - 1 if cu is not None else B
    require(tuple(k.shape) == (B, T, H, K), f"Expected k shape {(B, T, H, K)}, got {k.shape}")
    require(tuple(v.shape) == (B, T, H, V), f"Expected v shape {(B, T, H, V)}, got {v.shape}")
    require((gk is None) or (tuple(gk.shape) == (B, T, H, K)),
            f"Expected gk shape {(B, T, H, K)}, got {getattr(gk, 'shape', None)}")
    require((gv is None) or (tuple(gv.shape) == (B, T, H, V)),
            f"Expected gv shape {(B, T, H, V)}, got {getattr(gv, 'shape', None)}")
    require((initial_state is None) or (tuple(initial_state.shape) == (N, H, K, V)),
            f"Expected initial_state shape {(N, H, K, V)}, got "
            f"{getattr(initial_state, 'shape', None)}")
    require((cu_seqlens is None) or (B == 1),
            f"Batch size must be 1 when using cu_seqlens, got {B}")
    scale = scale if scale is not None else K ** -0.5
    return _FusedRecurrentGLAFunction.apply(q, k, v, gk, gv, initial_state, float(scale),
                                            bool(output_final_state), bool(reverse), cu)


def _bwd(q, k, v, gk, gv, o, do, dht, scale, initial_state, reverse, cu):
    B, T, H, K = q.shape
    V = v.shape[-1]
    dev = check_device(q, k, v, gk, gv, o, do, dht, initial_state)
    cdt = _compute_dtype(q, k, v, gk, gv, do)
    c = lambda x: None if x is None else x.to(cdt).contiguous()  # noqa: E731
    f = lambda x: None if x is None else x.to(torch.float32).contiguous()  # noqa: E731
    if cu is not None:
        kept, keep = _lib.drop_empty(cu)
        if keep is not None:   # empty sequences: gradients of the others; dh0 = dht for these
            if keep:
                dq, dk, dv, dgk, dgv, dh0 = _bwd(q, k, v, gk, gv, o, do,
                                                 _lib.gather_states(dht, keep), scale,
                                                 _lib.gather_states(initial_state, keep),
                                                 reverse, kept)
            else:
                z = lambda D, on=True: (torch.zeros(B, T, H, D, dtype=torch.float32,  # noqa
                                                    device=dev) if on else None)
                dq, dk, dv, dgk, dgv, dh0 = (z(K), z(K), z(V), z(K, gk is not None),
                                             z(V, gv is not None), None)
            if initial_state is not None:
                dh0 = _lib.scatter_states(dh0, dht, keep, tuple(initial_state.shape), dev)
            return dq, dk, dv, dgk, dgv, dh0
    seq = SeqLayout(B, T, 1, cu, dev)
    dq = _out(B, T, H, K, torch.float32, dev, cu)
    dk = _out(B, T, H, K, torch.float32, dev, cu)
    dv = _out(B, T, H, V, torch.float32, dev, cu)
    dgk = _out(B, T, H, K, torch.float32, dev, cu) if gk is not None else None
    dgv = _out(B, T, H, V, torch.float32, dev, cu) if gv is not None else None
    dh0 = (torch.empty(seq.N, H, K, V, dtype=torch.float32, device=dev)
           if initial_state is not None else None)
    need_ht = dht is not None and (gk is not None or gv is not None)
    ht_ws = torch.empty(seq.N, H, K, V, dtype=torch.float32, device=dev) if need_ht else None
    call("tops_gla_fused_recurrent_bwd", ptr(c(q)), ptr(c(k)), ptr(c(v)), ptr(c(gk)),
         ptr(c(gv)), ptr(f(o)), ptr(c(do)), ptr(f(dht)), ptr(f(initial_state)), ptr(dq),
         ptr(dk), ptr(dv), ptr(dgk), ptr(dgv), ptr(dh0), ptr(ht_ws), float(scale),
         int(bool(reverse)), B, T, H, K, V, ptr(seq.cu), seq.N, dtype_code(cdt),
         stream_of(dev))
    return dq, dk, dv, dgk, dgv, dh0


def fused_recurrent_gla_bwd(q, k, v, gk=None, gv=None, o=None, do=None, dht=None, scale=None,
                            initial_state=None, reverse=False, cu_seqlens=None):
    """Fused recurrent backward. Reference: ``tops/ops/gla/fused_recurrent.py:879-956``.

    Returns ``(dq, dk, dv, dgk, dgv, dh0)``: float32 gradients (the reference's dtype), dgk /
    dgv None without the matching gate, dh0 None without ``initial_state``. ``o`` (the
    forward output) is required when ``gv`` is used.
    """
    B, T, H, K = q.shape
    V = v.shape[-1]
    cu = None if cu_seqlens is None else _lib.to_list(cu_seqlens)
    N = len(cu) - 1 if cu is not None else B
    scale = scale if scale is not None else K ** -0.5
    require(tuple(k.shape) == (B, T, H, K))
    require(tuple(v.shape) == (B, T, H, V))
    require(do is not None and tuple(do.shape) == (B, T, H, V))
    require((gk is None) or (tuple(gk.shape) == (B, T, H, K)))
    require((gv is None) or (tuple(gv.shape) == (B, T, H, V)))
    require((initial_state is None) or (tuple(initial_state.shape) == (N, H, K, V)))
    require((dht is None) or (tuple(dht.shape) == (N, H, K, V)))
    require((cu_seqlens is None) or (B == 1))
    require(gv is None or o is not None, "o (forward output) is required when gv is used")
    return _bwd(q, k, v, gk, gv, o, do, dht, scale, initial_state, reverse, cu)
