"""Fused recurrent GLA on the MI355X HIP kernel, mirroring
``tops/ops/gla/fused_recurrent.py``.

The state update is element-wise (no matrix product), so the kernel streams the sequence
once, keeps the K x V state in VGPRs and uses only fp32 VALU work plus LDS broadcasts.
"""

from __future__ import annotations

import torch

from ... import _lib
from ..._lib import SeqLayout, call, check_device, dtype_code, ptr, stream_of

__all__ = ["fused_recurrent_gla", "fused_recurrent_gla_fwd", "fused_recurrent_gla_bwd"]


def _run(q, k, v, gk, gv, scale, initial_state, output_final_state, reverse, cu_seqlens,
         out_dtype):
    B, T, H, K = q.shape
    V = v.shape[-1]
    dev = check_device(q, k, v, gk, gv, initial_state)
    xs = [x for x in (q, k, v, gk, gv) if x is not None]
    cdt = torch.bfloat16 if {x.dtype for x in xs} == {torch.bfloat16} else torch.float32
    c = lambda x: None if x is None else x.to(cdt).contiguous()  # noqa: E731
    odt = torch.float32 if out_dtype == torch.float32 or cdt == torch.float32 else cdt
    seq = SeqLayout(B, T, 1, cu_seqlens, dev)
    o = torch.empty(B, T, H, V, dtype=odt, device=dev)
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
    assert tuple(k.shape) == (B, T, H, K), f"Expected k shape {(B, T, H, K)}, got {k.shape}"
    assert tuple(v.shape) == (B, T, H, V), f"Expected v shape {(B, T, H, V)}, got {v.shape}"
    assert (gk is None) or (tuple(gk.shape) == (B, T, H, K)), \
        f"Expected gk shape {(B, T, H, K)}, got {gk.shape}"
    assert (gv is None) or (tuple(gv.shape) == (B, T, H, V)), \
        f"Expected gv shape {(B, T, H, V)}, got {gv.shape}"
    assert (initial_state is None) or (tuple(initial_state.shape) == (N, H, K, V)), \
        f"Expected initial_state shape {(N, H, K, V)}, got {initial_state.shape}"
    assert (cu_seqlens is None) or (B == 1), \
        f"Batch size must be 1 when using cu_seqlens, got {B}"
    return _run(q, k, v, gk, gv, scale, initial_state, output_final_state, reverse, cu,
                torch.float32)


def fused_recurrent_gla(q, k, v, gk=None, gv=None, scale=None, initial_state=None,
                        output_final_state=False, reverse=False, cu_seqlens=None):
    """Fused recurrent GLA, public API. Reference: ``tops/ops/gla/fused_recurrent.py:438-481``.
    """
    return fused_recurrent_gla_fwd(q, k, v, gk=gk, gv=gv, scale=scale,
                                   initial_state=initial_state,
                                   output_final_state=output_final_state, reverse=reverse,
                                   cu_seqlens=cu_seqlens)


def fused_recurrent_gla_bwd(q, k, v, gk=None, gv=None, o=None, do=None, dht=None, scale=None,
                            initial_state=None, reverse=False, cu_seqlens=None):
    """Reference: ``tops/ops/gla/fused_recurrent.py:879-956``. Not yet on the HIP path."""
    raise NotImplementedError(
        "fused_recurrent_gla_bwd is not yet implemented on the HIP path; use chunk_gla's "
        "backward (mathematically identical gradients)")
