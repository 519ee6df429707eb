"""Step recurrence of simple GLA on the recurrent HIP kernel, mirroring
``tops/ops/simple_gla/naive.py``."""

from __future__ import annotations

import torch

from ... import _lib
from ..._lib import require
from ..gla.fused_recurrent import fused_recurrent_gla

__all__ = ["simple_gla_naive"]


def simple_gla_naive(q, k, v, *, g=None, g_gamma=None, scale=None, initial_state=None,
                     output_final_state=False, chunk_size=64, cu_seqlens_cpu=None):
    """``S = S exp(g_t) + k_t^T v_t``, ``o_t = (scale q_t) S`` in float32.
    Reference: ``tops/ops/simple_gla/naive.py:5-94``.

    ``g`` ``[B, T, H, K]`` and ``g_gamma`` (4-D, broadcast to q's shape) are log-decays; the
    step's decay is their sum, either alone, or none (``naive.py:53-60``). With
    ``cu_seqlens_cpu`` the tokens are the flattened ``[B * T]`` axis split into sequences.
    ``chunk_size`` is unused (as in the reference). Returns (o float32 ``[B, T, H, V]``,
    final state float32 ``[N, H, K, V]`` or None).
    """
    del chunk_size
    B, T, H, K = q.shape
    V = v.shape[-1]
    require((g is None) or (g.dim() == 4))
    require((g_gamma is None) or (g_gamma.dim() == 4))
    f32 = torch.float32
    if g is None:
        gate = g_gamma.to(f32).expand(B, T, H, K) if g_gamma is not None else None
    else:
        gate = g.to(f32) + g_gamma.to(f32) if g_gamma is not None else g.to(f32)
    qf, kf, vf = (x.to(f32) for x in (q, k, v))
    cu = None
    if cu_seqlens_cpu is not None:
        cu = _lib.to_list(cu_seqlens_cpu)
        qf, kf = (x.reshape(1, B * T, H, K) for x in (qf, kf))
        vf = vf.reshape(1, B * T, H, V)
        gate = None if gate is None else gate.reshape(1, B * T, H, K)
    h0 = None if initial_state is None else initial_state.to(f32)
    o, ht = fused_recurrent_gla(qf, kf, vf, gk=None if gate is None else gate.contiguous(),
                                scale=K ** -0.5 if scale is None else float(scale),
                                initial_state=h0, output_final_state=output_final_state,
                                cu_seqlens=cu)
    return o.reshape(B, T, H, V).to(f32), (ht if output_final_state else None)
