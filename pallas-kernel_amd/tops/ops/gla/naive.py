"""``naive_recurrent_gla`` (reference: ``tops/ops/gla/naive.py:5-99``).

The reference's step-by-step form is the same recurrence the fused recurrent kernel runs,
so it is served by that kernel, with ``o`` returned in the input dtype as the reference
does (``naive.py:83,99``) and the final state in float32.
"""

from __future__ import annotations

import torch

from ... import _lib
from ..._lib import require
from .fused_recurrent import _run

__all__ = ["naive_recurrent_gla"]


def naive_recurrent_gla(q, k, v, gk, scale=None, initial_state=None, output_final_state=False,
                        cu_seqlens=None):
    B, T, H, K = q.shape
    V = v.shape[-1]
    if cu_seqlens is not None:
        require(B == 1, "cu_seqlens requires B=1")
    N = B if cu_seqlens is None else len(_lib.to_list(cu_seqlens)) - 1
    require(tuple(k.shape) == (B, T, H, K) and tuple(gk.shape) == (B, T, H, K),
            f"Expected k, gk shape {(B, T, H, K)}")
    require(tuple(v.shape) == (B, T, H, V), f"Expected v shape {(B, T, H, V)}")
    require(initial_state is None or tuple(initial_state.shape) == (N, H, K, V),
            f"Expected initial_state shape {(N, H, K, V)}")
    scale = K ** -0.5 if scale is None else scale
    cu = None if cu_seqlens is None else _lib.to_list(cu_seqlens)
    o, ht = _run(q, k, v, gk, None, scale, initial_state, output_final_state, False, cu,
                 q.dtype if q.dtype in (torch.float32, torch.bfloat16) else torch.float32)
    return o.to(q.dtype), ht
