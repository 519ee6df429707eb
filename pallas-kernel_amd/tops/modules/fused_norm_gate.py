"""RMSNorm fused with a SiLU output gate. Reference: ``tops/modules/fused_norm_gate.py:6-37``."""

from __future__ import annotations

import torch

from ._norm import RMSNormGatedFn


class FusedRMSNormGated(torch.nn.Module):
    """``output = RMSNorm(x) * silu(g)`` over the last dimension (float32 arithmetic, output in
    x's dtype), on the ``tops_gla_rmsnorm_gated`` kernels (forward and backward).

    ``rngs`` is accepted for signature parity with the reference (the weight starts at ones).
    """

    def __init__(self, hidden_size, elementwise_affine=True, eps=1e-5, *, rngs=None,
                 device=None):
        super().__init__()
        del rngs
        self.hidden_size = hidden_size
        self.eps = eps
        self.elementwise_affine = elementwise_affine
        if elementwise_affine:
            self.weight = torch.nn.Parameter(torch.ones(hidden_size, dtype=torch.float32,
                                                        device=device))
        else:
            self.register_parameter("weight", None)

    def forward(self, x, g):
        return RMSNormGatedFn.apply(x, g, self.weight, self.eps)
