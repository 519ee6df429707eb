"""Root-mean-square layer norm. Reference: ``tops/modules/layernorm.py:6-35``."""

from __future__ import annotations

import torch

from ._norm import RMSNormGatedFn


class RMSNorm(torch.nn.Module):
    """``x * rsqrt(mean(x^2) + eps) * weight`` over the last dimension (float32 arithmetic,
    output in x's dtype), on the ``tops_gla_rmsnorm_gated`` kernels without a gate.

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

    def forward(self, x):
        return RMSNormGatedFn.apply(x, None, self.weight, self.eps)
