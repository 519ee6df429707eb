"""Layer building blocks on the MI355X kernels (mirror of the reference's ``tops.modules``)."""

from .convolution import ShortConvolution
from .fused_norm_gate import FusedRMSNormGated
from .layernorm import RMSNorm

__all__ = ["FusedRMSNormGated", "RMSNorm", "ShortConvolution"]
