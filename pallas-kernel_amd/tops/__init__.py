"""tops (MI355X): Gated Linear Attention on hand-written HIP kernels for gfx950.

Mirrors the public API of the reference package ``tops`` (``tops.ops.gla``) over torch
tensors on a ROCm device. Every compute call goes through ``libtops_gla.so`` (C ABI in
``include/tops_gla.h``); there is no CPU fallback.
"""

__version__ = "0.1.0"
