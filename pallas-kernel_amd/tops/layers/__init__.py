"""Layers on the MI355X kernels (mirror of the reference's ``tops.layers``)."""

from .gla import GatedLinearAttention

__all__ = ["GatedLinearAttention"]
