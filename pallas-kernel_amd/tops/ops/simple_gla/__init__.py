"""Simple GLA operators: GLA whose log-decay is one scalar per token and head (reference
export list: ``tops/ops/simple_gla/__init__.py:1-3``)."""

from .chunk import (
    chunk_simple_gla_bwd,
    chunk_simple_gla_fwd,
    chunk_simple_gla_fwd_intra_ref,
    chunk_simple_gla_fwd_o_ref,
    chunk_simple_gla_fwd_ref,
)
from .naive import simple_gla_naive

__all__ = [
    "chunk_simple_gla_bwd",
    "chunk_simple_gla_fwd",
    "chunk_simple_gla_fwd_intra_ref",
    "chunk_simple_gla_fwd_o_ref",
    "chunk_simple_gla_fwd_ref",
    "simple_gla_naive",
]
