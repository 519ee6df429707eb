"""``fused_chunk_gla`` (reference: ``tops/ops/gla/fused_chunk.py:4-30``): delegates to
``chunk_gla`` exactly as the reference does."""

from .chunk import chunk_gla

__all__ = ["fused_chunk_gla"]


def fused_chunk_gla(q, k, v, g, scale=None, initial_state=None, output_final_state=False,
                    cu_seqlens=None, chunk_size=16):
    return chunk_gla(q=q, k=k, v=v, g=g, scale=scale, initial_state=initial_state,
                     output_final_state=output_final_state, cu_seqlens=cu_seqlens,
                     chunk_size=chunk_size)
