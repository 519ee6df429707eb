"""Host-side helpers mirroring ``tops/utils.py`` (reference lines cited per function)."""

from __future__ import annotations

import torch

from ._lib import require


def next_power_of_2(n: int) -> int:
    """Smallest power of two >= n (``tops/utils.py:6-16``)."""
    return 1 if n <= 1 else 1 << (int(n) - 1).bit_length()


def cdiv(x, y: int):
    """Ceiling division (``tops/utils.py:18-25``)."""
    return (x + y - 1) // y


def align_up(x: int, align: int) -> int:
    """Round up to a multiple of ``align`` (``tops/utils.py:28-29``)."""
    return cdiv(x, align) * align


def prepare_lens(cu_seqlens: torch.Tensor) -> torch.Tensor:
    """Per-sequence lengths from cumulative offsets (``tops/utils.py:62-67``)."""
    return cu_seqlens[1:] - cu_seqlens[:-1]


def prepare_chunk_indices(cu_seqlens: torch.Tensor, chunk_size: int) -> torch.Tensor:
    """``[NT, 2]`` (sequence id, chunk id within the sequence) for varlen inputs
    (``tops/utils.py:70-89``)."""
    lens = prepare_lens(torch.as_tensor(cu_seqlens).to(torch.int64).cpu())
    n = cdiv(lens, chunk_size)
    seq_ids = torch.repeat_interleave(torch.arange(len(lens)), n)
    offs = torch.repeat_interleave(torch.cumsum(n, 0) - n, n)
    blk = torch.arange(int(n.sum())) - offs
    return torch.stack([seq_ids, blk], 1).to(torch.int32)


def assert_shape(x, expected_shape, name="tensor"):
    """Shape assertion helper (``tops/utils.py:110-123``)."""
    if isinstance(x, (list, tuple)):
        names = name if isinstance(name, (list, tuple)) and len(name) == len(x) else None
        for i, t in enumerate(x):
            nm = names[i] if names else f"{name}_{i}"
            require(tuple(t.shape) == tuple(expected_shape),
                    f"[{nm}] Expected shape {tuple(expected_shape)}, got {tuple(t.shape)}")
    else:
        require(tuple(x.shape) == tuple(expected_shape),
                f"[{name}] Expected shape {tuple(expected_shape)}, got {tuple(x.shape)}")


def assert_shape_or_none(x, expected_shape, name="tensor"):
    """Like ``assert_shape`` but skips None entries (``tops/utils.py:91-108``)."""
    if x is None:
        return
    if isinstance(x, (list, tuple)):
        names = name if isinstance(name, (list, tuple)) and len(name) == len(x) else None
        for i, t in enumerate(x):
            if t is not None:
                assert_shape(t, expected_shape, names[i] if names else f"{name}_{i}")
    else:
        assert_shape(x, expected_shape, name)


def pad_to_multiple(x: torch.Tensor, multiple, axis, val=0):
    """Right-pad ``axis`` (or several) to a multiple (``tops/utils.py:37-59``)."""
    if isinstance(multiple, int):
        multiple = [multiple]
    if isinstance(axis, int):
        axis = [axis]
    require(len(multiple) == len(axis),
            f"Length of multiple {len(multiple)} must match length of axis {len(axis)}")
    pads = [0] * (2 * x.dim())
    for ax, mu in zip(axis, multiple):
        ax = ax % x.dim()
        rem = x.shape[ax] % mu
        if rem:
            pads[2 * (x.dim() - 1 - ax) + 1] = mu - rem
    if not any(pads):
        return x
    return torch.nn.functional.pad(x, pads, value=val)
