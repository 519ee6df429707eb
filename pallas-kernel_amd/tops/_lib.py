"""ctypes binding of ``libtops_gla.so`` (C ABI: ``include/tops_gla.h``).

The library is loaded after torch so that it binds to the HIP runtime torch already loaded
(both carry SONAME ``libamdhip64.so.7``): one runtime, one set of streams in the process.
Every entry point enqueues on torch's current stream of the tensors' device. A missing
library or a non-ROCm tensor raises; nothing falls back to the CPU.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get(
    "TOPS_GLA_LIB", os.path.join(os.path.dirname(_HERE), "lib", "libtops_gla.so"))

F32, BF16 = 0, 1
_DT = {torch.float32: F32, torch.bfloat16: BF16}

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float

# name -> argtypes (order of include/tops_gla.h)
_SIGS = {
    "tops_gla_chunk_local_cumsum": [_P, _P, _I64, _I64, _I64, _I64, _I, _I, _I, _F, _I, _P, _P,
                                    _I64, _I64, _I, _I, _P],
    "tops_gla_chunk_fwd_h": [_P, _P, _P, _I, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64,
                             _I, _P, _P, _I64, _I64, _I, _P],
    "tops_gla_chunk_bwd_dh": [_P, _P, _I, _P, _P, _P, _P, _P, _I64, _F, _I64, _I64, _I64, _I64,
                              _I64, _I, _P, _P, _I64, _I64, _I, _P],
    "tops_gla_chunk_fwd_o": [_P, _P, _P, _P, _I, _P, _P, _P, _P, _F, _I64, _I64, _I64, _I64,
                             _I64, _I, _P, _P, _I64, _I64, _I, _P],
    "tops_gla_chunk_ws_bytes": [_I64, _I64, _I64, _I64, _I64, _I, _I64, _I, _I, _I],
    "tops_gla_chunk_fwd": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _F, _I64, _I64, _I64, _I64,
                           _I64, _I, _P, _P, _I64, _I64, _I, _P],
    "tops_gla_chunk_fwd_noalloc": [_P, _P, _P, _P, _P, _P, _P, _P, _F, _I64, _I64, _I64, _I64,
                                   _I64, _I, _P, _P, _I64, _I64, _I, _P],
    "tops_gla_chunk_bwd": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64,
                           _F, _I64, _I64, _I64, _I64, _I64, _I, _P, _P, _I64, _I64, _I, _P],
    "tops_gla_chunk_bwd_dqkg": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _F, _I64, _I64, _I64,
                                _I64, _I64, _I, _P, _P, _I64, _I64, _I, _P],
    "tops_gla_chunk_bwd_dv": [_P, _P, _P, _P, _P, _P, _F, _I64, _I64, _I64, _I64, _I64, _I, _P,
                              _P, _I64, _I64, _I, _P],
    "tops_gla_fused_recurrent_fwd": [_P, _P, _P, _P, _P, _P, _P, _P, _F, _I, _I64, _I64, _I64,
                                     _I64, _I64, _P, _I64, _I, _I, _P],
    "tops_gla_fused_recurrent_bwd": [_P] * 16 + [_F, _I, _I64, _I64, _I64, _I64, _I64, _P,
                                                 _I64, _I, _P],
    "tops_gla_full_head": [_I64, _I64, _I, _I, _I],
    "tops_gla_simple_chunk_fwd": [_P] * 4 + [_I64] + [_P] * 5 + [_I64, _F] + [_I64] * 5 +
                                 [_I, _P, _P, _I64, _I64, _I, _P],
    "tops_gla_simple_chunk_bwd": [_P] * 4 + [_I64] + [_P] * 11 + [_I64, _F] + [_I64] * 5 +
                                 [_I, _P, _P, _I64, _I64, _I, _P],
    "tops_gla_rmsnorm_gated_fwd": [_P, _P, _P, _P, _P, _I64, _I64, _F, _I, _P],
    "tops_gla_rmsnorm_gated_bwd": [_P] * 9 + [_I64, _I64, _I64, _I, _P],
    "tops_gla_rmsnorm_ws_bytes": [_I64, _I64],
    "tops_gla_gate_logsigmoid_fwd": [_P, _P, _I64, _F, _I, _F, _I, _P],
    "tops_gla_gate_logsigmoid_bwd": [_P, _P, _P, _I64, _F, _I, _F, _I, _P],
    "tops_gla_concat_cols": [_P, _P, _I, _I64, _P, _I, _P],
    "tops_gla_short_conv_fwd": [_P, _P, _P, _P, _I64, _I64, _I64, _I, _I, _P, _I64, _I64, _I,
                                _P],
    "tops_gla_short_conv_bwd": [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I, _I, _P,
                                _I64, _I64, _I, _P],
    "tops_gla_short_conv_ws_bytes": [_I64, _I64, _I64, _I, _I64, _I64, _I],
    "tops_gla_bwd_part_dA": [_P, _P, _P, _F, _I64, _I64, _I64, _I64, _I, _P],
    "tops_gla_bwd_part_dv": [_P] * 6 + [_I64] * 5 + [_I, _P],
    "tops_gla_bwd_part_dqk_intra": [_P] * 6 + [_I64] * 4 + [_I, _P],
    "tops_gla_bwd_part_dqkg": [_P] * 12 + [_F] + [_I64] * 5 + [_I, _P],
}
_SIGS["tops_gla_kernel_timing"] = [_I]
_SIGS["tops_gla_kernel_ms"] = [_I]

# entry points that do not return a status code
_RESTYPE = {"tops_gla_chunk_ws_bytes": ctypes.c_int64, "tops_gla_kernel_ms": ctypes.c_float,
            "tops_gla_rmsnorm_ws_bytes": ctypes.c_int64,
            "tops_gla_short_conv_ws_bytes": ctypes.c_int64}

EXPORTED = ["tops_gla_last_error", "tops_gla_version"] + list(_SIGS)


class ArgumentError(ValueError, AssertionError):
    """A refused argument. The reference reports these with ``assert`` (AssertionError); the
    checks here guard device memory accesses, so they are real raises that ``python -O``
    keeps, and the type is both a ValueError and an AssertionError so that callers written
    against either keep working."""


def require(cond, msg="invalid argument"):
    """Raise ArgumentError(msg) unless cond."""
    if not cond:
        raise ArgumentError(msg)


_lib = None
_lock = threading.Lock()


def load():
    """Load the shared library (once) and declare every prototype."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"tops GLA: {LIB_PATH} is not built; run `python -c 'import "
                    f"__graft_entry__ as g; g.build()'` or `make -C pallas-kernel_amd/csrc`")
            lib = ctypes.CDLL(LIB_PATH)
            lib.tops_gla_last_error.restype = ctypes.c_char_p
            lib.tops_gla_last_error.argtypes = []
            lib.tops_gla_version.restype = ctypes.c_char_p
            lib.tops_gla_version.argtypes = []
            for name, args in _SIGS.items():
                fn = getattr(lib, name)
                fn.argtypes = args
                fn.restype = _RESTYPE.get(name, ctypes.c_int)
            _lib = lib
    return _lib


def call(name, *args):
    """Invoke ``name``; map the C status to a Python exception."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.tops_gla_last_error().decode()
        if rc == 1:
            raise ValueError(f"{name}: {msg}")
        if rc == 2:
            raise NotImplementedError(f"{name}: {msg}")
        raise RuntimeError(f"{name}: {msg}")


def full_head(K, V, chunk, dtype, backward):
    """True when the full-head kernels run this shape (see tops_gla_full_head)."""
    return bool(load().tops_gla_full_head(K, V, chunk, dtype_code(dtype), int(bool(backward))))


def seg_workspace(B, T, H, K, V, chunk, varlen, dtype, device, N=None, backward=False):
    """Workspace of tops_gla_chunk_fwd (``backward`` false) or tops_gla_chunk_bwd (true):
    sequence segments, gate-range flags, wide heads' gating, and for the backward the
    fallback's final states. Returns (tensor or None, bytes). ``varlen``: the cu_seqlens list
    (or a true value with ``N`` given), else falsy."""
    if N is None:
        N = len(varlen) - 1 if isinstance(varlen, (list, tuple)) else B
    n = int(load().tops_gla_chunk_ws_bytes(B, T, H, K, V, chunk, N, int(bool(varlen)),
                                           dtype_code(dtype), int(bool(backward))))
    if n <= 0:
        return None, 0
    return torch.empty(n, dtype=torch.uint8, device=device), n


class _DevPtr(ctypes.c_void_p):
    """A tensor's device pointer that keeps the tensor alive: ``ptr(x.contiguous())`` inside
    an argument list must not let a temporary go back to the caching allocator (and be
    handed to the next temporary) before the entry point has enqueued its kernels."""


def ptr(t):
    """Device pointer of a tensor (None -> NULL); holds a reference to the tensor."""
    if t is None:
        return None
    p = _DevPtr(t.data_ptr())
    p.tensor = t
    return p


def dtype_code(dt):
    if dt not in _DT:
        raise TypeError(f"tops GLA kernels take float32 or bfloat16, got {dt}")
    return _DT[dt]


def check_device(*tensors):
    """All tensors on one ROCm device; returns it."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(
                "tops GLA runs only on a ROCm GPU (tensor on %s); there is no CPU path" % t.device)
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} vs {t.device}")
    return dev


def stream_of(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


class SeqLayout:
    """Sequence/chunk description passed to every chunked entry point.

    Fixed-length: ``N = B`` sequences of T tokens. Varlen (``cu_seqlens``, B == 1): token
    offsets and per-sequence chunk offsets uploaded as int32 device arrays (cached).
    """

    _cache: dict = {}

    def __init__(self, B, T, chunk, cu_seqlens, device):
        self.B, self.T, self.C = int(B), int(T), int(chunk)
        if cu_seqlens is None:
            self.N = self.B
            self.NC = self.B * ((self.T + self.C - 1) // self.C)
            self.cu = self.chunk_cu = None
            self.cu_list = None
            return
        cu = to_list(cu_seqlens)
        require(self.B == 1, f"cu_seqlens requires B == 1, got B={self.B}")
        # every sequence holds at least one token: the kernels read a sequence's last row, so
        # an empty one is refused here rather than indexed (chunk_gla, fused_recurrent_gla and
        # the simple-GLA entry points leave empty sequences out before they get here)
        require(len(cu) >= 2 and cu[0] == 0 and all(b > a for a, b in zip(cu, cu[1:])),
                f"cu_seqlens must be strictly increasing from 0 (no empty sequences): {cu}")
        require(cu[-1] <= self.T, f"cu_seqlens[-1]={cu[-1]} exceeds T={self.T}")
        self.cu_list = cu
        self.N = len(cu) - 1
        nch = [(b - a + self.C - 1) // self.C for a, b in zip(cu, cu[1:])]
        coff = [0]
        for n in nch:
            coff.append(coff[-1] + n)
        self.NC = coff[-1]
        key = (tuple(cu), self.C, str(device))
        hit = SeqLayout._cache.get(key)
        if hit is None:
            hit = (torch.tensor(cu, dtype=torch.int32, device=device),
                   torch.tensor(coff, dtype=torch.int32, device=device))
            if len(SeqLayout._cache) > 64:
                SeqLayout._cache.clear()
            SeqLayout._cache[key] = hit
        self.cu, self.chunk_cu = hit

    def args(self):
        """``cu_seqlens, chunk_offsets, N, NC`` as C arguments."""
        return (ptr(self.cu), ptr(self.chunk_cu), self.N, self.NC)


def drop_empty(cu):
    """Varlen layouts may hold empty sequences: the reference gives one zero chunks
    (``chunk.py:751-793``) and its recurrence over zero tokens leaves the state as it was
    (``naive.py:56-80``). The kernels read a sequence's last row, so the host leaves empty
    sequences out: returns ``(cu without them, indices of the kept sequences)``, or
    ``(cu, None)`` when every sequence holds a token."""
    keep = [i for i in range(len(cu) - 1) if cu[i + 1] > cu[i]]
    if len(keep) == len(cu) - 1:
        return cu, None
    return [cu[0]] + [cu[i + 1] for i in keep], keep


def scatter_states(part, base, keep, shape, device):
    """Final states of every sequence from those of the kept ones (``part``, may be None when
    nothing was kept): an empty sequence's final state is its initial state (``base``, or
    zeros). Differentiable w.r.t. both."""
    full = (base.to(torch.float32) if base is not None
            else torch.zeros(shape, dtype=torch.float32, device=device))
    if part is None or not keep:
        return full.clone()
    idx = torch.tensor(keep, dtype=torch.long, device=device)
    return full.index_copy(0, idx, part.to(torch.float32))


def gather_states(x, keep):
    """The rows of the kept sequences of a per-sequence state tensor (or None)."""
    if x is None:
        return None
    return x.index_select(0, torch.tensor(keep, dtype=torch.long, device=x.device))


def to_list(cu):
    if isinstance(cu, torch.Tensor):
        return [int(x) for x in cu.detach().cpu().reshape(-1).tolist()]
    try:
        import numpy as np

        return [int(x) for x in np.asarray(cu).reshape(-1).tolist()]
    except Exception:  # pragma: no cover - plain sequences
        return [int(x) for x in cu]
