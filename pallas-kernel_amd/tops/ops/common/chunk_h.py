"""Inter-chunk state scans on the MI355X kernels, mirroring ``tops/ops/common/chunk_h.py``.

``chunk_fwd_h_kernel`` / ``chunk_fwd_h_ref`` return the state at the start of every chunk
(``h [B, NT, H, K, V]``) and the final state; ``chunk_bwd_dh_kernel`` / ``chunk_bwd_dh_ref``
return the state gradient at every chunk (``dh``) and ``dh0``. All four run the HIP scans
behind ``tops_gla_chunk_fwd_h`` / ``tops_gla_chunk_bwd_dh``; the ``*_ref`` names keep the
reference's jnp signatures. Gates are chunk-local cumsums: ``gk [B, T, H, K]``, scalar
``g [B, T, H]`` (broadcast over K) or the per-head constant ``g_gamma [H]`` (whose cumsum is
``g_gamma * (i + 1)`` at row i of a chunk).
"""

from __future__ import annotations

import torch

from ... import _lib
from ..._lib import SeqLayout, call, check_device, dtype_code, ptr, require, stream_of

__all__ = ["chunk_fwd_h_kernel", "chunk_fwd_h_ref", "chunk_bwd_dh_kernel", "chunk_bwd_dh_ref"]

_CHUNKS = (4, 8, 16, 32, 64)


def _gate_cumsum(like, g, g_gamma, gk, C, cu):
    """One [B, T, H, K] chunk-local gate cumsum from whichever gate form is given (or None)."""
    B, T, H, K = like.shape
    if gk is not None:
        return gk
    if g is not None:
        return g.unsqueeze(-1).expand(B, T, H, K)
    if g_gamma is not None:
        gg = g_gamma.to(torch.float32).reshape(1, 1, H, 1)
        pos = torch.empty(T, dtype=torch.float32, device=like.device)
        bounds = _lib.to_list(cu) if cu is not None else [0, T]
        for a, b in zip(bounds, bounds[1:]):   # position within the chunk of its sequence
            pos[a:b] = (torch.arange(b - a, device=like.device) % C + 1).to(torch.float32)
        return (pos.reshape(1, T, 1, 1) * gg).expand(B, T, H, K)
    return None


def _check(T, C, cu):
    require(T % C == 0, "T mod chunk_size must equal to 0.")
    if cu is not None:
        require(all(c % C == 0 for c in _lib.to_list(cu)),
                "cu_seqlens must be multiples of chunk_size")


def _kernel_chunk(C):
    """Kernel chunk for chunk size C: C itself (4, 8, 16, 32, 64) or 64 for multiples of 64 (the
    states at C-row boundaries are among the 64-row ones)."""
    if C in _CHUNKS:
        return C
    if C % 64 == 0:
        return 64
    raise NotImplementedError(f"chunk_size {C}: the kernels take 4, 8, 16, 32, 64 or multiples "
                              "of 64")


def _rechunk_cumsum(gc, C, KC, cu):
    """A chunk-local cumsum over C-row chunks as one over KC-row chunks (KC divides C)."""
    if gc is None or KC == C:
        return gc
    B, T, H, K = gc.shape
    x = gc.to(torch.float32).reshape(B, T // KC, KC, H, K)
    starts = set(range(0, T, C)) | (set(_lib.to_list(cu)) if cu is not None else set())
    first = torch.tensor([b * KC in starts for b in range(T // KC)], device=gc.device)
    prev_last = torch.zeros_like(x[:, :, -1])
    prev_last[:, 1:] = x[:, :-1, -1]
    prev_last[:, first] = 0.0
    return (x - prev_last[:, :, None]).reshape(B, T, H, K).to(gc.dtype)


def _fwd(k, v, gk, h0, output_final_state, cu, C, states_in_fp32):
    """States at the start of every C-row chunk (run on C-row kernel chunks)."""
    B, T, H, K = k.shape
    V = v.shape[-1]
    dev = check_device(k, v, gk, h0)
    xs = [k, v] + ([gk] if gk is not None else [])
    cdt = torch.bfloat16 if {x.dtype for x in xs} == {torch.bfloat16} else torch.float32
    kk, vv = k.to(cdt).contiguous(), v.to(cdt).contiguous()
    gg = torch.zeros_like(kk) if gk is None else gk.to(cdt).contiguous()
    seq = SeqLayout(B, T, C, cu, dev)
    N = seq.N
    if h0 is not None:
        require(tuple(h0.shape) == (N, H, K, V), f"Expected h0 shape {(N, H, K, V)}")
    h = torch.empty(B, seq.NC // B, H, K, V, dtype=cdt, device=dev)
    ht = torch.empty(N, H, K, V, dtype=torch.float32, device=dev)
    call("tops_gla_chunk_fwd_h", ptr(kk), ptr(vv), ptr(gg), 1,
         ptr(None if h0 is None else h0.to(torch.float32).contiguous()), ptr(h), ptr(ht), None,
         0, B, T, H, K, V, C, *seq.args(), dtype_code(cdt), stream_of(dev))
    h = h.to(torch.float32 if states_in_fp32 else k.dtype)
    return h, (ht if output_final_state else None)


def _bwd(q, gk, do, dht, scale, cu, C, states_in_fp32, want_dh0):
    """State gradients after every C-row chunk (run on C-row kernel chunks)."""
    B, T, H, K = q.shape
    V = do.shape[-1]
    dev = check_device(q, gk, do, dht)
    xs = [q, do] + ([gk] if gk is not None else [])
    cdt = torch.bfloat16 if {x.dtype for x in xs} == {torch.bfloat16} else torch.float32
    qq, dd = q.to(cdt).contiguous(), do.to(cdt).contiguous()
    gg = torch.zeros_like(qq) if gk is None else gk.to(cdt).contiguous()
    seq = SeqLayout(B, T, C, cu, dev)
    N = seq.N
    if dht is not None:
        require(tuple(dht.shape) == (N, H, K, V), f"Expected dht shape {(N, H, K, V)}")
    dh = torch.empty(B, seq.NC // B, H, K, V, dtype=cdt, device=dev)
    dh0 = torch.empty(N, H, K, V, dtype=torch.float32, device=dev) if want_dh0 else None
    call("tops_gla_chunk_bwd_dh", ptr(qq), ptr(gg), 1, ptr(dd),
         ptr(None if dht is None else dht.to(torch.float32).contiguous()), ptr(dh), ptr(dh0),
         None, 0, float(scale), B, T, H, K, V, C, *seq.args(), dtype_code(cdt), stream_of(dev))
    return dh.to(torch.float32 if states_in_fp32 else q.dtype), dh0


def chunk_fwd_h_kernel(k, v, *, g=None, g_gamma=None, gk=None, gv=None, h0=None,
                       output_final_state=False, cu_seqlens=None, chunk_size=64,
                       split_size=None, states_in_fp32=False, interpret=False):
    """Reference: ``tops/ops/common/chunk_h.py:137-274``. Returns ``(h, ht)``: h
    ``[B, T / split_size, H, K, V]`` (the state at the start of every split, k's dtype or
    float32) and ht float32 ``[N, H, K, V]`` or None. ``interpret`` is accepted for API
    parity."""
    del interpret
    require(gv is None, "gv is not supported by chunk_fwd_h")
    C = chunk_size
    S = C if split_size is None else split_size
    require(S % C == 0, f"The `split_size` (got {S}) must be a multiple of `chunk_size` {C}")
    _check(k.shape[1], S, cu_seqlens)
    KC = _kernel_chunk(C)
    gc = _rechunk_cumsum(_gate_cumsum(k, g, g_gamma, gk, C, cu_seqlens), C, KC, cu_seqlens)
    h, ht = _fwd(k, v, gc, h0, output_final_state, cu_seqlens, KC, states_in_fp32)
    return h[:, ::S // KC], ht


def chunk_fwd_h_ref(k, v, g=None, g_gamma=None, gk=None, gv=None, h0=None,
                    output_final_state=False, states_in_fp32=False, cu_seqlens=None,
                    cu_seqlens_cpu=None, chunk_size=64):
    """Reference: ``tops/ops/common/chunk_h.py:277-396`` (same results on the HIP scan).
    Returns ``(h [B, NT, H, K, V], ht [N, H, K, V] float32 or None)``."""
    require(gv is None, "gv is not supported by chunk_fwd_h")
    cu = cu_seqlens_cpu if cu_seqlens_cpu is not None else cu_seqlens
    C = chunk_size
    _check(k.shape[1], C, cu)
    KC = _kernel_chunk(C)
    gc = _rechunk_cumsum(_gate_cumsum(k, g, g_gamma, gk, C, cu), C, KC, cu)
    h, ht = _fwd(k, v, gc, h0, output_final_state, cu, KC, states_in_fp32)
    return h[:, ::C // KC], ht


def chunk_bwd_dh_kernel(q, k, v, g=None, g_gamma=None, gk=None, do=None, dht=None, scale=1.0,
                        output_dh0=False, cu_seqlens=None, chunk_size=128, split_size=None,
                        states_in_fp32=False, interpret=False):
    """Reference: ``tops/ops/common/chunk_h.py:605-697``. Returns ``(dh, dh0)``: entry i of
    dh ``[B, T / split_size, H, K, V]`` is the gradient of the state after the first chunk
    of split i (the reference stores it there, ``:535-542``); dh0 ``[N, H, K, V]`` float32
    when ``output_dh0``. k and v are unused (as in the reference); ``interpret`` is accepted
    for API parity."""
    del k, v, interpret
    C = chunk_size
    S = C if split_size is None else split_size
    require(S % C == 0, f"The `split_size` (got {S}) must be a multiple of `chunk_size` {C}")
    _check(q.shape[1], S, cu_seqlens)
    KC = _kernel_chunk(C)
    gc = _rechunk_cumsum(_gate_cumsum(q, g, g_gamma, gk, C, cu_seqlens), C, KC, cu_seqlens)
    dh, dh0 = _bwd(q, gc, do, dht, scale, cu_seqlens, KC, states_in_fp32, output_dh0)
    return dh[:, C // KC - 1::S // KC], dh0


def chunk_bwd_dh_ref(q, k, v, gk, do, h0=None, dht=None, scale=1.0, cu_seqlens_cpu=None,
                     chunk_size=64):
    """Reference: ``tops/ops/common/chunk_h.py:399-492``. Returns ``(dh [B, NT, H, K, V]
    float32, dh0 [N, H, K, V] float32 or None)``; dh0 is returned when h0 or dht is given."""
    del k, v
    C = chunk_size
    _check(q.shape[1], C, cu_seqlens_cpu)
    KC = _kernel_chunk(C)
    gc = _rechunk_cumsum(gk, C, KC, cu_seqlens_cpu)
    dh, dh0 = _bwd(q, gc, do, dht, scale, cu_seqlens_cpu, KC, True,
                   h0 is not None or dht is not None)
    return dh[:, C // KC - 1::C // KC], dh0
