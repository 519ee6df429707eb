"""numpy restatement of the reference's simple GLA (scalar gates): TEST INFRASTRUCTURE ONLY.

Imported only by ``tests/`` as the checker; the product path never imports this module.

Simple GLA is GLA whose log-decay is the same for every key column: a per-head constant
``g_gamma [H]``, a per-token scalar ``g [B, T, H]``, or both (their sum). Functions restate
``tops/ops/simple_gla/{naive,chunk}.py`` and the scalar-gate branches of
``tops/ops/common/chunk_h.py`` / ``chunk_o.py`` (cited per function). Arithmetic in ``dtype``
(float64 by default).

How each function is pinned (``tests/test_oracle.py``):

* ``simple_gla_naive`` -- equals ``gla.naive_recurrent_gla`` with the gates broadcast over
  the key columns (the per-element recurrence it specializes); with zero gates it equals the
  dense causal linear-attention closed form ``o_t = scale sum_{s<=t} (q_t . k_s) v_s``
  computed without any recurrence.
* ``chunk_simple_gla_fwd_intra`` -- the brute-force pairwise closed form
  ``scale (q_i . k_j) exp(gamma (i - j))`` for every (i, j) of a chunk.
* ``chunk_fwd_h_scalar`` / ``chunk_fwd_o_scalar`` / ``chunk_simple_gla_fwd`` /
  ``chunk_simple_gla_fwd_ref`` -- equal ``simple_gla_naive`` (outputs and final states) for
  chunk sizes 16..64, g_gamma, a per-token scalar g given as its chunk-local cumsum, both,
  none, h0, custom scale and varlen.
* ``chunk_simple_gla_bwd`` -- equals torch float64 autograd of an independent naive
  restatement written in the test (dq, dk, dv, dh0).
"""

from __future__ import annotations

import numpy as np

from . import gla

__all__ = [
    "simple_gla_naive",
    "chunk_simple_gla_fwd_intra",
    "chunk_simple_gla_fwd_o",
    "chunk_fwd_h_scalar",
    "chunk_fwd_o_scalar",
    "chunk_simple_gla_fwd",
    "chunk_simple_gla_fwd_ref",
    "chunk_simple_gla_bwd",
    "scalar_cumsum",
]


def _arr(x, dtype):
    return None if x is None else np.asarray(x, dtype=dtype)


def simple_gla_naive(q, k, v, g=None, g_gamma=None, scale=None, initial_state=None,
                     output_final_state=False, cu_seqlens=None, dtype=np.float64):
    """Step recurrence, ``tops/ops/simple_gla/naive.py:5-94``.

    The decay of step t is ``g`` (per element ``[B, T, H, K]``) plus ``g_gamma`` (broadcast to
    it), or either alone, or zero (``naive.py:53-60``); then ``S = S exp(g_t) + k_t^T v_t`` and
    ``o_t = (scale q_t) S`` (``:84-89``). Returns (o, final states or None).
    """
    q, k, v, g, g_gamma = (_arr(x, dtype) for x in (q, k, v, g, g_gamma))
    B, T, H, K = q.shape
    if g is None:
        gate = np.broadcast_to(g_gamma, q.shape) if g_gamma is not None else np.zeros_like(q)
    else:
        gate = g + g_gamma if g_gamma is not None else g
    return gla.naive_recurrent_gla(q, k, v, np.ascontiguousarray(gate), scale, initial_state,
                                   output_final_state, cu_seqlens, dtype)


def scalar_cumsum(g_raw, chunk_size, cu_seqlens=None, dtype=np.float64):
    """Chunk-local cumsum of a per-token scalar gate ``[B, T, H]`` (chunks restart at every
    multiple of chunk_size and at sequence starts), the form ``chunk_fwd_h`` / ``chunk_fwd_o``
    take their scalar ``g`` in (``chunk_h.py:82-86``, ``chunk_o.py:171``)."""
    g_raw = _arr(g_raw, dtype)
    B, T, H = g_raw.shape
    out = np.zeros_like(g_raw)
    for b, _, bos, eos in gla.segments(B, T, cu_seqlens):
        for t0 in range(bos, eos, chunk_size):
            t1 = min(t0 + chunk_size, eos)
            out[b, t0:t1] = np.cumsum(g_raw[b, t0:t1], axis=0)
    return out


def chunk_simple_gla_fwd_intra(q, k, g_gamma, scale, chunk_size=64, dtype=np.float64):
    """Unmasked intra-chunk matrix with the Toeplitz decay,
    ``tops/ops/simple_gla/chunk.py:27-70``: ``A[i, j] = scale (q_i . k_j) exp(g_h (i - j))``
    for every (i, j) of a chunk. Returns ``[B, T, H, C]``."""
    q, k = _arr(q, dtype), _arr(k, dtype)
    gh = _arr(g_gamma, dtype).reshape(-1)
    B, T, H, K = q.shape
    C = chunk_size
    NT = T // C
    A = np.einsum("bnihk,bnjhk->bnihj", q.reshape(B, NT, C, H, K), k.reshape(B, NT, C, H, K))
    pos = np.arange(1, C + 1, dtype=dtype)
    decay = np.exp(gh[None, :, None] * (pos[:, None, None] - pos[None, None, :]))   # [i, h, j]
    return (A * scale * decay[None, None]).reshape(B, T, H, C)


def chunk_simple_gla_fwd_o(q, v, g_gamma, A, h, scale, chunk_size=64, dtype=np.float64):
    """Output combine, ``tops/ops/simple_gla/chunk.py:73-123``:
    ``o_i = scale (q_i exp(g_h (i + 1))) h_n + sum_{j <= i} A_ij v_j``."""
    q, v, A, h = (_arr(x, dtype) for x in (q, v, A, h))
    gh = _arr(g_gamma, dtype).reshape(-1)
    B, T, H, K = q.shape
    V = v.shape[-1]
    C = chunk_size
    qc = q.reshape(-1, C, H, K)
    vc = v.reshape(-1, C, H, V)
    hc = h.reshape(-1, H, K, V)
    Ac = A.reshape(-1, C, H, C)
    pos = np.arange(1, C + 1, dtype=dtype)
    ge = np.exp(gh[None, :] * pos[:, None])                                   # [C, H]
    o_inter = scale * np.einsum("nchk,nhkv->nchv", qc * ge[None, :, :, None], hc)
    mask = np.tril(np.ones((C, C), bool))[:, None, :]
    o_intra = np.einsum("nihj,njhv->nihv", np.where(mask, Ac, 0.0), vc)
    return (o_inter + o_intra).reshape(B, T, H, V)


def _effective_cumsum(B, T, H, g, g_gamma, C, cu_seqlens, dtype):
    """Per-token chunk-local cumsum ``G [B, T, H]`` of the scalar gates: the given cumsum g
    plus the g_gamma ramp ``g_h * (row + 1)`` (``chunk_h.py:82-91``, ``chunk_o.py:216-225``)."""
    G = np.zeros((B, T, H), dtype) if g is None else _arr(g, dtype).copy()
    if g_gamma is not None:
        gh = _arr(g_gamma, dtype).reshape(-1)
        for b, _, bos, eos in gla.segments(B, T, cu_seqlens):
            for t0 in range(bos, eos, C):
                rows = np.arange(min(C, eos - t0), dtype=dtype)
                G[b, t0:t0 + len(rows)] += (rows + 1)[:, None] * gh[None, :]
    return G


def chunk_fwd_h_scalar(k, v, g=None, g_gamma=None, h0=None, output_final_state=False,
                       cu_seqlens=None, chunk_size=64, dtype=np.float64):
    """State at every chunk start with scalar gates, ``tops/ops/common/chunk_h.py:18-119``
    (branches ``:82-91``): ``h <- exp(G_last) h + sum_j (k_j exp(G_last - G_j))^T v_j`` with G
    the effective per-token cumsum, G_last its value at the chunk's last valid row.
    Returns (h [B, NT, H, K, V], ht [N, H, K, V] or zeros)."""
    k, v = _arr(k, dtype), _arr(v, dtype)
    B, T, H, K = k.shape
    G = _effective_cumsum(B, T, H, g, g_gamma, chunk_size, cu_seqlens, dtype)
    return gla.chunk_fwd_h(k, v, np.repeat(G[..., None], K, axis=-1), h0, output_final_state,
                           cu_seqlens, chunk_size, dtype=dtype)


def chunk_fwd_o_scalar(q, k, v, h, g=None, g_gamma=None, scale=None, cu_seqlens=None,
                       chunk_size=64, dtype=np.float64):
    """Chunk output with scalar gates, ``tops/ops/common/chunk_o.py:165-240``:
    ``O_c = scale (Q_c H_c exp(G) + causal(Q_c K_c^T exp(G_i - G_j)) V_c)``."""
    q, k, v, h = (_arr(x, dtype) for x in (q, k, v, h))
    B, T, H, K = q.shape
    V = v.shape[-1]
    C = chunk_size
    scale = K ** -0.5 if scale is None else float(scale)
    G = _effective_cumsum(B, T, H, g, g_gamma, C, cu_seqlens, dtype)
    NT = T // C
    qc, kc = q.reshape(B, NT, C, H, K), k.reshape(B, NT, C, H, K)
    vc, Gc = v.reshape(B, NT, C, H, V), G.reshape(B, NT, C, H)
    hc = h.reshape(B, NT, H, K, V)
    o_inter = np.einsum("bnchk,bnhkv->bnchv", qc, hc) * np.exp(Gc)[..., None]
    A = np.einsum("bnihk,bnjhk->bnihj", qc, kc)
    diff = Gc[:, :, :, :, None] - np.moveaxis(Gc, 2, 3)[:, :, None, :, :]       # [b,n,i,h,j]
    mask = np.tril(np.ones((C, C), bool))[:, None, :]
    A = np.where(mask, A * np.exp(np.where(mask, diff, 0.0)), 0.0)
    o_intra = np.einsum("bnihj,bnjhv->bnihv", A, vc)
    return (scale * (o_inter + o_intra)).reshape(B, T, H, V)


def chunk_simple_gla_fwd(q, k, v, g=None, g_gamma=None, scale=None, h0=None, use_ht=False,
                         cu_seqlens=None, chunk_size=64, dtype=np.float64):
    """``chunk_simple_gla_fwd``, ``tops/ops/simple_gla/chunk.py:471-519``: states by
    ``chunk_fwd_h`` then ``chunk_fwd_o``, both with g (the chunk-local cumsum of a per-token
    scalar gate, ``[B, T, H]``) and / or g_gamma ``[H]``. With cu_seqlens the sequences are
    ``[cu[i], cu[i + 1])`` of the flattened ``B * T`` token axis. Returns (o, ht or None)."""
    q, k, v = (_arr(x, dtype) for x in (q, k, v))
    B, T, H, K = q.shape
    V = v.shape[-1]
    if cu_seqlens is not None:
        q, k, v = (x.reshape(1, B * T, H, -1) for x in (q, k, v))
        g = None if g is None else _arr(g, dtype).reshape(1, B * T, H)
        Bq, Tq = 1, B * T
    else:
        Bq, Tq = B, T
    h, ht = chunk_fwd_h_scalar(k, v, g, g_gamma, h0, use_ht, cu_seqlens, chunk_size, dtype)
    o = chunk_fwd_o_scalar(q, k, v, h, g, g_gamma, scale, cu_seqlens, chunk_size, dtype)
    del Bq, Tq
    return o.reshape(B, T, H, V), (ht if use_ht else None)


def chunk_simple_gla_fwd_ref(q, k, v, g_gamma, scale, initial_state=None,
                             output_final_state=False, chunk_size=64, dtype=np.float64):
    """``chunk_simple_gla_fwd_ref``, ``tops/ops/simple_gla/chunk.py:126-170``: pads T to a
    multiple of the chunk, then states, intra matrix and output. Returns (ht or None, o)."""
    q, k, v = (_arr(x, dtype) for x in (q, k, v))
    B, T, H, K = q.shape
    C = chunk_size
    Tp = -(-T // C) * C
    if Tp != T:
        pad = ((0, 0), (0, Tp - T), (0, 0), (0, 0))
        q, k, v = (np.pad(x, pad) for x in (q, k, v))
    h, ht = chunk_fwd_h_scalar(k, v, None, g_gamma, initial_state, output_final_state, None, C,
                               dtype)
    A = chunk_simple_gla_fwd_intra(q, k, g_gamma, scale, C, dtype)
    o = chunk_simple_gla_fwd_o(q, v, g_gamma, A, h, scale, C, dtype)
    return (ht if output_final_state else None), o[:, :T]


def chunk_simple_gla_bwd(q, k, v, g_gamma, scale, initial_state, do, dht, chunk_size=64,
                         dtype=np.float64):
    """``chunk_simple_gla_bwd``, ``tops/ops/simple_gla/chunk.py:538-615``: the GLA backward on
    the key-column gate built from g_gamma (``_build_gk_from_gamma``, ``:522-535``; dh scan,
    intra matrix and the fused dq / dk / dv). Returns (dq, dk, dv, dh0 or None)."""
    q = _arr(q, dtype)
    H = q.shape[2]
    gg = _arr(g_gamma, dtype).reshape(1, 1, H, 1)
    dq, dk, dv, _, dh0 = gla.chunk_gla_bwd(q, k, v, None, gg, None, scale, initial_state, None,
                                           None, do, dht, None, chunk_size, dtype=dtype)
    return dq, dk, dv, (dh0 if initial_state is not None else None)
