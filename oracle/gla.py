"""numpy restatement of the reference's GLA algorithms: TEST INFRASTRUCTURE ONLY.

Imported only by ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg, as the checker. The product path never imports this module.

Every public function restates the reference (``/root/reference``, package ``tops``) and
cites the file:line it follows. All arithmetic is done in ``dtype`` (float64 by default;
``bench.py`` times the float32 variant as the CPU baseline, matching the reference's fp32
compute). Shapes follow the reference: ``[B, T, H, D]`` with D fastest; varlen packs
sequences along T with ``B == 1`` and ``cu_seqlens`` of length ``N + 1``.

How each function is pinned (``tests/test_oracle.py``):

* ``naive_recurrent_gla`` -- a dense closed form over all (t, s) pairs on tiny shapes
  (independent of the step loop), state-split continuity, ``output_final_state`` = None.
* ``fused_recurrent_gla_fwd`` -- the same dense closed form with gk and gv gates, equality
  with ``naive_recurrent_gla`` for gk-only, ``reverse`` == forward on time-flipped inputs.
* ``fused_recurrent_gla_bwd`` -- torch float64 autograd of an independent restatement written
  in the test, plus central finite differences on one tiny case.
* ``chunk_local_cumsum`` -- per-chunk ``np.cumsum`` closed form, first row of each chunk equals
  the raw gate, reverse = flipped cumsum, ``scale`` multiplies.
* ``chunk_fwd_h`` -- ``h[:, 0] == h0``, final state equals the naive final state, zero-padding
  invariance.
* ``chunk_gla_fwd_intra_gk`` -- brute-force O(C^2 K) pairwise closed form.
* ``chunk_gla_fwd_o_gk`` / ``chunk_gla_fwd`` / ``chunk_gla`` -- equal to the naive recurrence
  for chunk sizes 4..64, odd T, varlen (aligned and not), h0, custom scale.
* ``chunk_bwd_dh``, ``chunk_gla_bwd_dA/_dv/_dqk_intra/_dqkg``, ``chunk_gla_bwd`` -- the
  composition equals torch float64 autograd of an independent naive restatement, for
  several chunk sizes, h0/dht, odd T and varlen; ``chunk_bwd_dh``'s ``dh0`` equals autograd's
  gradient of the initial state.
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "naive_recurrent_gla",
    "fused_recurrent_gla_fwd",
    "fused_recurrent_gla",
    "fused_recurrent_gla_bwd",
    "chunk_local_cumsum",
    "chunk_fwd_h",
    "chunk_gla_fwd_intra_gk",
    "chunk_gla_fwd_o_gk",
    "chunk_gla_fwd",
    "chunk_gla",
    "chunk_bwd_dh",
    "chunk_gla_bwd_dA",
    "chunk_gla_bwd_dv",
    "chunk_gla_bwd_dqk_intra",
    "chunk_gla_bwd_dqkg",
    "chunk_gla_bwd",
    "segments",
]


def _arr(x, dtype):
    return None if x is None else np.asarray(x, dtype=dtype)


def _scale(scale, K):
    return K ** -0.5 if scale is None else float(scale)


def segments(B, T, cu_seqlens):
    """One ``(batch_row, seq_index, bos, eos)`` per sequence.

    Fixed-length: sequence i is batch row i over ``[0, T)``. Varlen (``B == 1``): sequence i is
    ``[cu[i], cu[i+1])`` of row 0 (``tops/ops/gla/naive.py:49-56``).
    """
    if cu_seqlens is None:
        return [(b, b, 0, T) for b in range(B)]
    cu = [int(c) for c in np.asarray(cu_seqlens).reshape(-1).tolist()]
    assert B == 1, "cu_seqlens requires B=1"
    return [(0, i, cu[i], cu[i + 1]) for i in range(len(cu) - 1)]


# ---------------------------------------------------------------------------
# Recurrent forms
# ---------------------------------------------------------------------------


def naive_recurrent_gla(q, k, v, gk, scale=None, initial_state=None,
                        output_final_state=False, cu_seqlens=None, dtype=np.float64):
    """Step-by-step recurrence, ``tops/ops/gla/naive.py:5-99``.

    ``h_t = h_{t-1} * exp(gk_t)[:, None] + k_t v_t^T``; ``o_t = (scale q_t) h_t`` (decay before
    the update, ``o_t`` includes token t; ``naive.py:89-96``). Returns ``o`` in ``dtype`` (the
    reference casts to the input dtype) and the final state or None.
    """
    q, k, v, gk = (_arr(x, dtype) for x in (q, k, v, gk))
    h0 = _arr(initial_state, dtype)
    B, T, H, K = q.shape
    V = v.shape[-1]
    scale = _scale(scale, K)
    o = np.zeros((B, T, H, V), dtype)
    finals = []
    for b, i, bos, eos in segments(B, T, cu_seqlens):
        h = np.zeros((H, K, V), dtype)
        if h0 is not None:
            h = h + h0[i]
        for t in range(bos, eos):
            h = h * np.exp(gk[b, t])[:, :, None] + k[b, t][:, :, None] * v[b, t][:, None, :]
            o[b, t] = np.einsum("hk,hkv->hv", q[b, t] * scale, h)
        finals.append(h)
    return o, (np.stack(finals) if output_final_state else None)


def fused_recurrent_gla_fwd(q, k, v, g=None, g_gamma=None, gk=None, gv=None, scale=None,
                            initial_state=None, output_final_state=False, reverse=False,
                            cu_seqlens=None, dtype=np.float64):
    """Recurrent forward with every gate kind, ``tops/ops/gla/fused_recurrent.py:17-132``.

    Gates are applied to the state before the rank-1 update in the order g, g_gamma, gk, gv
    (``:103-112``); ``reverse`` walks each sequence from its last token (``:96``). ``o`` is
    returned in ``dtype`` (the reference returns float32, ``:262,369``).
    """
    q, k, v = (_arr(x, dtype) for x in (q, k, v))
    g, g_gamma, gk, gv = (_arr(x, dtype) for x in (g, g_gamma, gk, gv))
    h0 = _arr(initial_state, dtype)
    B, T, H, K = q.shape
    V = v.shape[-1]
    scale = _scale(scale, K)
    o = np.zeros((B, T, H, V), dtype)
    finals = []
    for b, i, bos, eos in segments(B, T, cu_seqlens):
        h = np.zeros((H, K, V), dtype)
        if h0 is not None:
            h = h + h0[i]
        ts = range(eos - 1, bos - 1, -1) if reverse else range(bos, eos)
        for t in ts:
            if g is not None:
                h = h * np.exp(g[b, t])[:, None, None]
            if g_gamma is not None:
                h = h * np.exp(g_gamma)[:, None, None]
            if gk is not None:
                h = h * np.exp(gk[b, t])[:, :, None]
            if gv is not None:
                h = h * np.exp(gv[b, t])[:, None, :]
            h = h + k[b, t][:, :, None] * v[b, t][:, None, :]
            o[b, t] = np.einsum("hk,hkv->hv", q[b, t] * scale, h)
        finals.append(h)
    return o, (np.stack(finals) if output_final_state else None)


def fused_recurrent_gla(q, k, v, gk=None, gv=None, scale=None, initial_state=None,
                        output_final_state=False, reverse=False, cu_seqlens=None,
                        dtype=np.float64):
    """Public signature of ``tops/ops/gla/fused_recurrent.py:438-481`` (gk/gv gates only)."""
    return fused_recurrent_gla_fwd(q, k, v, gk=gk, gv=gv, scale=scale,
                                   initial_state=initial_state,
                                   output_final_state=output_final_state, reverse=reverse,
                                   cu_seqlens=cu_seqlens, dtype=dtype)


def fused_recurrent_gla_bwd(q, k, v, gk=None, gv=None, o=None, do=None, dht=None, scale=None,
                            initial_state=None, reverse=False, cu_seqlens=None,
                            dtype=np.float64):
    """Recurrent backward, ``tops/ops/gla/fused_recurrent.py:879-956`` (API and returns).

    Computed with the direct reverse recurrence of
    ``tests/src/ops/common/fused_recurrent.py:141-305``: ``dh_t += scale q_t do_t^T``;
    ``dk_t = dh_t v_t``; ``dv_t = dh_t^T k_t``; ``dq_t = scale h_t do_t``;
    ``dgk_t = sum_v dh_t * (G_t h_{t-1})``; ``dgv_t = sum_k dh_t * (G_t h_{t-1})``;
    ``dh_{t-1} = G_t dh_t``. ``o`` is accepted for API parity (the reference needs it for gv).
    Returns ``(dq, dk, dv, dgk, dgv, dh0)``; ``dh0`` is None without ``initial_state``.
    """
    del o
    q, k, v, do = (_arr(x, dtype) for x in (q, k, v, do))
    gk, gv, dht = (_arr(x, dtype) for x in (gk, gv, dht))
    h0 = _arr(initial_state, dtype)
    B, T, H, K = q.shape
    V = v.shape[-1]
    scale = _scale(scale, K)
    dq = np.zeros_like(q)
    dk = np.zeros_like(k)
    dv = np.zeros_like(v)
    dgk = np.zeros_like(q) if gk is not None else None
    dgv = np.zeros_like(v) if gv is not None else None
    dh0s = []
    for b, i, bos, eos in segments(B, T, cu_seqlens):
        ts = list(range(eos - 1, bos - 1, -1) if reverse else range(bos, eos))
        h = np.zeros((H, K, V), dtype)
        if h0 is not None:
            h = h + h0[i]
        gated = {}
        for t in ts:
            hg = h
            if gk is not None:
                hg = hg * np.exp(gk[b, t])[:, :, None]
            if gv is not None:
                hg = hg * np.exp(gv[b, t])[:, None, :]
            gated[t] = hg
            h = hg + k[b, t][:, :, None] * v[b, t][:, None, :]
            dq[b, t] = scale * np.einsum("hkv,hv->hk", h, do[b, t])
        dh = np.zeros((H, K, V), dtype)
        if dht is not None:
            dh = dh + dht[i]
        for t in reversed(ts):
            dh = dh + scale * q[b, t][:, :, None] * do[b, t][:, None, :]
            dk[b, t] = np.einsum("hkv,hv->hk", dh, v[b, t])
            dv[b, t] = np.einsum("hkv,hk->hv", dh, k[b, t])
            if gk is not None:
                dgk[b, t] = (dh * gated[t]).sum(-1)
            if gv is not None:
                dgv[b, t] = (dh * gated[t]).sum(-2)
            if gv is not None:
                dh = dh * np.exp(gv[b, t])[:, None, :]
            if gk is not None:
                dh = dh * np.exp(gk[b, t])[:, :, None]
        dh0s.append(dh)
    dh0 = np.stack(dh0s) if h0 is not None else None
    return dq, dk, dv, dgk, dgv, dh0


# ---------------------------------------------------------------------------
# Chunked forms
# ---------------------------------------------------------------------------


def chunk_local_cumsum(g, chunk_size, reverse=False, scale=None, cu_seqlens=None,
                       head_first=False, dtype=np.float64):
    """Chunk-local (optionally reverse) prefix sum, ``tops/ops/gla/chunk.py:55-198``.

    Chunks start at each sequence's first token and the last chunk of a sequence may be
    partial (``chunk.py:70-83``); ``scale`` multiplies the result (``:104-105``);
    ``head_first`` means ``[B, H, T, S]`` input/output (``:123-128``).
    """
    assert chunk_size == 2 ** (chunk_size.bit_length() - 1), "chunk_size must be power of 2"
    g = _arr(g, dtype)
    if head_first:
        g = g.transpose(0, 2, 1, 3)
    B, T, H, S = g.shape
    C = chunk_size
    out = np.zeros_like(g)
    for b, _, bos, eos in segments(B, T, cu_seqlens):
        for c0 in range(bos, eos, C):
            c1 = min(c0 + C, eos)
            blk = g[b, c0:c1]
            out[b, c0:c1] = np.cumsum(blk[::-1], 0)[::-1] if reverse else np.cumsum(blk, 0)
    if scale is not None:
        out = out * scale
    if head_first:
        out = out.transpose(0, 2, 1, 3)
    return out


def chunk_fwd_h(k, v, gk=None, h0=None, output_final_state=False, cu_seqlens=None,
                chunk_size=64, dtype=np.float64):
    """State at the start of every chunk, ``tops/ops/gla/chunk.py:206-292``.

    ``gk`` is the chunk-local cumsum. ``h[n] = h_n``; ``h_{n+1} = exp(gamma_n) h_n +
    (k * exp(gamma_n - gk))^T v`` with ``gamma_n`` the chunk's last cumsum row
    (``chunk.py:270-289``). Requires ``T % C == 0`` (and chunk-aligned ``cu_seqlens``).
    Returns ``h [B, NT, H, K, V]`` and ``ht [N, H, K, V]`` (zeros unless
    ``output_final_state``, as ``chunk.py:246,290-291``).
    """
    k, v, gk, h0 = (_arr(x, dtype) for x in (k, v, gk, h0))
    B, T, H, K = k.shape
    V = v.shape[-1]
    C = chunk_size
    assert T % C == 0, "T must be a multiple of chunk_size for chunk_fwd_h"
    segs = segments(B, T, cu_seqlens)
    for _, _, bos, eos in segs:
        assert bos % C == 0 and eos % C == 0, "cu_seqlens must be multiples of chunk_size"
    h_all = np.zeros((B, T // C, H, K, V), dtype)
    ht = np.zeros((len(segs), H, K, V), dtype)
    for b, i, bos, eos in segs:
        h = np.zeros((H, K, V), dtype)
        if h0 is not None:
            h = h + h0[i]
        for t0 in range(bos, eos, C):
            h_all[b, t0 // C] = h
            bk, bv = k[b, t0:t0 + C], v[b, t0:t0 + C]
            if gk is not None:
                bg = gk[b, t0:t0 + C]
                last = bg[-1]
                h = h * np.exp(last)[:, :, None]
                bk = bk * np.exp(last[None] - bg)
            h = h + np.einsum("chk,chv->hkv", bk, bv)
        if output_final_state:
            ht[i] = h
    return h_all, ht


def chunk_gla_fwd_intra_gk(q, k, g, scale, chunk_size=64, dtype=np.float64):
    """Unmasked intra-chunk matrix, ``tops/ops/gla/chunk.py:300-342``.

    ``A[i, j] = scale * sum_k q_ik k_jk exp(g_ik - g_jk)`` for every (i, j) of a chunk, with
    the chunk's first row as the exponent reference (``chunk.py:329-332``). Returns
    ``[B, T, H, C]``.
    """
    q, k, g = (_arr(x, dtype) for x in (q, k, g))
    B, T, H, K = q.shape
    C = chunk_size
    assert T % C == 0
    NT = T // C
    qc, kc, gc = (x.reshape(B, NT, C, H, K) for x in (q, k, g))
    gn = gc[:, :, 0:1]
    A = np.einsum("bnihk,bnjhk->bnihj", qc * np.exp(gc - gn), kc * np.exp(gn - gc)) * scale
    return A.reshape(B, T, H, C)


def chunk_gla_fwd_o_gk(q, v, g, A, h, scale, chunk_size=64, dtype=np.float64):
    """Output combine, ``tops/ops/gla/chunk.py:441-496``.

    ``o_i = scale (q_i * exp(g_i)) h_n + sum_{j <= i} A_ij v_j`` (causal mask ``:484-489``).
    """
    q, v, g, A, h = (_arr(x, dtype) for x in (q, v, g, A, h))
    B, T, H, K = q.shape
    V = v.shape[-1]
    C = chunk_size
    assert T % C == 0
    qc = q.reshape(-1, C, H, K)
    vc = v.reshape(-1, C, H, V)
    gc = g.reshape(-1, C, H, K)
    hc = h.reshape(-1, H, K, V)
    Ac = A.reshape(-1, C, H, C)
    o_inter = scale * np.einsum("nchk,nhkv->nchv", qc * np.exp(gc), hc)
    mask = np.tril(np.ones((C, C), bool))[:, None, :]
    o_intra = np.einsum("nihj,njhv->nihv", np.where(mask, Ac, 0.0), vc)
    return (o_inter + o_intra).reshape(B, T, H, V)


def _pad_chunks(tensors, B, T, cu_seqlens, C):
    """Pad T (fixed-length) or every varlen segment (``chunk.py:751-793``) to a multiple of C.

    Returns ``(padded tensors, padded cu_seqlens or None, unpad function)``.
    """
    if cu_seqlens is None:
        Tp = -(-T // C) * C
        if Tp == T:
            return tensors, None, lambda x: x
        pw = ((0, 0), (0, Tp - T), (0, 0), (0, 0))
        return [np.pad(x, pw) for x in tensors], None, lambda x: x[:, :T]
    segs = segments(B, T, cu_seqlens)
    lens = [eos - bos for _, _, bos, eos in segs]
    plens = [-(-L // C) * C for L in lens]
    new_cu = np.concatenate([[0], np.cumsum(plens)]).astype(np.int64)
    if lens == plens:
        return tensors, new_cu, lambda x: x
    out = []
    for x in tensors:
        parts = []
        for (_, _, bos, eos), pL in zip(segs, plens):
            seg = x[:, bos:eos]
            parts.append(np.pad(seg, ((0, 0), (0, pL - (eos - bos))) + ((0, 0),) * (x.ndim - 2)))
        out.append(np.concatenate(parts, axis=1))

    def unpad(x):
        return np.concatenate([x[:, new_cu[i]:new_cu[i] + L] for i, L in enumerate(lens)], 1)

    return out, new_cu, unpad


def chunk_gla_fwd(q, k, v, g, g_gamma, g_cumsum, scale, initial_state, output_final_state,
                  cu_seqlens=None, chunk_size=64, dtype=np.float64):
    """Forward orchestrator, ``tops/ops/gla/chunk.py:1083-1179``.

    Defaults ``g`` to the broadcast ``g_gamma`` or zeros (``:1114-1118``), pads T / varlen
    segments to a multiple of the chunk size (``:1120-1126``), then cumsum, state scan,
    intra matrix and output. Returns ``(g_cumsum, A, h, ht, o)`` with g_cumsum, A and h in
    the padded chunk layout and ``o`` unpadded; ``ht`` is None unless requested.
    """
    q, k, v = (_arr(x, dtype) for x in (q, k, v))
    B, T, H, K = q.shape
    C = chunk_size
    if g is None:
        g = np.broadcast_to(_arr(g_gamma, dtype), q.shape) if g_gamma is not None else \
            np.zeros_like(q)
    g = _arr(g, dtype)
    (q, k, v, g), cu, unpad = _pad_chunks([q, k, v, g], B, T, cu_seqlens, C)
    if g_cumsum is None:
        g_cumsum = chunk_local_cumsum(g, C, cu_seqlens=cu, dtype=dtype)
    h, ht = chunk_fwd_h(k, v, g_cumsum, initial_state, output_final_state, cu, C, dtype=dtype)
    A = chunk_gla_fwd_intra_gk(q, k, g_cumsum, scale, C, dtype=dtype)
    o = chunk_gla_fwd_o_gk(q, v, g_cumsum, A, h, scale, C, dtype=dtype)
    return g_cumsum, A, h, (ht if output_final_state else None), unpad(o)


def chunk_gla(q, k, v, g=None, g_gamma=None, scale=None, initial_state=None,
              output_final_state=False, cu_seqlens=None, chunk_size=16, dtype=np.float64):
    """Public chunked forward, ``tops/ops/gla/chunk.py:1187-1251``: returns ``(o, ht|None)``."""
    K = np.shape(q)[-1]
    _, _, _, ht, o = chunk_gla_fwd(q, k, v, g, g_gamma, None, _scale(scale, K), initial_state,
                                   output_final_state, cu_seqlens, chunk_size, dtype=dtype)
    return o, ht


# ---------------------------------------------------------------------------
# Chunked backward
# ---------------------------------------------------------------------------


def chunk_bwd_dh(q, gk, do, h0=None, dht=None, scale=1.0, cu_seqlens=None, chunk_size=64,
                 dtype=np.float64):
    """Reverse state-gradient scan, ``tops/ops/common/chunk_h.py:399-492``.

    ``dh[n]`` is the gradient w.r.t. the state after chunk n: store, then
    ``dh <- exp(gamma_n) dh + (scale q exp(gk))^T do`` (``:464-487``); ``dh0`` is the final
    value, returned when ``h0`` or ``dht`` is given (``:445-449``).
    """
    q, gk, do, dht = (_arr(x, dtype) for x in (q, gk, do, dht))
    B, T, H, K = q.shape
    V = do.shape[-1]
    C = chunk_size
    assert T % C == 0
    segs = segments(B, T, cu_seqlens)
    dh_all = np.zeros((B, T // C, H, K, V), dtype)
    dh0 = np.zeros((len(segs), H, K, V), dtype) if (h0 is not None or dht is not None) \
        else None
    for b, i, bos, eos in segs:
        dh = np.zeros((H, K, V), dtype)
        if dht is not None:
            dh = dh + dht[i]
        for t0 in range(eos - C, bos - 1, -C):
            dh_all[b, t0 // C] = dh
            bq, bdo = q[b, t0:t0 + C], do[b, t0:t0 + C]
            if gk is not None:
                bg = gk[b, t0:t0 + C]
                qh = bq * np.exp(bg) * scale
                dh = dh * np.exp(bg[-1])[:, :, None]
            else:
                qh = bq * scale
            dh = dh + np.einsum("chk,chv->hkv", qh, bdo)
        if dh0 is not None:
            dh0[i] = dh
    return dh_all, dh0


def chunk_gla_bwd_dA(v, do, scale, chunk_size=64, dtype=np.float64):
    """``dA = scale tril(do v^T)`` per chunk, ``tops/ops/gla/chunk.py:504-539``."""
    v, do = _arr(v, dtype), _arr(do, dtype)
    B, T, H, V = v.shape
    C = chunk_size
    NT = T // C
    dA = np.einsum("bnihv,bnjhv->bnihj", do.reshape(B, NT, C, H, V),
                   v.reshape(B, NT, C, H, V)) * scale
    mask = np.tril(np.ones((C, C), bool))[None, None, :, None, :]
    return np.where(mask, dA, 0.0).reshape(B, T, H, C)


def chunk_gla_bwd_dv(k, g_cumsum, A, do, dh, chunk_size=64, dtype=np.float64):
    """``dv = tril(A)^T do + (k exp(gamma - g)) dh``, ``tops/ops/gla/chunk.py:547-595``."""
    k, g, A, do, dh = (_arr(x, dtype) for x in (k, g_cumsum, A, do, dh))
    B, T, H, K = k.shape
    V = do.shape[-1]
    C = chunk_size
    NT = T // C
    kc, gc = k.reshape(B, NT, C, H, K), g.reshape(B, NT, C, H, K)
    doc, Ac = do.reshape(B, NT, C, H, V), A.reshape(B, NT, C, H, C)
    mask = np.tril(np.ones((C, C), bool))[None, None, :, None, :]
    dv_intra = np.einsum("bnihj,bnihv->bnjhv", np.where(mask, Ac, 0.0), doc)
    gn = gc[:, :, -1]
    dv_inter = np.einsum("bnchk,bnhkv->bnchv", kc * np.exp(gn[:, :, None] - gc), dh)
    return (dv_intra + dv_inter).reshape(B, T, H, V)


def chunk_gla_bwd_dqk_intra(q, k, g_cumsum, dA, chunk_size=64, dtype=np.float64):
    """Intra-chunk dq, dk from dA, ``tops/ops/gla/chunk.py:603-648``."""
    q, k, g, dA = (_arr(x, dtype) for x in (q, k, g_cumsum, dA))
    B, T, H, K = q.shape
    C = chunk_size
    NT = T // C
    qc, kc, gc = (x.reshape(B, NT, C, H, K) for x in (q, k, g))
    dAc = dA.reshape(B, NT, C, H, C)
    dq = np.exp(gc) * np.einsum("bnihj,bnjhk->bnihk", dAc, kc * np.exp(-gc))
    dk = np.exp(-gc) * np.einsum("bnihj,bnihk->bnjhk", dAc, qc * np.exp(gc))
    return dq.reshape(B, T, H, K), dk.reshape(B, T, H, K)


def chunk_gla_bwd_dqkg(q, k, v, h, g_cumsum, do, dh, dq, dk, scale, chunk_size=64,
                       dtype=np.float64):
    """Inter-chunk dq, dk and the gate gradient, ``tops/ops/gla/chunk.py:656-743``.

    ``dg = revcumsum_chunk(q dq - k dk) + exp(gamma) sum_v(h dh) + sum_j dk_inter k``.
    """
    q, k, v, h, g, do, dh, dq, dk = (_arr(x, dtype) for x in (q, k, v, h, g_cumsum, do, dh,
                                                              dq, dk))
    B, T, H, K = q.shape
    V = v.shape[-1]
    C = chunk_size
    NT = T // C
    qc, kc, gc, dqc, dkc = (x.reshape(B, NT, C, H, K) for x in (q, k, g, dq, dk))
    vc, doc = v.reshape(B, NT, C, H, V), do.reshape(B, NT, C, H, V)
    gn = gc[:, :, -1]
    dq_inter = scale * np.exp(gc) * np.einsum("bnchv,bnhkv->bnchk", doc, h)
    dk_inter = np.exp(gn[:, :, None] - gc) * np.einsum("bnchv,bnhkv->bnchk", vc, dh)
    dqt, dkt = dqc + dq_inter, dkc + dk_inter
    dgk_inter = np.exp(gn) * np.einsum("bnhkv,bnhkv->bnhk", h, dh) + (dk_inter * kc).sum(2)
    dg_raw = qc * dqt - kc * dkt
    dg = np.cumsum(dg_raw[:, :, ::-1], axis=2)[:, :, ::-1] + dgk_inter[:, :, None]
    return dqt.reshape(B, T, H, K), dkt.reshape(B, T, H, K), dg.reshape(B, T, H, K)


def chunk_gla_bwd(q, k, v, g, g_gamma, g_cumsum, scale, initial_state, h, A, do, dht,
                  cu_seqlens=None, chunk_size=64, dtype=np.float64):
    """Backward orchestrator, ``tops/ops/gla/chunk.py:815-977``.

    Pads like the forward (``:877-896``), recomputes g_cumsum / h / A when None, then
    dh scan, dv, dA, intra dq/dk, inter dq/dk/dg; unpads (``:956-965``) and sum-reduces dg to
    ``g_gamma``'s shape when only ``g_gamma`` was given (``:967-975``). Returns
    ``(dq, dk, dv, dg, dh0)``.
    """
    q, k, v, do = (_arr(x, dtype) for x in (q, k, v, do))
    B, T, H, K = q.shape
    C = chunk_size
    g_orig = g
    if g is None:
        g = np.broadcast_to(_arr(g_gamma, dtype), q.shape) if g_gamma is not None else \
            np.zeros_like(q)
    g = _arr(g, dtype)
    (q, k, v, g, do), cu, unpad = _pad_chunks([q, k, v, g, do], B, T, cu_seqlens, C)
    if g_cumsum is None:
        g_cumsum = chunk_local_cumsum(g, C, cu_seqlens=cu, dtype=dtype)
    if h is None:
        h, _ = chunk_fwd_h(k, v, g_cumsum, initial_state, False, cu, C, dtype=dtype)
    dh, dh0 = chunk_bwd_dh(q, g_cumsum, do, initial_state, dht, scale, cu, C, dtype=dtype)
    if A is None:
        A = chunk_gla_fwd_intra_gk(q, k, g_cumsum, scale, C, dtype=dtype)
    dv = chunk_gla_bwd_dv(k, g_cumsum, A, do, dh, C, dtype=dtype)
    dA = chunk_gla_bwd_dA(v, do, scale, C, dtype=dtype)
    dq, dk = chunk_gla_bwd_dqk_intra(q, k, g_cumsum, dA, C, dtype=dtype)
    dq, dk, dg = chunk_gla_bwd_dqkg(q, k, v, h, g_cumsum, do, dh, dq, dk, scale, C,
                                    dtype=dtype)
    dq, dk, dv, dg = (unpad(x) for x in (dq, dk, dv, dg))
    if g_orig is None and g_gamma is not None:
        gg = np.asarray(g_gamma)
        extra = dg.ndim - gg.ndim
        dg = dg.sum(axis=tuple(range(extra))) if extra > 0 else dg
        for ax in range(dg.ndim):
            if gg.shape[ax] == 1 and dg.shape[ax] != 1:
                dg = dg.sum(axis=ax, keepdims=True)
        dg = dg.reshape(gg.shape)
    return dq, dk, dv, dg, dh0
