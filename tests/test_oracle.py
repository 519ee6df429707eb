"""Pins the numpy oracle (CPU only).

Each check is independent of the oracle's own formulas: dense closed forms over (t, s)
pairs, brute-force loops, invariants, torch float64 autograd of a restatement written here,
and central finite differences. A dropped decay term, an off-by-one in the decay order, a
wrong reverse-cumsum direction or a transposed operand fails at least one of them.
"""

import numpy as np
import pytest
import torch

import oracle as orc

RNG = np.random.default_rng


def _logsig(x):
    return -np.logaddexp(0.0, -x)


def _inputs(B, T, H, K, V, seed, gate_div=1.0, h0=False, N=None):
    r = RNG(seed)
    q = r.standard_normal((B, T, H, K))
    k = r.standard_normal((B, T, H, K))
    v = r.standard_normal((B, T, H, V))
    g = _logsig(r.standard_normal((B, T, H, K))) / gate_div
    N = B if N is None else N
    s0 = r.standard_normal((N, H, K, V)) if h0 else None
    return q, k, v, g, s0


def _dense_recurrent(q, k, v, gk, gv, scale, h0):
    """Closed form of the gated recurrence for ONE sequence [T, H, *]: every (t, s) pair."""
    T, H, K = q.shape
    V = v.shape[-1]
    GK = np.cumsum(gk, 0) if gk is not None else np.zeros((T, H, K))
    GV = np.cumsum(gv, 0) if gv is not None else np.zeros((T, H, V))
    o = np.zeros((T, H, V))
    for t in range(T):
        acc = np.zeros((H, K, V))
        if h0 is not None:
            acc += np.exp(GK[t])[:, :, None] * np.exp(GV[t])[:, None, :] * h0
        for s in range(t + 1):
            dec = np.exp(GK[t] - GK[s])[:, :, None] * np.exp(GV[t] - GV[s])[:, None, :]
            acc += dec * k[s][:, :, None] * v[s][:, None, :]
        o[t] = np.einsum("hk,hkv->hv", q[t] * scale, acc)
        if t == T - 1:
            final = acc
    return o, final


# ---------------------------------------------------------------------------
# recurrent forms
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("h0", [False, True])
def test_naive_matches_dense_closed_form(h0):
    B, T, H, K, V = 2, 9, 2, 4, 3
    q, k, v, g, s0 = _inputs(B, T, H, K, V, 1, h0=h0)
    o, ht = orc.naive_recurrent_gla(q, k, v, g, initial_state=s0, output_final_state=True)
    for b in range(B):
        od, fd = _dense_recurrent(q[b], k[b], v[b], g[b], None, K ** -0.5,
                                  None if s0 is None else s0[b])
        np.testing.assert_allclose(o[b], od, rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(ht[b], fd, rtol=1e-12, atol=1e-12)


def test_naive_state_split_and_no_final_state():
    q, k, v, g, _ = _inputs(1, 12, 2, 4, 5, 2)
    o_full, s_full = orc.naive_recurrent_gla(q, k, v, g, output_final_state=True)
    o1, s1 = orc.naive_recurrent_gla(q[:, :5], k[:, :5], v[:, :5], g[:, :5],
                                     output_final_state=True)
    o2, s2 = orc.naive_recurrent_gla(q[:, 5:], k[:, 5:], v[:, 5:], g[:, 5:],
                                     initial_state=s1, output_final_state=True)
    np.testing.assert_allclose(np.concatenate([o1, o2], 1), o_full, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(s2, s_full, rtol=1e-12, atol=1e-12)
    assert orc.naive_recurrent_gla(q, k, v, g)[1] is None


def test_naive_varlen_equals_separate():
    q, k, v, g, s0 = _inputs(1, 11, 2, 3, 4, 3, h0=True, N=3)
    cu = [0, 4, 5, 11]
    o, ht = orc.naive_recurrent_gla(q, k, v, g, initial_state=s0, output_final_state=True,
                                    cu_seqlens=cu)
    for i in range(3):
        sl = slice(cu[i], cu[i + 1])
        oi, si = orc.naive_recurrent_gla(q[:, sl], k[:, sl], v[:, sl], g[:, sl],
                                         initial_state=s0[i:i + 1], output_final_state=True)
        np.testing.assert_allclose(o[:, sl], oi, rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(ht[i], si[0], rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("gate", ["gk", "gv", "gk+gv", "none"])
def test_fused_recurrent_matches_dense(gate):
    B, T, H, K, V = 1, 7, 2, 3, 4
    r = RNG(5)
    q, k = r.standard_normal((2, B, T, H, K))
    v = r.standard_normal((B, T, H, V))
    gk = _logsig(r.standard_normal((B, T, H, K))) if "gk" in gate else None
    gv = _logsig(r.standard_normal((B, T, H, V))) if "gv" in gate else None
    s0 = r.standard_normal((B, H, K, V))
    o, ht = orc.fused_recurrent_gla(q, k, v, gk=gk, gv=gv, scale=0.3, initial_state=s0,
                                    output_final_state=True)
    od, fd = _dense_recurrent(q[0], k[0], v[0], None if gk is None else gk[0],
                              None if gv is None else gv[0], 0.3, s0[0])
    np.testing.assert_allclose(o[0], od, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(ht[0], fd, rtol=1e-12, atol=1e-12)
    if gate == "gk":
        on, hn = orc.naive_recurrent_gla(q, k, v, gk, scale=0.3, initial_state=s0,
                                         output_final_state=True)
        np.testing.assert_allclose(o, on, rtol=1e-12, atol=1e-12)


def test_fused_recurrent_reverse_is_flipped_forward():
    r = RNG(6)
    q, k = r.standard_normal((2, 1, 10, 2, 3))
    v = r.standard_normal((1, 10, 2, 5))
    gk = _logsig(r.standard_normal((1, 10, 2, 3)))
    gv = _logsig(r.standard_normal((1, 10, 2, 5)))
    cu = [0, 4, 10]
    o_r, h_r = orc.fused_recurrent_gla(q, k, v, gk, gv, reverse=True, cu_seqlens=cu,
                                       output_final_state=True)
    for i in range(2):
        sl = slice(cu[i], cu[i + 1])
        f = lambda x: x[:, sl][:, ::-1]  # noqa: E731
        o_f, h_f = orc.fused_recurrent_gla(f(q), f(k), f(v), f(gk), f(gv),
                                           output_final_state=True)
        np.testing.assert_allclose(o_r[:, sl], o_f[:, ::-1], rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(h_r[i], h_f[0], rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------------------
# torch float64 restatement used for autograd pins
# ---------------------------------------------------------------------------


def _torch_recurrent(q, k, v, gk, gv, scale, h0, segs, reverse=False):
    """Independent autograd-friendly restatement (no in-place ops)."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    rows = [[None] * T for _ in range(B)]
    finals = []
    for b, i, bos, eos in segs:
        h = torch.zeros(H, K, V, dtype=q.dtype) if h0 is None else h0[i]
        ts = range(eos - 1, bos - 1, -1) if reverse else range(bos, eos)
        for t in ts:
            if gk is not None:
                h = h * torch.exp(gk[b, t])[:, :, None]
            if gv is not None:
                h = h * torch.exp(gv[b, t])[:, None, :]
            h = h + k[b, t][:, :, None] * v[b, t][:, None, :]
            rows[b][t] = torch.einsum("hk,hkv->hv", q[b, t] * scale, h)
        finals.append(h)
    zero = torch.zeros(H, V, dtype=q.dtype)
    o = torch.stack([torch.stack([r if r is not None else zero for r in row]) for row in rows])
    return o, torch.stack(finals)


def _autograd(q, k, v, gk, gv, scale, h0, do, dht, cu, reverse=False):
    tq, tk, tv = (torch.tensor(x, requires_grad=True) for x in (q, k, v))
    tgk = None if gk is None else torch.tensor(gk, requires_grad=True)
    tgv = None if gv is None else torch.tensor(gv, requires_grad=True)
    th0 = None if h0 is None else torch.tensor(h0, requires_grad=True)
    segs = orc.segments(q.shape[0], q.shape[1], cu)
    o, ht = _torch_recurrent(tq, tk, tv, tgk, tgv, scale, th0, segs, reverse)
    loss = (o * torch.tensor(do)).sum()
    if dht is not None:
        loss = loss + (ht * torch.tensor(dht)).sum()
    loss.backward()
    g = lambda t: None if t is None else t.grad.numpy()  # noqa: E731
    return g(tq), g(tk), g(tv), g(tgk), g(tgv), g(th0)


# ---------------------------------------------------------------------------
# chunked forward
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("C", [4, 8, 16, 32])
@pytest.mark.parametrize("reverse", [False, True])
def test_cumsum_closed_form(C, reverse):
    r = RNG(7)
    B, T, H, S = 2, 4 * C, 3, 5
    g = r.standard_normal((B, T, H, S))
    out = orc.chunk_local_cumsum(g, C, reverse=reverse, scale=0.5)
    gc = g.reshape(B, T // C, C, H, S)
    ref = np.flip(np.cumsum(np.flip(gc, 2), 2), 2) if reverse else np.cumsum(gc, 2)
    np.testing.assert_allclose(out, 0.5 * ref.reshape(B, T, H, S), rtol=1e-13, atol=1e-13)
    first = out.reshape(B, T // C, C, H, S)[:, :, -1 if reverse else 0]
    np.testing.assert_allclose(first, 0.5 * gc[:, :, -1 if reverse else 0], rtol=1e-13)
    hf = orc.chunk_local_cumsum(g.transpose(0, 2, 1, 3), C, reverse=reverse, scale=0.5,
                                head_first=True)
    np.testing.assert_allclose(hf.transpose(0, 2, 1, 3), out, rtol=1e-13)


def test_cumsum_varlen_unaligned():
    r = RNG(8)
    g = r.standard_normal((1, 23, 2, 3))
    cu = [0, 7, 20, 23]
    out = orc.chunk_local_cumsum(g, 4, cu_seqlens=cu)
    for i in range(3):
        for c0 in range(cu[i], cu[i + 1], 4):
            c1 = min(c0 + 4, cu[i + 1])
            np.testing.assert_allclose(out[:, c0:c1], np.cumsum(g[:, c0:c1], 1), rtol=1e-13)


def test_fwd_h_invariants():
    B, T, H, K, V, C = 2, 64, 2, 8, 16, 16
    q, k, v, g, s0 = _inputs(B, T, H, K, V, 9, h0=True)
    gc = orc.chunk_local_cumsum(g, C)
    h, ht = orc.chunk_fwd_h(k, v, gc, s0, True, chunk_size=C)
    np.testing.assert_allclose(h[:, 0], s0, rtol=1e-13)
    _, hn = orc.naive_recurrent_gla(q, k, v, g, initial_state=s0, output_final_state=True)
    np.testing.assert_allclose(ht, hn, rtol=1e-10, atol=1e-10)
    # state at chunk n equals the naive state after n*C tokens
    for n in range(1, T // C):
        _, hs = orc.naive_recurrent_gla(q[:, :n * C], k[:, :n * C], v[:, :n * C],
                                        g[:, :n * C], initial_state=s0,
                                        output_final_state=True)
        np.testing.assert_allclose(h[:, n], hs, rtol=1e-10, atol=1e-10)
    # zero padding (k = v = g = 0) leaves the state unchanged
    pad = lambda x: np.pad(x, ((0, 0), (0, C), (0, 0), (0, 0)))  # noqa: E731
    h2, ht2 = orc.chunk_fwd_h(pad(k), pad(v), orc.chunk_local_cumsum(pad(g), C), s0, True,
                              chunk_size=C)
    np.testing.assert_allclose(ht2, ht, rtol=1e-13)
    np.testing.assert_allclose(h2[:, :T // C], h, rtol=1e-13)
    _, ht_off = orc.chunk_fwd_h(k, v, gc, s0, False, chunk_size=C)
    assert not ht_off.any()


def test_intra_bruteforce():
    B, T, H, K, C = 1, 32, 2, 4, 16
    q, k, _, g, _ = _inputs(B, T, H, K, 1, 10)
    gc = orc.chunk_local_cumsum(g, C)
    A = orc.chunk_gla_fwd_intra_gk(q, k, gc, 0.7, C)
    ref = np.zeros_like(A)
    for t in range(T):
        n0 = (t // C) * C
        for j in range(C):
            for h in range(H):
                ref[0, t, h, j] = 0.7 * sum(q[0, t, h, d] * k[0, n0 + j, h, d] *
                                            np.exp(gc[0, t, h, d] - gc[0, n0 + j, h, d])
                                            for d in range(K))
    np.testing.assert_allclose(A, ref, rtol=1e-11, atol=1e-11)


CHUNK_CASES = [
    dict(B=2, T=32, H=2, K=8, V=16, C=16, seed=42),
    dict(B=2, T=32, H=2, K=8, V=16, C=16, seed=13, h0=True),
    dict(B=1, T=64, H=2, K=16, V=8, C=64, seed=7, h0=True),
    dict(B=2, T=37, H=2, K=8, V=4, C=16, seed=40),
    dict(B=1, T=50, H=1, K=4, V=8, C=8, seed=41, scale=0.1, h0=True),
    dict(B=1, T=3, H=2, K=4, V=4, C=16, seed=31),
    dict(B=1, T=40, H=2, K=4, V=8, C=4, seed=503),
    dict(B=1, T=48, H=2, K=8, V=8, C=16, seed=11, cu=[0, 16, 48], h0=True),
    dict(B=1, T=50, H=2, K=4, V=8, C=16, seed=402, cu=[0, 13, 37, 50], h0=True),
    dict(B=1, T=70, H=1, K=4, V=4, C=32, seed=9, cu=[0, 3, 70]),
]


def _cid(c):
    return "-".join(f"{k}{v}" for k, v in c.items() if k != "cu") + ("-varlen" if "cu" in c
                                                                    else "")


@pytest.mark.parametrize("cfg", CHUNK_CASES, ids=[_cid(c) for c in CHUNK_CASES])
def test_chunk_gla_equals_naive(cfg):
    cu = cfg.get("cu")
    N = len(cu) - 1 if cu else cfg["B"]
    q, k, v, g, s0 = _inputs(cfg["B"], cfg["T"], cfg["H"], cfg["K"], cfg["V"], cfg["seed"],
                             h0=cfg.get("h0", False), N=N)
    sc = cfg.get("scale")
    o, ht = orc.chunk_gla(q, k, v, g, scale=sc, initial_state=s0, output_final_state=True,
                          cu_seqlens=cu, chunk_size=cfg["C"])
    on, hn = orc.naive_recurrent_gla(q, k, v, g, scale=sc, initial_state=s0,
                                     output_final_state=True, cu_seqlens=cu)
    np.testing.assert_allclose(o, on, rtol=1e-9, atol=1e-9)
    np.testing.assert_allclose(ht, hn, rtol=1e-9, atol=1e-9)
    assert orc.chunk_gla(q, k, v, g, cu_seqlens=cu, chunk_size=cfg["C"])[1] is None


def test_chunk_gla_g_gamma_equals_broadcast():
    q, k, v, _, _ = _inputs(1, 32, 2, 4, 4, 12)
    gg = -np.abs(RNG(12).standard_normal((2, 1))) * 0.1
    o1, _ = orc.chunk_gla(q, k, v, g_gamma=gg, chunk_size=16)
    o2, _ = orc.chunk_gla(q, k, v, g=np.broadcast_to(gg, q.shape), chunk_size=16)
    np.testing.assert_allclose(o1, o2, rtol=1e-13)


# ---------------------------------------------------------------------------
# chunked backward vs autograd
# ---------------------------------------------------------------------------

BWD_CASES = [
    dict(B=2, T=32, H=2, K=8, V=16, C=16, seed=42),
    dict(B=2, T=32, H=2, K=8, V=16, C=16, seed=15, h0=True, dht=True),
    dict(B=1, T=64, H=1, K=16, V=8, C=64, seed=7, h0=True),
    dict(B=1, T=37, H=2, K=4, V=8, C=8, seed=40, dht=True),
    dict(B=1, T=40, H=1, K=4, V=4, C=4, seed=503, scale=0.2, h0=True, dht=True),
    dict(B=1, T=45, H=2, K=4, V=8, C=16, seed=604, cu=[0, 20, 45], h0=True, dht=True),
    dict(B=1, T=48, H=1, K=4, V=4, C=32, seed=20, cu=[0, 16, 48], h0=True),
]


@pytest.mark.parametrize("cfg", BWD_CASES, ids=[_cid(c) for c in BWD_CASES])
def test_chunk_bwd_equals_autograd(cfg):
    cu = cfg.get("cu")
    N = len(cu) - 1 if cu else cfg["B"]
    B, T, H, K, V = (cfg[x] for x in "BTHKV")
    q, k, v, g, s0 = _inputs(B, T, H, K, V, cfg["seed"], h0=cfg.get("h0", False), N=N)
    r = RNG(cfg["seed"] + 1)
    do = r.standard_normal((B, T, H, V))
    dht = r.standard_normal((N, H, K, V)) if cfg.get("dht") else None
    sc = cfg.get("scale", K ** -0.5)
    dq, dk, dv, dg, dh0 = orc.chunk_gla_bwd(q, k, v, g, None, None, sc, s0, None, None, do,
                                            dht, cu_seqlens=cu, chunk_size=cfg["C"])
    gq, gk_, gv, gg, _, gh0 = _autograd(q, k, v, g, None, sc, s0, do, dht, cu)
    for name, a, b in [("dq", dq, gq), ("dk", dk, gk_), ("dv", dv, gv), ("dg", dg, gg)]:
        np.testing.assert_allclose(a, b, rtol=1e-8, atol=1e-8, err_msg=name)
    if s0 is not None:
        np.testing.assert_allclose(dh0, gh0, rtol=1e-8, atol=1e-8)
    if s0 is None and dht is None:
        assert dh0 is None


def test_chunk_bwd_finite_differences():
    """Central differences of the oracle's own forward (no torch)."""
    B, T, H, K, V, C = 1, 5, 1, 3, 2, 2
    q, k, v, g, s0 = _inputs(B, T, H, K, V, 77, h0=True)
    r = RNG(78)
    do = r.standard_normal((B, T, H, V))
    dht = r.standard_normal((1, H, K, V))

    def loss(q_, k_, v_, g_, s_):
        o, ht = orc.chunk_gla(q_, k_, v_, g_, initial_state=s_, output_final_state=True,
                              chunk_size=C)
        return (o * do).sum() + (ht * dht).sum()

    grads = orc.chunk_gla_bwd(q, k, v, g, None, None, K ** -0.5, s0, None, None, do, dht,
                              chunk_size=C)
    args = [q, k, v, g, s0]
    order = [0, 1, 2, 3, 4]  # dq, dk, dv, dg, dh0
    eps = 1e-6
    for ai, gi in zip(range(5), order):
        x = args[ai]
        num = np.zeros_like(x)
        for idx in np.ndindex(x.shape):
            xp, xm = x.copy(), x.copy()
            xp[idx] += eps
            xm[idx] -= eps
            a_p = list(args)
            a_m = list(args)
            a_p[ai], a_m[ai] = xp, xm
            num[idx] = (loss(*a_p) - loss(*a_m)) / (2 * eps)
        np.testing.assert_allclose(grads[gi], num, rtol=1e-6, atol=1e-6)


def test_bwd_subfunctions_compose():
    """dh from chunk_bwd_dh equals autograd's gradient of the chunk-end states."""
    B, T, H, K, V, C = 1, 32, 1, 4, 4, 8
    q, k, v, g, s0 = _inputs(B, T, H, K, V, 21, h0=True)
    do = RNG(22).standard_normal((B, T, H, V))
    gc = orc.chunk_local_cumsum(g, C)
    dh, dh0 = orc.chunk_bwd_dh(q, gc, do, s0, None, K ** -0.5, chunk_size=C)
    # dh[n] = dL/d(state after chunk n), with loss restricted to outputs of later chunks
    for n in range(T // C):
        t1 = (n + 1) * C
        if t1 >= T:
            assert not dh[0, n].any()
            continue
        _, s_end = orc.naive_recurrent_gla(q[:, :t1], k[:, :t1], v[:, :t1], g[:, :t1],
                                           initial_state=s0, output_final_state=True)
        _, _, _, _, _, gs = _autograd(q[:, t1:], k[:, t1:], v[:, t1:], g[:, t1:], None,
                                      K ** -0.5, s_end, do[:, t1:], None, None)
        np.testing.assert_allclose(dh[0, n], gs[0], rtol=1e-9, atol=1e-9)


@pytest.mark.parametrize("gate", ["gk", "gk+gv", "gv"])
@pytest.mark.parametrize("reverse", [False, True])
def test_fused_recurrent_bwd_equals_autograd(gate, reverse):
    r = RNG(30)
    B, T, H, K, V = 1, 9, 2, 3, 4
    q, k = r.standard_normal((2, B, T, H, K))
    v = r.standard_normal((B, T, H, V))
    gk = _logsig(r.standard_normal((B, T, H, K))) if "gk" in gate else None
    gv = _logsig(r.standard_normal((B, T, H, V))) if "gv" in gate else None
    cu = [0, 4, 9]
    s0 = r.standard_normal((2, H, K, V))
    do = r.standard_normal((B, T, H, V))
    dht = r.standard_normal((2, H, K, V))
    dq, dk, dv, dgk, dgv, dh0 = orc.fused_recurrent_gla_bwd(
        q, k, v, gk, gv, None, do, dht, 0.5, s0, reverse=reverse, cu_seqlens=cu)
    a = _autograd(q, k, v, gk, gv, 0.5, s0, do, dht, cu, reverse=reverse)
    for name, x, y in zip(["dq", "dk", "dv", "dgk", "dgv", "dh0"],
                          [dq, dk, dv, dgk, dgv, dh0], a):
        if x is None:
            assert y is None, name
            continue
        np.testing.assert_allclose(x, y, rtol=1e-9, atol=1e-9, err_msg=name)


# ---------------------------------------------------------------------------
# the layer restatement (oracle/layer.py)
# ---------------------------------------------------------------------------


def test_layer_recurrence_matches_numpy_naive():
    """The torch recurrence of the layer oracle equals the pinned numpy naive recurrence."""
    import torch

    from oracle import layer as L

    r = np.random.default_rng(31)
    B, T, H, K, V = 2, 9, 2, 4, 3
    q, k = r.standard_normal((2, B, T, H, K))
    v = r.standard_normal((B, T, H, V))
    g = -np.logaddexp(0.0, -r.standard_normal((B, T, H, K)))
    s0 = r.standard_normal((B, H, K, V))
    t = lambda x: torch.tensor(x, dtype=torch.float64)  # noqa: E731
    o, ht = L.recurrence(t(q), t(k), t(v), t(g), 0.5, t(s0))
    on, hn = orc.naive_recurrent_gla(q, k, v, g, scale=0.5, initial_state=s0,
                                     output_final_state=True)
    np.testing.assert_allclose(o.numpy(), on, atol=1e-12)
    np.testing.assert_allclose(ht.numpy(), hn, atol=1e-12)
    cu = [0, 4, 9]
    o2, h2 = L.recurrence(t(q[:1]), t(k[:1]), t(v[:1]), t(g[:1]), 0.5, t(s0), cu)
    on2, hn2 = orc.naive_recurrent_gla(q[:1], k[:1], v[:1], g[:1], scale=0.5, initial_state=s0,
                                       output_final_state=True, cu_seqlens=cu)
    np.testing.assert_allclose(o2.numpy(), on2, atol=1e-12)
    np.testing.assert_allclose(h2.numpy(), hn2, atol=1e-12)


def test_layer_norm_gate_and_conv_closed_forms():
    import torch
    import torch.nn.functional as F

    from oracle import layer as L

    g = torch.Generator().manual_seed(3)
    x = torch.randn(5, 16, generator=g, dtype=torch.float64)
    y = L.rms_norm(x, eps=0.0)
    np.testing.assert_allclose((y * y).mean(-1).numpy(), 1.0, atol=1e-12)   # unit RMS rows
    gate = torch.randn(5, 16, generator=g, dtype=torch.float64)
    np.testing.assert_allclose(L.rms_norm(x, None, 0.0, gate).numpy(),
                               (y * gate * torch.sigmoid(gate)).numpy(), atol=1e-12)
    # log_sigmoid gate: log(1/(1+e^-x)) / n, clipped
    z = torch.linspace(-30, 30, 61, dtype=torch.float64)
    np.testing.assert_allclose(L.gate_logsigmoid(z, 16).numpy(),
                               (-np.log1p(np.exp(-z.numpy())) / 16), atol=1e-12)
    assert float(L.gate_logsigmoid(z, 16, -0.5).min()) == -0.5
    # causal depthwise conv == brute-force taps over the zero-padded past
    W, D, T = 3, 4, 7
    xx = torch.randn(2, T, D, generator=g, dtype=torch.float64)
    w = torch.randn(D, 1, W, generator=g, dtype=torch.float64)
    b = torch.randn(D, generator=g, dtype=torch.float64)
    yy = L.short_conv(xx, w, b, activation=None)
    ref = torch.zeros_like(xx)
    for t in range(T):
        for j in range(W):
            ts = t - W + 1 + j
            if ts >= 0:
                ref[:, t] += w[:, 0, j] * xx[:, ts]
    ref += b
    np.testing.assert_allclose(yy.numpy(), ref.numpy(), atol=1e-12)
    # varlen restarts at every sequence
    yv = L.short_conv(xx[:1], w, b, activation=None, cu_seqlens=[0, 3, 7])
    np.testing.assert_allclose(yv[:, 3:].numpy(), L.short_conv(xx[:1, 3:], w, b, None).numpy(),
                               atol=1e-12)
    assert torch.allclose(L.short_conv(xx, w, b, "silu"), F.silu(yy))


# ---------------------------------------------------------------------------
# simple GLA (scalar gates)
# ---------------------------------------------------------------------------

SG = orc.simple_gla


def _sg_inputs(B, T, H, K, V, seed, h0=False, N=None):
    r = RNG(seed)
    q = r.standard_normal((B, T, H, K))
    k = r.standard_normal((B, T, H, K))
    v = r.standard_normal((B, T, H, V))
    g_raw = _logsig(r.standard_normal((B, T, H))) / 4      # per-token scalar gates
    gamma = -np.abs(r.standard_normal(H)) * 0.3              # per-head constant
    N = B if N is None else N
    s0 = r.standard_normal((N, H, K, V)) if h0 else None
    return q, k, v, g_raw, gamma, s0


def test_simple_naive_is_broadcast_gla_and_linear_attention():
    B, T, H, K, V = 2, 11, 3, 4, 5
    q, k, v, g_raw, gamma, s0 = _sg_inputs(B, T, H, K, V, 1, h0=True)
    gk = np.repeat(g_raw[..., None], K, -1) + gamma[None, None, :, None]
    o, S = SG.simple_gla_naive(q, k, v, g=np.repeat(g_raw[..., None], K, -1),
                               g_gamma=np.broadcast_to(gamma[None, None, :, None], q.shape),
                               initial_state=s0, output_final_state=True)
    o2, S2 = orc.naive_recurrent_gla(q, k, v, gk, None, s0, True)
    np.testing.assert_allclose(o, o2, rtol=1e-13, atol=1e-13)
    np.testing.assert_allclose(S, S2, rtol=1e-13, atol=1e-13)
    # no gate, no h0: causal linear attention, every (t, s) pair
    o0, _ = SG.simple_gla_naive(q, k, v, scale=0.3)
    ref = np.zeros_like(o0)
    for b in range(B):
        for t in range(T):
            for s in range(t + 1):
                ref[b, t] += 0.3 * np.einsum("hk,hk->h", q[b, t], k[b, s])[:, None] * v[b, s]
    np.testing.assert_allclose(o0, ref, rtol=1e-12, atol=1e-12)


def test_simple_intra_bruteforce():
    B, T, H, K, C = 1, 16, 2, 3, 8
    q, k, _, _, gamma, _ = _sg_inputs(B, T, H, K, 1, 2)
    A = SG.chunk_simple_gla_fwd_intra(q, k, gamma, 0.5, C)
    for n in range(T // C):
        for i in range(C):
            for j in range(C):
                for h in range(H):
                    a = 0.5 * np.dot(q[0, n * C + i, h], k[0, n * C + j, h]) * \
                        np.exp(gamma[h] * (i - j))
                    assert abs(A[0, n * C + i, h, j] - a) < 1e-12


SG_CASES = [
    dict(B=2, T=64, H=2, K=4, V=6, C=16, gate="g_gamma"),
    dict(B=1, T=96, H=3, K=5, V=4, C=32, gate="g"),
    dict(B=2, T=64, H=2, K=4, V=4, C=64, gate="both", h0=True),
    dict(B=1, T=48, H=2, K=3, V=5, C=16, gate="none", h0=True, scale=0.2),
    dict(B=2, T=64, H=2, K=4, V=4, C=16, gate="both", cu=[0, 32, 80, 128], h0=True),
]


@pytest.mark.parametrize("cfg", SG_CASES, ids=[str(i) for i in range(len(SG_CASES))])
def test_chunk_simple_gla_equals_naive(cfg):
    B, T, H, K, V, C = (cfg[x] for x in ("B", "T", "H", "K", "V", "C"))
    cu = cfg.get("cu")
    N = len(cu) - 1 if cu else B
    q, k, v, g_raw, gamma, s0 = _sg_inputs(B, T, H, K, V, 3, cfg.get("h0", False), N)
    gate = cfg["gate"]
    use_g = gate in ("g", "both")
    use_gamma = gate in ("g_gamma", "both")
    g_cum = SG.scalar_cumsum(g_raw.reshape(1, B * T, H) if cu else g_raw, C, cu)
    g_cum = g_cum.reshape(B, T, H)
    sc = cfg.get("scale")
    o, ht = SG.chunk_simple_gla_fwd(q, k, v, g=g_cum if use_g else None,
                                    g_gamma=gamma if use_gamma else None, scale=sc, h0=s0,
                                    use_ht=True, cu_seqlens=cu, chunk_size=C)
    gk = np.zeros((B, T, H, K))
    if use_g:
        gk += g_raw[..., None]
    if use_gamma:
        gk += gamma[None, None, :, None]
    flat = (lambda x: x.reshape(1, B * T, *x.shape[2:])) if cu else (lambda x: x)
    o2, S2 = orc.naive_recurrent_gla(flat(q), flat(k), flat(v), flat(gk), sc, s0, True, cu)
    np.testing.assert_allclose(o, o2.reshape(o.shape), rtol=1e-11, atol=1e-11)
    np.testing.assert_allclose(ht, S2, rtol=1e-11, atol=1e-11)


def test_chunk_simple_gla_fwd_ref_equals_naive_with_padding():
    """Odd T: the reference pads with zero rows whose gate still decays the final state."""
    B, T, H, K, V, C = 2, 40, 2, 4, 3, 16
    q, k, v, _, gamma, s0 = _sg_inputs(B, T, H, K, V, 4, h0=True)
    ht, o = SG.chunk_simple_gla_fwd_ref(q, k, v, gamma, 0.4, s0, True, C)
    gk = np.broadcast_to(gamma[None, None, :, None], (B, T, H, K))
    o2, S2 = orc.naive_recurrent_gla(q, k, v, gk, 0.4, s0, True)
    np.testing.assert_allclose(o, o2, rtol=1e-11, atol=1e-11)
    Tp = 48   # the padded rows decay the state by gamma per row
    np.testing.assert_allclose(ht, S2 * np.exp(gamma * (Tp - T))[None, :, None, None],
                               rtol=1e-11, atol=1e-11)


@pytest.mark.parametrize("h0,dht", [(False, False), (True, False), (True, True)])
def test_chunk_simple_gla_bwd_equals_autograd(h0, dht):
    B, T, H, K, V, C = 2, 48, 2, 4, 3, 16
    q, k, v, _, gamma, s0 = _sg_inputs(B, T, H, K, V, 5, h0=h0)
    r = RNG(6)
    do = r.standard_normal((B, T, H, V))
    dh = r.standard_normal((B, H, K, V)) if dht else None
    dq, dk, dv, dh0 = SG.chunk_simple_gla_bwd(q, k, v, gamma, 0.3, s0, do, dh, C)
    gk = np.ascontiguousarray(np.broadcast_to(gamma[None, None, :, None], (B, T, H, K)))
    gq, gk_, gv, _, _, gh0 = _autograd(q, k, v, gk, None, 0.3, s0, do, dh, None)
    for name, a, b in [("dq", dq, gq), ("dk", dk, gk_), ("dv", dv, gv)]:
        np.testing.assert_allclose(a, b, rtol=1e-9, atol=1e-9, err_msg=name)
    if h0:
        np.testing.assert_allclose(dh0, gh0, rtol=1e-9, atol=1e-9)
    else:
        assert dh0 is None
