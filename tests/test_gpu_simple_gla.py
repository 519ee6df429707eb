"""GPU parity: simple GLA (scalar gates) vs the numpy oracle (``oracle/simple_gla.py``).

Cases follow the reference's tables: ``tests/ops/simple_gla/test_chunk_simple_gla.py:45-89``
(forward: K, V in {128, 256}, gate none / g_gamma, h0, custom scale, long sequences, many
heads), ``test_pallas_simple_gla_bwd.py:20-45`` (backward with g_gamma, chunk sizes 16 / 32 /
64, h0) and ``test_simple_gla.py:50-108`` (the naive recurrence on small dims, odd T, g /
g_gamma / both), plus per-token scalar gates given as their chunk-local cumsum, varlen,
dht, strong decays (a 64-row chunk decaying by e^-220), and chunk_gla with a per-head
g_gamma. g_gamma = logsigmoid(randn(H)) as in the reference's forward test. bf16 inputs
run the scalar-gate full-head kernels; float32 inputs (and shapes off the full-head path)
the recurrent kernel on the broadcast gate. Tolerances: float32 max-abs <= 1e-4 x
max(1, max|ref|); bfloat16 max-abs / max|ref| <= 2e-2.
"""

import numpy as np
import pytest
import torch

import oracle as orc
from gla_cases import check, logsigmoid, round_bf16, to_dev, to_np

pytestmark = pytest.mark.gpu

SG = orc.simple_gla


def _sgla():
    import tops.ops.simple_gla as S

    return S


def _tol(ref):
    return 1e-4 * max(1.0, float(np.abs(ref).max()))


def _chk(name, got, ref, dtype):
    if dtype == "f32":
        check(name, to_np(got), ref, "f32", atol=_tol(ref))
    else:
        check(name, to_np(got), ref, "bf16")


def _inputs(cfg, dtype):
    B, T, H, K, V = (cfg[x] for x in "BTHKV")
    r = np.random.default_rng(cfg["seed"])
    q = r.standard_normal((B, T, H, K))
    k = r.standard_normal((B, T, H, K))
    v = r.standard_normal((B, T, H, V))
    gamma = logsigmoid(r.standard_normal(H))
    if cfg.get("strong"):   # e^-3.5 per step on the first head
        gamma[0] = -3.5
    g_raw = logsigmoid(r.standard_normal((B, T, H))) / 4
    N = B
    h0 = r.standard_normal((N, H, K, V)) if cfg.get("h0") else None
    do = r.standard_normal((B, T, H, V))
    dht = r.standard_normal((N, H, K, V)) if cfg.get("dht") else None
    if dtype == "bf16":
        q, k, v, gamma, h0 = (None if x is None else round_bf16(x) for x in (q, k, v, gamma, h0))
        do = round_bf16(do)
    return q, k, v, gamma, g_raw, h0, do, dht


FWD_CASES = [
    dict(B=2, T=64, H=4, K=128, V=128, seed=42),
    dict(B=2, T=128, H=4, K=128, V=128, seed=13),
    dict(B=1, T=256, H=2, K=128, V=128, seed=7, h0=True),
    dict(B=2, T=64, H=1, K=128, V=128, seed=10),
    dict(B=2, T=64, H=4, K=128, V=256, seed=20, gate="g_gamma"),
    dict(B=2, T=64, H=4, K=256, V=128, seed=21, gate="g_gamma"),
    dict(B=8, T=64, H=4, K=128, V=128, seed=50),
    dict(B=1, T=128, H=16, K=128, V=128, seed=60, gate="g_gamma"),
    dict(B=2, T=64, H=4, K=128, V=128, seed=152, gate="g_gamma", h0=True),
    dict(B=2, T=64, H=4, K=128, V=128, seed=200, scale=0.1, h0=True),
    dict(B=1, T=512, H=2, K=128, V=128, seed=303, gate="g_gamma", h0=True),
    dict(B=2, T=256, H=4, K=128, V=128, seed=361, gate="g_gamma"),
    dict(B=2, T=4096, H=16, K=128, V=128, seed=151, gate="g_gamma", h0=True),
    # per-token scalar gates (chunk-local cumsum), alone and with g_gamma; varlen
    dict(B=2, T=256, H=2, K=128, V=128, seed=500, gate="g", C=64),
    dict(B=1, T=256, H=2, K=128, V=256, seed=501, gate="both", C=32, h0=True),
    dict(B=2, T=2048, H=2, K=128, V=128, seed=502, gate="both", C=64, h0=True),
    dict(B=3, T=128, H=2, K=128, V=128, seed=503, gate="both", C=64, h0=True,
         cu=[0, 64, 256, 384]),
    dict(B=2, T=512, H=2, K=128, V=128, seed=504, gate="both", C=64, h0=True, strong=True),
    dict(B=1, T=256, H=2, K=256, V=128, seed=505, gate="g_gamma", h0=True, strong=True),
]


def _cid(c):
    return "-".join(f"{k}{v}" for k, v in c.items() if k != "seed").replace(" ", "")


def _gates_for(cfg, gamma, g_raw):
    gate = cfg.get("gate", "none")
    B, T, H = cfg["B"], cfg["T"], cfg["H"]
    C = cfg.get("C", 64)
    cu = cfg.get("cu")
    g_cum = None
    if gate in ("g", "both"):
        g_cum = SG.scalar_cumsum(g_raw.reshape(1, B * T, H) if cu else g_raw, C, cu)
        g_cum = g_cum.reshape(B, T, H)
    return g_cum, (gamma if gate in ("g_gamma", "both") else None)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("cfg", FWD_CASES, ids=[_cid(c) for c in FWD_CASES])
def test_chunk_simple_gla_fwd(cfg, dtype):
    S = _sgla()
    if dtype == "f32" and cfg["T"] * cfg["H"] * cfg["B"] > 20000:
        pytest.skip("float32 runs the per-element kernels: the bf16 case covers the size")
    q, k, v, gamma, g_raw, h0, _, _ = _inputs(cfg, dtype)
    g_cum, gg = _gates_for(cfg, gamma, g_raw)
    C = cfg.get("C", 64)
    cu = cfg.get("cu")
    sc = cfg.get("scale")
    o_ref, ht_ref = SG.chunk_simple_gla_fwd(q, k, v, g=g_cum, g_gamma=gg, scale=sc, h0=h0,
                                            use_ht=True, cu_seqlens=cu, chunk_size=C)
    d = lambda x: to_dev(x, dtype)  # noqa: E731
    o, ht = S.chunk_simple_gla_fwd(
        d(q), d(k), d(v), g=None if g_cum is None else to_dev(g_cum, "f32"),
        g_gamma=None if gg is None else d(gg), scale=sc,
        h0=None if h0 is None else to_dev(h0, "f32"), use_ht=True,
        cu_seqlens=None if cu is None else torch.tensor(cu, dtype=torch.int32), chunk_size=C)
    assert o.dtype == d(q).dtype and ht.dtype == torch.float32
    _chk("o", o, o_ref, dtype)
    _chk("ht", ht, ht_ref, dtype)
    o2, ht2 = S.chunk_simple_gla_fwd(d(q), d(k), d(v), g_gamma=None if gg is None else d(gg),
                                     g=None if g_cum is None else to_dev(g_cum, "f32"),
                                     scale=sc, use_ht=False, chunk_size=C,
                                     h0=None if h0 is None else to_dev(h0, "f32"),
                                     cu_seqlens=None if cu is None else
                                     torch.tensor(cu, dtype=torch.int32))
    assert ht2 is None
    assert torch.equal(o2, o)


BWD_CASES = [
    dict(B=2, T=64, H=4, K=128, V=128, seed=42, C=16),
    dict(B=1, T=128, H=2, K=128, V=128, seed=7, C=16),
    dict(B=2, T=64, H=4, K=128, V=128, seed=13, C=16, h0=True),
    dict(B=2, T=64, H=1, K=128, V=128, seed=10, C=16),
    dict(B=1, T=256, H=2, K=128, V=128, seed=300, C=16),
    dict(B=4, T=64, H=8, K=128, V=128, seed=99, C=16),
    dict(B=2, T=128, H=4, K=128, V=128, seed=502, C=32),
    dict(B=2, T=128, H=4, K=128, V=128, seed=503, C=64),
    dict(B=2, T=128, H=2, K=128, V=128, seed=504, C=64, h0=True, dht=True),
    dict(B=1, T=2048, H=4, K=128, V=128, seed=505, C=64, h0=True, dht=True),
    dict(B=2, T=64, H=2, K=128, V=256, seed=506, C=64, h0=True),   # recurrent kernel
    dict(B=2, T=1024, H=2, K=128, V=128, seed=508, C=64, h0=True, dht=True, strong=True),
]


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("cfg", BWD_CASES, ids=[_cid(c) for c in BWD_CASES])
def test_chunk_simple_gla_bwd(cfg, dtype):
    S = _sgla()
    q, k, v, gamma, _, h0, do, dht = _inputs(cfg, dtype)
    if cfg["seed"] % 2:   # the reference's -|rand| * 0.5 style of decay, on odd seeds
        gamma = -np.abs(gamma) * 0.5
        gamma = round_bf16(gamma) if dtype == "bf16" else gamma
    C = cfg["C"]
    sc = cfg["K"] ** -0.5
    dq_r, dk_r, dv_r, dh0_r = SG.chunk_simple_gla_bwd(q, k, v, gamma, sc, h0, do, dht, C)
    d = lambda x: to_dev(x, dtype)  # noqa: E731
    dq, dk, dv, dh0 = S.chunk_simple_gla_bwd(
        d(q), d(k), d(v), d(gamma), sc, None if h0 is None else to_dev(h0, "f32"), d(do),
        None if dht is None else to_dev(dht, "f32"), chunk_size=C)
    for name, a, b in [("dq", dq, dq_r), ("dk", dk, dk_r), ("dv", dv, dv_r)]:
        assert a.dtype == d(q).dtype
        _chk(name, a, b, dtype)
    if h0 is None:
        assert dh0 is None
    else:
        _chk("dh0", dh0, dh0_r, dtype)


NAIVE_CASES = [
    dict(B=2, T=32, H=4, K=32, V=64, seed=42),
    dict(B=2, T=32, H=4, K=32, V=64, seed=13, h0=True),
    dict(B=2, T=32, H=4, K=16, V=128, seed=20, gate="g_gamma"),
    dict(B=1, T=1, H=2, K=32, V=64, seed=30, gate="both"),
    dict(B=2, T=37, H=4, K=16, V=32, seed=40, gate="both", h0=True),
    dict(B=1, T=128, H=2, K=64, V=128, seed=152, gate="g_gamma"),
    dict(B=2, T=32, H=2, K=8, V=16, seed=71, gate="g", h0=True, scale=0.1),
    dict(B=3, T=32, H=2, K=32, V=64, seed=72, gate="both", h0=True, cu=[0, 10, 60, 96]),
]


@pytest.mark.parametrize("cfg", NAIVE_CASES, ids=[_cid(c) for c in NAIVE_CASES])
def test_simple_gla_naive(cfg):
    S = _sgla()
    B, T, H, K = cfg["B"], cfg["T"], cfg["H"], cfg["K"]
    q, k, v, gamma, g_raw, h0, _, _ = _inputs(cfg, "f32")
    gate = cfg.get("gate", "g")
    g4 = np.repeat(g_raw[..., None], K, -1) if gate in ("g", "both") else None
    gg4 = (np.broadcast_to(gamma[None, None, :, None], (1, 1, H, 1))
           if gate in ("g_gamma", "both") else None)
    cu = cfg.get("cu")
    sc = cfg.get("scale")
    flat = (lambda x: None if x is None else x.reshape(1, B * T, *x.shape[2:])) if cu else \
        (lambda x: x)
    o_ref, s_ref = SG.simple_gla_naive(flat(q), flat(k), flat(v), flat(g4), gg4, sc, h0, True,
                                       cu)
    d = lambda x: None if x is None else to_dev(x, "f32")  # noqa: E731
    o, s = S.simple_gla_naive(d(q), d(k), d(v), g=d(g4), g_gamma=d(gg4), scale=sc,
                              initial_state=d(h0), output_final_state=True,
                              cu_seqlens_cpu=cu)
    assert o.dtype == torch.float32
    _chk("o", o, o_ref.reshape(B, T, H, -1), "f32")
    _chk("S", s, s_ref, "f32")


def test_simple_refs():
    """fwd_intra_ref, fwd_o_ref and fwd_ref (odd T: padded rows decay the final state)."""
    S = _sgla()
    cfg = dict(B=2, T=128, H=2, K=128, V=128, seed=9, h0=True)
    q, k, v, gamma, _, h0, _, _ = _inputs(cfg, "f32")
    d = lambda x: to_dev(x, "f32")  # noqa: E731
    C = 32
    A = S.chunk_simple_gla_fwd_intra_ref(d(q), d(k), d(gamma), 0.3, chunk_size=C)
    A_ref = SG.chunk_simple_gla_fwd_intra(q, k, gamma, 0.3, C)
    _chk("A", A, A_ref, "f32")
    h_ref, _ = SG.chunk_fwd_h_scalar(k, v, None, gamma, h0, False, None, C)
    o = S.chunk_simple_gla_fwd_o_ref(d(q), d(v), d(gamma), A, d(h_ref), 0.3, chunk_size=C)
    _chk("o", o, SG.chunk_simple_gla_fwd_o(q, v, gamma, A_ref, h_ref, 0.3, C), "f32")
    for dtype in ("f32", "bf16"):
        qd, kd, vd, gd, _, h0d, _, _ = _inputs(dict(cfg, T=100), dtype)
        ht_r, o_r = SG.chunk_simple_gla_fwd_ref(qd, kd, vd, gd, 0.3, h0d, True, C)
        dd = lambda x: to_dev(x, dtype)  # noqa: E731
        ht, o2 = S.chunk_simple_gla_fwd_ref(dd(qd), dd(kd), dd(vd), dd(gd), 0.3,
                                            to_dev(h0d, "f32"), True, chunk_size=C)
        _chk("o_ref", o2, o_r, dtype)
        _chk("ht_ref", ht, ht_r, dtype)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_chunk_gla_g_gamma_per_head(dtype):
    """chunk_gla(g_gamma=[H]) takes the scalar-gate path; the gate stays float32 (as the
    reference's ramp), and its gradient is reduced to g_gamma's shape."""
    import tops.ops.gla as G

    cfg = dict(B=2, T=640, H=4, K=128, V=128, seed=77, h0=True)
    q, k, v, gamma, _, h0, do, _ = _inputs(cfg, dtype)
    gamma = (-np.abs(gamma) * 0.37).reshape(4, 1)   # per head: (H, 1); not bf16-exact
    d = lambda x: to_dev(x, dtype)  # noqa: E731
    tq, tk, tv = (d(x).requires_grad_() for x in (q, k, v))
    tg = to_dev(gamma, "f32").requires_grad_()
    th0 = to_dev(h0, "f32").requires_grad_()
    o, ht = G.chunk_gla(tq, tk, tv, g_gamma=tg, initial_state=th0, output_final_state=True,
                        chunk_size=64)
    (o.float() * to_dev(do, "f32")).sum().backward()
    o_ref, ht_ref = orc.chunk_gla(q, k, v, g_gamma=gamma, initial_state=h0,
                                  output_final_state=True, chunk_size=64)
    _chk("o", o, o_ref, dtype)
    _chk("ht", ht, ht_ref, dtype)
    dq_r, dk_r, dv_r, dg_r, dh0_r = orc.chunk_gla_bwd(q, k, v, None, gamma, None, 128 ** -0.5, h0,
                                                      None, None, do, None, chunk_size=64)
    for name, a, b in [("dq", tq.grad, dq_r), ("dk", tk.grad, dk_r), ("dv", tv.grad, dv_r),
                       ("dh0", th0.grad, dh0_r), ("dg_gamma", tg.grad, dg_r)]:
        _chk(name, a, b, dtype)
