"""GPU parity: chunked GLA (forward, backward, sub-functions) vs the numpy oracle.

Inputs follow the reference's test tables (``tests/ops/gla/test_pallas_chunk_gla.py:24-126``,
``test_pallas_chunk_bwd.py:20-80``): odd T, T=1/3, K != V, small dims, many heads, custom
scale, h0/dht, varlen with chunk-aligned and unaligned segments, chunk sizes 16/32/64.
Gates are ``logsigmoid(randn)`` (the reference tests' un-normalized gates) unless noted.
Tolerances: float32 max-abs <= 1e-4; bfloat16 max-abs / max|ref| <= 2e-2 (written in
``gla_cases``).
"""

import numpy as np
import pytest
import torch

import oracle as orc
from gla_cases import check, make_inputs, round_bf16, to_dev, to_np

pytestmark = pytest.mark.gpu

torch.backends.cuda.matmul.allow_tf32 = False


def _gla():
    import tops.ops.gla as G

    return G


FWD_CASES = [
    dict(B=2, T=32, H=4, K=32, V=64, seed=42),
    dict(B=2, T=32, H=4, K=32, V=64, seed=13, h0=True),
    dict(B=1, T=128, H=2, K=64, V=128, seed=7),
    dict(B=2, T=32, H=1, K=32, V=64, seed=10),
    dict(B=2, T=32, H=4, K=16, V=128, seed=20),
    dict(B=2, T=32, H=4, K=128, V=16, seed=21),
    dict(B=1, T=1, H=2, K=32, V=64, seed=30),
    dict(B=1, T=3, H=2, K=32, V=64, seed=31),
    dict(B=2, T=37, H=4, K=16, V=32, seed=40),
    dict(B=1, T=100, H=2, K=32, V=64, seed=42, h0=True),
    dict(B=1, T=64, H=16, K=32, V=64, seed=60),
    dict(B=2, T=32, H=2, K=8, V=16, seed=71, h0=True),
    dict(B=2, T=32, H=4, K=32, V=64, seed=200, scale=0.1),
    dict(B=1, T=96, H=4, K=32, V=64, seed=10, cu=[0, 32, 64, 96]),
    dict(B=1, T=48, H=4, K=32, V=64, seed=18, cu=[0, 16, 48], h0=True),
    dict(B=1, T=50, H=2, K=16, V=32, seed=402, cu=[0, 13, 37, 50]),
    dict(B=1, T=45, H=2, K=32, V=64, seed=404, cu=[0, 20, 45], h0=True),
    dict(B=1, T=512, H=2, K=32, V=64, seed=304, h0=True),
    dict(B=1, T=256, H=2, K=128, V=64, seed=351),
    dict(B=1, T=256, H=2, K=256, V=512, seed=5, h0=True, C=64),
    dict(B=1, T=256, H=1, K=192, V=96, seed=6, C=32),
    # C1: fp32, B=1 T=256 H=2 K=V=64, chunk 64, g/16
    dict(B=1, T=256, H=2, K=64, V=64, seed=1, C=64, gate_div=16.0),
    # long bf16 chunk-64 sequences: the full-head kernels split them into segments
    # (2048 tokens -> 4 segments of 8 chunks; 2000 -> partial last chunk; 1536 -> 3 segments)
    dict(B=2, T=2048, H=2, K=128, V=128, seed=801, C=64, h0=True, gate_div=16.0),
    dict(B=1, T=2000, H=3, K=64, V=128, seed=802, C=64, h0=True),
    dict(B=2, T=1536, H=1, K=96, V=40, seed=803, C=64, h0=True, gate_div=4.0),
    # wide heads on the full-head forward: K = 256 in 64-column V tiles (a partial last
    # tile), segmented (1024 tokens -> 2 segments x 3 V tiles)
    dict(B=1, T=1024, H=2, K=256, V=160, seed=804, C=64, h0=True, gate_div=16.0),
    dict(B=1, T=300, H=2, K=200, V=72, seed=805, C=64, h0=True),
    # V in (64, 128] but not a multiple of 64 (whole-row o / h stores with plain stores, a
    # partial second v half), K not a multiple of 64; partial last chunk, two segments
    dict(B=1, T=1100, H=2, K=112, V=96, seed=830, C=64, h0=True, gate_div=8.0),
    dict(B=2, T=700, H=1, K=64, V=80, seed=831, C=64),
    # K = 200 (a partial last 64-column K slice) with three V tiles: per-chunk gating
    # workspace, partial last chunk; 1100 tokens -> two segments streaming it
    dict(B=1, T=300, H=2, K=200, V=200, seed=806, C=64, h0=True, gate_div=4.0),
    dict(B=1, T=1100, H=2, K=200, V=192, seed=807, C=64, h0=True, gate_div=16.0),
    # varlen wide head: no gating workspace (fixed-length only), every tile gates for itself
    dict(B=1, T=400, H=2, K=256, V=192, seed=808, C=64, h0=True, cu=[0, 70, 256, 400],
         gate_div=8.0),
    # varlen on the main shape (full-head kernels, unsegmented): unaligned sequences, one of a
    # single token
    dict(B=1, T=700, H=2, K=128, V=128, seed=809, C=64, h0=True, cu=[0, 130, 131, 500, 700],
         gate_div=8.0),
    # empty sequences (their final state is their initial state) on the main shape and on the
    # per-chunk kernels, the latter with tokens after the last sequence (outputs zero there)
    dict(B=1, T=200, H=2, K=128, V=128, seed=820, C=64, h0=True, cu=[0, 0, 70, 70, 200],
         gate_div=8.0),
    dict(B=1, T=60, H=2, K=32, V=64, seed=821, h0=True, cu=[0, 20, 20, 50]),
]


def _cid(c):
    s = f"B{c['B']}T{c['T']}H{c['H']}K{c['K']}V{c['V']}-C{c.get('C', 16)}"
    for key in ("h0", "dht"):
        if c.get(key):
            s += f"-{key}"
    if c.get("cu"):
        s += f"-segs{len(c['cu']) - 1}"
    if "scale" in c:
        s += f"-s{c['scale']}"
    return s


def _run_fwd(cfg, dtype):
    G = _gla()
    cu = cfg.get("cu")
    N = len(cu) - 1 if cu else cfg["B"]
    q, k, v, g, s0, _, _ = make_inputs(cfg["B"], cfg["T"], cfg["H"], cfg["K"], cfg["V"],
                                       cfg["seed"], gate_div=cfg.get("gate_div", 1.0),
                                       h0=cfg.get("h0", False), N=N, dtype=dtype)
    o, ht = G.chunk_gla(to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype), to_dev(g, dtype),
                        scale=cfg.get("scale"), initial_state=to_dev(s0, "state"),
                        output_final_state=True,
                        cu_seqlens=None if cu is None else torch.tensor(cu),
                        chunk_size=cfg.get("C", 16))
    torch.cuda.synchronize()
    on, hn = orc.naive_recurrent_gla(q, k, v, g, scale=cfg.get("scale"), initial_state=s0,
                                     output_final_state=True, cu_seqlens=cu)
    return to_np(o), to_np(ht), on, hn, o.dtype


@pytest.mark.parametrize("cfg", FWD_CASES, ids=[_cid(c) for c in FWD_CASES])
def test_chunk_gla_fwd_f32(cfg):
    o, ht, on, hn, odt = _run_fwd(cfg, "f32")
    assert odt == torch.float32
    check("o", o, on, "f32")
    check("ht", ht, hn, "f32")


@pytest.mark.parametrize("cfg", FWD_CASES, ids=[_cid(c) for c in FWD_CASES])
def test_chunk_gla_fwd_bf16(cfg):
    o, ht, on, hn, odt = _run_fwd(cfg, "bf16")
    assert odt == torch.bfloat16
    check("o", o, on, "bf16")
    check("ht", ht, hn, "bf16")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_only_empty_sequences(dtype):
    """Every sequence empty: nothing runs; o is zero, ht = h0, dh0 = dht, no other
    gradient."""
    G = _gla()
    B, T, H, K, V = 1, 5, 2, 64, 64
    q, k, v, g, s0, do, dht = make_inputs(B, T, H, K, V, 830, h0=True, dht=True, N=2,
                                          dtype=dtype)
    tq, tk, tv, tg = (to_dev(x, dtype).requires_grad_() for x in (q, k, v, g))
    th0 = to_dev(s0, "state").requires_grad_()
    o, ht = G.chunk_gla(tq, tk, tv, tg, initial_state=th0, output_final_state=True,
                        cu_seqlens=torch.tensor([0, 0, 0]), chunk_size=64)
    assert o.shape == (B, T, H, V) and not o.float().abs().max().item()
    assert torch.equal(ht, th0.detach())
    (ht * to_dev(dht, "state")).sum().backward()
    assert torch.equal(th0.grad, to_dev(dht, "state"))


def test_forward_same_with_and_without_grad():
    """The full-head forward stores the per-chunk states (the backward's residual) only when a
    gradient is wanted; o and the final state are bit-identical either way, segmented (1024
    tokens: 2 segments) and not."""
    G = _gla()
    for T in (256, 1024):
        q, k, v, g, s0, _, _ = make_inputs(2, T, 2, 128, 128, 611, gate_div=16.0, h0=True,
                                           dtype="bf16")
        x = [to_dev(a, "bf16") for a in (q, k, v, g)]
        h0 = to_dev(s0, "state")
        o0, h0n = G.chunk_gla(*x, initial_state=h0, output_final_state=True, chunk_size=64)
        xg = [a.clone().requires_grad_() for a in x]
        o1, h1n = G.chunk_gla(*xg, initial_state=h0, output_final_state=True, chunk_size=64)
        torch.cuda.synchronize()
        assert torch.equal(o0, o1.detach()), f"T={T}: o differs"
        assert torch.equal(h0n, h1n.detach()), f"T={T}: final state differs"
        o_ref, _ = orc.naive_recurrent_gla(q, k, v, g, initial_state=s0, output_final_state=True)
        check("o", to_np(o0), o_ref, "bf16")


def test_no_final_state_and_state_split():
    G = _gla()
    q, k, v, g, _, _, _ = make_inputs(1, 40, 2, 16, 32, 77)
    d = lambda x: to_dev(x, "f32")  # noqa: E731
    o, s = G.chunk_gla(d(q), d(k), d(v), d(g), output_final_state=False)
    assert s is None
    _, s_full = G.chunk_gla(d(q), d(k), d(v), d(g), output_final_state=True)
    _, s1 = G.chunk_gla(d(q[:, :20]), d(k[:, :20]), d(v[:, :20]), d(g[:, :20]),
                        output_final_state=True)
    _, s2 = G.chunk_gla(d(q[:, 20:]), d(k[:, 20:]), d(v[:, 20:]), d(g[:, 20:]),
                        initial_state=s1, output_final_state=True)
    check("split", to_np(s2), to_np(s_full), "f32")


BWD_CASES = [
    dict(B=2, T=32, H=4, K=32, V=64, seed=42),
    dict(B=2, T=32, H=4, K=32, V=64, seed=15, h0=True, dht=True),
    dict(B=1, T=128, H=2, K=64, V=128, seed=7, dht=True),
    dict(B=2, T=32, H=4, K=16, V=128, seed=20, h0=True),
    dict(B=2, T=32, H=4, K=128, V=16, seed=21),
    dict(B=2, T=37, H=4, K=16, V=32, seed=40, dht=True),
    dict(B=1, T=64, H=16, K=32, V=64, seed=60),
    dict(B=2, T=32, H=2, K=8, V=16, seed=70, h0=True),
    dict(B=2, T=32, H=4, K=32, V=64, seed=200, scale=0.1),
    dict(B=1, T=256, H=2, K=32, V=64, seed=303, h0=True, dht=True),
    dict(B=2, T=64, H=4, K=32, V=64, seed=500, C=32),
    # the reference table's chunk sizes 8 and 4 (test_pallas_chunk_bwd.py:43,45,73)
    dict(B=1, T=128, H=2, K=32, V=64, seed=501, C=8, h0=True, dht=True),
    dict(B=1, T=64, H=2, K=32, V=64, seed=503, C=4),
    dict(B=1, T=64, H=2, K=16, V=32, seed=511, C=8, cu=[0, 32, 64]),
    dict(B=2, T=128, H=4, K=32, V=64, seed=502, C=64, h0=True, dht=True),
    dict(B=1, T=48, H=4, K=32, V=64, seed=20, cu=[0, 16, 48], h0=True, dht=True),
    dict(B=1, T=45, H=2, K=32, V=64, seed=604, cu=[0, 20, 45], h0=True, dht=True),
    dict(B=1, T=50, H=2, K=16, V=32, seed=602, cu=[0, 13, 37, 50]),
    dict(B=1, T=256, H=2, K=256, V=512, seed=8, C=64, h0=True, dht=True),
    dict(B=1, T=192, H=2, K=128, V=128, seed=4, C=64, h0=True, dht=True, gate_div=16.0),
    dict(B=2, T=2048, H=2, K=128, V=128, seed=811, C=64, h0=True, dht=True, gate_div=16.0),
    dict(B=1, T=2000, H=3, K=64, V=128, seed=812, C=64, h0=True, dht=True),
    dict(B=2, T=1536, H=1, K=96, V=40, seed=813, C=64, dht=True, gate_div=4.0),
    # 128 x 64 state tiles: the backward's fp32 exchange must not alias the A / dA tiles
    dict(B=1, T=1024, H=2, K=128, V=64, seed=814, C=64, h0=True, dht=True, gate_div=4.0),
    # K, V not multiples of 64: the dq / dk / dg rows and o / h rows are not whole lines (plain
    # stores), a partial second v half, a partial last chunk, two segments
    dict(B=1, T=1100, H=2, K=112, V=96, seed=832, C=64, h0=True, dht=True, gate_div=8.0),
    dict(B=2, T=700, H=1, K=64, V=80, seed=833, C=64, dht=True),
    # wide head: full-head forward and dh scan (V tiles, segments), per-chunk gradients
    dict(B=1, T=1024, H=2, K=256, V=192, seed=815, C=64, h0=True, dht=True, gate_div=16.0),
    # K = 200, three V tiles: the scans and the dv kernel stream the per-chunk gating (a
    # partial last K slice, a partial last chunk, two segments)
    dict(B=1, T=1100, H=2, K=200, V=192, seed=816, C=64, h0=True, dht=True, gate_div=8.0),
    dict(B=1, T=300, H=2, K=200, V=200, seed=817, C=64, dht=True, gate_div=4.0),
    # varlen wide head (no gating workspace)
    dict(B=1, T=400, H=2, K=256, V=192, seed=818, C=64, h0=True, dht=True, cu=[0, 70, 256, 400],
         gate_div=8.0),
    # per-chunk dq / dk / dg with K <= 128 and V > 128 (128-wide key tiles): a partial last
    # chunk, V = 136 (a partial last 64-column V tile), K = 96 (a partial key tile), varlen
    dict(B=2, T=130, H=3, K=128, V=256, seed=831, C=64, h0=True, dht=True, gate_div=4.0),
    dict(B=1, T=250, H=2, K=96, V=136, seed=832, C=64, dht=True, cu=[0, 40, 250],
         gate_div=4.0),
    # varlen on the main shape (full-head kernels): unaligned sequences, one of a single token
    dict(B=1, T=700, H=2, K=128, V=128, seed=819, C=64, h0=True, dht=True,
         cu=[0, 130, 131, 500, 700], gate_div=8.0),
    # empty sequences: no gradient flows through them, dh0 = dht
    dict(B=1, T=200, H=2, K=128, V=128, seed=820, C=64, h0=True, dht=True,
         cu=[0, 0, 70, 70, 200], gate_div=8.0),
    dict(B=1, T=50, H=2, K=32, V=64, seed=822, h0=True, dht=True, cu=[0, 20, 20, 50, 50]),
]


def _run_bwd(cfg, dtype):
    G = _gla()
    cu = cfg.get("cu")
    N = len(cu) - 1 if cu else cfg["B"]
    B, T, H, K, V = (cfg[x] for x in "BTHKV")
    q, k, v, g, s0, do, dht = make_inputs(B, T, H, K, V, cfg["seed"],
                                          gate_div=cfg.get("gate_div", 1.0),
                                          h0=cfg.get("h0", False), dht=cfg.get("dht", False),
                                          N=N, dtype=dtype)
    sc = cfg.get("scale")
    tq, tk, tv, tg = (to_dev(x, dtype).requires_grad_() for x in (q, k, v, g))
    th0 = to_dev(s0, "state")
    if th0 is not None:
        th0.requires_grad_()
    o, ht = G.chunk_gla(tq, tk, tv, tg, scale=sc, initial_state=th0, output_final_state=True,
                        cu_seqlens=None if cu is None else torch.tensor(cu),
                        chunk_size=cfg.get("C", 16))
    loss = (o.float() * to_dev(do, "f32")).sum()
    if dht is not None:
        loss = loss + (ht * to_dev(dht, "state")).sum()
    loss.backward()
    torch.cuda.synchronize()
    ref = orc.chunk_gla_bwd(q, k, v, g, None, None, K ** -0.5 if sc is None else sc, s0, None,
                            None, do, dht, cu_seqlens=cu, chunk_size=16)
    got = [to_np(x.grad) for x in (tq, tk, tv, tg)] + [None if th0 is None else to_np(th0.grad)]
    return got, ref


@pytest.mark.parametrize("cfg", BWD_CASES, ids=[_cid(c) for c in BWD_CASES])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_chunk_gla_bwd(cfg, dtype):
    """Every gradient against the float64 oracle; float32 at the north-star bar, max-abs
    error 1e-4 (absolute), bf16 at error / max |ref| 2e-2."""
    got, ref = _run_bwd(cfg, dtype)
    errs = {}
    # wide heads (K = 256, V = 512): dq / dk / dv sum up to 512 + 64 products per element,
    # values up to ~10^2, where float32 rounding alone reaches 1e-4
    wide = "sums over wide heads" if cfg["K"] * cfg["V"] > 128 * 128 else None
    for name, a, b in zip(["dq", "dk", "dv", "dg", "dh0"], got, ref):
        if a is None:
            continue
        errs[name] = check(name, a, b, dtype, rel_f32=wide)
    print(f"  {dtype} errors: " + ", ".join(f"{n} {e:.2e}" for n, e in errs.items()),
          flush=True)


# ---------------------------------------------------------------------------
# sub-functions
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("C", [4, 16, 64])
@pytest.mark.parametrize("reverse", [False, True])
@pytest.mark.parametrize("varlen", [False, True])
def test_chunk_local_cumsum(C, reverse, varlen):
    G = _gla()
    r = np.random.default_rng(3)
    cu = [0, 7, 20, 70] if varlen else None
    B = 1 if varlen else 2
    g = r.standard_normal((B, 70, 3, 40))
    out = G.chunk_local_cumsum(to_dev(g, "f32"), C, reverse=reverse, scale=0.5,
                               cu_seqlens=cu)
    ref = orc.chunk_local_cumsum(g, C, reverse=reverse, scale=0.5, cu_seqlens=cu)
    check("cumsum", to_np(out), ref, "f32", atol=1e-5)
    hf = G.chunk_local_cumsum(to_dev(g.transpose(0, 2, 1, 3), "f32"), C, reverse=reverse,
                              head_first=True, cu_seqlens=cu)
    ref2 = orc.chunk_local_cumsum(g, C, reverse=reverse, cu_seqlens=cu)
    check("cumsum_hf", to_np(hf).transpose(0, 2, 1, 3), ref2, "f32", atol=1e-5)


def test_fwd_subfunctions_compose():
    """chunk_local_cumsum -> chunk_fwd_h -> intra -> o_gk reproduces the oracle's pieces."""
    G = _gla()
    B, T, H, K, V, C = 2, 128, 2, 64, 32, 32
    q, k, v, g, s0, _, _ = make_inputs(B, T, H, K, V, 11, h0=True)
    d = lambda x: to_dev(x, "f32")  # noqa: E731
    gc = G.chunk_local_cumsum(d(g), C)
    gc_ref = orc.chunk_local_cumsum(g, C)
    check("g_cumsum", to_np(gc), gc_ref, "f32", atol=1e-5)
    h, ht = G.chunk_fwd_h(d(k), d(v), gc, to_dev(s0, "state"), True, chunk_size=C)
    h_ref, ht_ref = orc.chunk_fwd_h(k, v, gc_ref, s0, True, chunk_size=C)
    check("h", to_np(h), h_ref, "f32")
    check("ht", to_np(ht), ht_ref, "f32")
    A = G.chunk_gla_fwd_intra_gk(d(q), d(k), gc, K ** -0.5, chunk_size=C)
    A_ref = orc.chunk_gla_fwd_intra_gk(q, k, gc_ref, K ** -0.5, C)
    check("A", to_np(A), A_ref, "f32", rel_f32="unmasked intra matrix")
    o = G.chunk_gla_fwd_o_gk(d(q), d(v), gc, A, h, K ** -0.5, chunk_size=C)
    o_ref = orc.chunk_gla_fwd_o_gk(q, v, gc_ref, A_ref, h_ref, K ** -0.5, C)
    check("o", to_np(o), o_ref, "f32")
    gcs, A2, h2, ht2, o2 = G.chunk_gla_fwd(d(q), d(k), d(v), d(g), None, None, K ** -0.5,
                                           to_dev(s0, "state"), True, chunk_size=C)
    check("fwd.o", to_np(o2), o_ref, "f32")
    check("fwd.h", to_np(h2), h_ref, "f32")
    check("fwd.ht", to_np(ht2), ht_ref, "f32")


SMALL_FWD_CASES = [
    # the reference table's chunk sizes 8 and 4 (test_pallas_chunk_bwd.py:43,45,73)
    dict(B=1, T=128, H=2, K=32, V=64, seed=501, C=8, h0=True),
    dict(B=1, T=64, H=2, K=32, V=64, seed=503, C=4),
    dict(B=1, T=64, H=2, K=16, V=32, seed=511, C=8, cu=[0, 32, 64]),
    # unaligned T and varlen (padded per segment by the orchestrator), K != V, wide K
    dict(B=2, T=37, H=3, K=16, V=24, seed=512, C=8, h0=True),
    dict(B=1, T=30, H=2, K=16, V=32, seed=513, C=4, cu=[0, 10, 30], h0=True),
    dict(B=1, T=32, H=1, K=256, V=8, seed=514, C=8),
]


@pytest.mark.parametrize("cfg", SMALL_FWD_CASES,
                         ids=[f"C{c['C']}-T{c['T']}-K{c['K']}{'-varlen' if c.get('cu') else ''}"
                              for c in SMALL_FWD_CASES])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_small_chunk_forward_subfunctions(cfg, dtype):
    """chunk_gla_fwd and its pieces (chunk_fwd_h, chunk_gla_fwd_intra_gk, chunk_gla_fwd_o_gk)
    at chunk sizes 4 and 8 against the oracle at the same chunk size; chunk_bwd_dh on the
    same gates."""
    from tops.ops.common import chunk_h as CH

    G = _gla()
    B, T, H, K, V, C = (cfg[x] for x in "BTHKVC")
    cu = cfg.get("cu")
    N = len(cu) - 1 if cu else B
    q, k, v, g, s0, do, dht = make_inputs(B, T, H, K, V, cfg["seed"], h0=cfg.get("h0", False),
                                          dht=True, N=N, dtype=dtype)
    d = lambda x: to_dev(x, dtype)  # noqa: E731
    tol = (lambda ref: 1e-4) if dtype == "f32" else (lambda ref: None)  # noqa: E731
    scale = K ** -0.5
    out = G.chunk_gla_fwd(d(q), d(k), d(v), d(g), None, None, scale,
                          to_dev(s0, "state"), True, cu_seqlens=cu, chunk_size=C)
    ref = orc.chunk_gla_fwd(q, k, v, g, None, None, scale, s0, True, cu_seqlens=cu,
                            chunk_size=C)
    # the intra matrix is unmasked, as the reference returns it: its upper triangle grows as
    # e^{g~_i - g~_j} with i < j (values up to ~10^3 here)
    unmasked = "unmasked intra matrix" if dtype == "f32" else None
    for name, a, b in zip(["g_cumsum", "A", "h", "ht", "o"], out, ref):
        check(name, to_np(a), b, dtype, atol=tol(b), rel_f32=unmasked if name == "A" else None)
    if T % C or cu is not None:
        return   # the pieces below take chunk-aligned, fixed-length inputs
    gc_ref = ref[0]
    gc = out[0]
    h, ht = G.chunk_fwd_h(d(k), d(v), gc, to_dev(s0, "state"), True, chunk_size=C)
    check("h", to_np(h), ref[2], dtype, atol=tol(ref[2]))
    check("ht", to_np(ht), ref[3], dtype, atol=tol(ref[3]))
    A = G.chunk_gla_fwd_intra_gk(d(q), d(k), gc, scale, chunk_size=C)
    check("A", to_np(A), ref[1], dtype, atol=tol(ref[1]), rel_f32=unmasked)
    o = G.chunk_gla_fwd_o_gk(d(q), d(v), gc, A, h, scale, chunk_size=C)
    check("o", to_np(o), ref[4], dtype, atol=tol(ref[4]))
    dh_ref, dh0_ref = orc.chunk_bwd_dh(q, gc_ref, do, s0, dht, scale, chunk_size=C)
    dh, dh0 = CH.chunk_bwd_dh_ref(d(q), None, None, gc, d(do), h0=to_dev(s0, "state"),
                                  dht=to_dev(dht, "state"), scale=scale, chunk_size=C)
    check("dh", to_np(dh), dh_ref, dtype, atol=tol(dh_ref))
    check("dh0", to_np(dh0), dh0_ref, dtype, atol=tol(dh0_ref))


def test_chunk_gla_fwd_and_bwd_orchestrators_padded():
    G = _gla()
    B, T, H, K, V, C = 1, 45, 2, 32, 64, 16
    cu = [0, 20, 45]
    q, k, v, g, s0, do, dht = make_inputs(B, T, H, K, V, 604, h0=True, dht=True, N=2)
    d = lambda x: to_dev(x, "f32")  # noqa: E731
    out = G.chunk_gla_fwd(d(q), d(k), d(v), d(g), None, None, K ** -0.5, to_dev(s0, "state"),
                          True, cu_seqlens=cu, chunk_size=C)
    ref = orc.chunk_gla_fwd(q, k, v, g, None, None, K ** -0.5, s0, True, cu_seqlens=cu,
                            chunk_size=C)
    for name, a, b in zip(["g_cumsum", "A", "h", "ht", "o"], out, ref):
        check(name, to_np(a), b, "f32",
              rel_f32="unmasked intra matrix" if name == "A" else None)
    grads = G.chunk_gla_bwd(d(q), d(k), d(v), d(g), None, None, K ** -0.5, to_dev(s0, "state"),
                            out[2], None, d(do), to_dev(dht, "state"), cu_seqlens=cu,
                            chunk_size=C)
    gref = orc.chunk_gla_bwd(q, k, v, g, None, None, K ** -0.5, s0, None, None, do, dht,
                             cu_seqlens=cu, chunk_size=C)
    for name, a, b in zip(["dq", "dk", "dv", "dg", "dh0"], grads, gref):
        check(name, to_np(a), b, "f32")


@pytest.mark.parametrize("cfg", [
    dict(B=1, T=128, H=2, K=32, V=64, seed=501, C=8, h0=True, dht=True),
    dict(B=1, T=64, H=2, K=32, V=64, seed=503, C=4),
    dict(B=1, T=64, H=2, K=16, V=32, seed=511, C=8, cu=[0, 32, 64]),
], ids=["C8-h0-dht", "C4", "C8-varlen"])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_chunk_gla_bwd_orchestrator_small_chunks(cfg, dtype):
    """chunk_gla_bwd called directly with the reference table's chunk sizes 8 and 4
    (test_pallas_chunk_bwd.py:43,45,73), against the oracle at the same chunk size."""
    G = _gla()
    B, T, H, K, V, C = (cfg[x] for x in "BTHKVC")
    cu = cfg.get("cu")
    N = len(cu) - 1 if cu else B
    q, k, v, g, s0, do, dht = make_inputs(B, T, H, K, V, cfg["seed"], h0=cfg.get("h0", False),
                                          dht=cfg.get("dht", False), N=N, dtype=dtype)
    d = lambda x: to_dev(x, dtype)  # noqa: E731
    grads = G.chunk_gla_bwd(d(q), d(k), d(v), d(g), None, None, K ** -0.5,
                            to_dev(s0, "state"), None, None, d(do), to_dev(dht, "state"),
                            cu_seqlens=cu, chunk_size=C)
    gref = orc.chunk_gla_bwd(q, k, v, g, None, None, K ** -0.5, s0, None, None, do, dht,
                             cu_seqlens=cu, chunk_size=C)
    for name, a, b in zip(["dq", "dk", "dv", "dg", "dh0"], grads, gref):
        if b is None:
            assert a is None, name
            continue
        check(name, to_np(a), b, dtype)   # float32: max-abs error 1e-4


def test_g_gamma_gradient_reduced():
    G = _gla()
    B, T, H, K, V = 1, 48, 2, 16, 16
    q, k, v, _, _, do, _ = make_inputs(B, T, H, K, V, 12)
    gg = -np.abs(np.random.default_rng(1).standard_normal((H, 1))) * 0.1
    d = lambda x: to_dev(x, "f32")  # noqa: E731
    tgg = d(gg).requires_grad_()
    o, _ = G.chunk_gla(d(q), d(k), d(v), g_gamma=tgg, chunk_size=16)
    (o * d(do)).sum().backward()
    o_ref, _ = orc.chunk_gla(q, k, v, g_gamma=gg, chunk_size=16)
    check("o", to_np(o), o_ref, "f32")
    _, _, _, dg_ref, _ = orc.chunk_gla_bwd(q, k, v, None, gg, None, K ** -0.5, None, None, None,
                                           do, None, chunk_size=16)
    # the gradient of a per-head decay sums dg over every token and key column of the head
    check("dg_gamma", to_np(tgg.grad), dg_ref, "f32", rel_f32="sum over a head's tokens")


def test_deterministic():
    G = _gla()
    q, k, v, g, s0, do, _ = make_inputs(2, 200, 3, 64, 64, 9, h0=True, dtype="bf16")
    outs = []
    for _ in range(2):
        tq, tk, tv, tg = (to_dev(x, "bf16").requires_grad_() for x in (q, k, v, g))
        o, _ = G.chunk_gla(tq, tk, tv, tg, chunk_size=64)
        (o.float() * to_dev(do, "f32")).sum().backward()
        outs.append([o.detach().clone()] + [x.grad.clone() for x in (tq, tk, tv, tg)])
    for a, b in zip(*outs):
        assert torch.equal(a, b)


# ---------------------------------------------------------------------------
# north-star shape: per-(b, h) slices against the oracle, full-size properties
# ---------------------------------------------------------------------------


def test_north_star_shape_slices():
    """C4 (B4 T8192 H16 K=V=128, bf16, chunk 64) fwd+bwd: two (b, h) slices vs the oracle,
    plus finiteness of every output at full size."""
    G = _gla()
    B, T, H, K, V = 4, 8192, 16, 128, 128
    gen = torch.Generator(device="cuda").manual_seed(4)
    mk = lambda *s: torch.randn(*s, generator=gen, device="cuda")  # noqa: E731
    q, k, v = (mk(B, T, H, K).to(torch.bfloat16) for _ in range(3))
    g = (torch.nn.functional.logsigmoid(mk(B, T, H, K)) / 16).to(torch.bfloat16)
    h0 = mk(B, H, K, V) * 0.1
    do = mk(B, T, H, V).to(torch.bfloat16)
    dht = mk(B, H, K, V) * 0.1
    tq, tk, tv, tg = (x.clone().requires_grad_() for x in (q, k, v, g))
    th0 = h0.clone().requires_grad_()
    o, ht = G.chunk_gla(tq, tk, tv, tg, initial_state=th0, output_final_state=True,
                        chunk_size=64)
    torch.autograd.backward([o, ht], [do, dht])
    torch.cuda.synchronize()
    for t in (o, ht, tq.grad, tk.grad, tv.grad, tg.grad, th0.grad):
        assert torch.isfinite(t.float()).all()
    for b, h in [(0, 0), (3, 15)]:
        sl = lambda x: to_np(x[b:b + 1, :, h:h + 1])  # noqa: E731
        s0 = to_np(h0[b:b + 1, h:h + 1])
        sdt = to_np(dht[b:b + 1, h:h + 1])
        qn, kn, vn, gn, don = (sl(x) for x in (q, k, v, g, do))
        on, hn = orc.chunk_gla(qn, kn, vn, gn, initial_state=s0, output_final_state=True,
                               chunk_size=64)
        check("o", sl(o), on, "bf16")
        check("ht", to_np(ht[b:b + 1, h:h + 1]), hn, "bf16")
        ref = orc.chunk_gla_bwd(qn, kn, vn, gn, None, None, K ** -0.5, s0, None, None, don,
                                sdt, chunk_size=64)
        for name, x, r in zip(["dq", "dk", "dv", "dg"], (tq, tk, tv, tg), ref):
            check(name, sl(x.grad), r, "bf16")
        check("dh0", to_np(th0.grad[b:b + 1, h:h + 1]), ref[4], "bf16")


def test_north_star_shape_all_slices_vs_torch_fp32():
    """C4 (B4 T8192 H16 K=V=128, bf16, chunk 64) fwd+bwd, every one of the 64 (b, h) slices
    against the float32 torch chunked GLA (``tests/torch_ref.py``, pinned to the oracle by
    ``test_torch_ref.py``) run on the GPU from the same bf16 inputs, gradients by torch
    autograd. Bar per slice and output: max-abs error / max |ref| of that slice <= 2e-2."""
    from gla_cases import BF16_RTOL_MAX
    from torch_ref import chunk_gla_torch

    G = _gla()
    B, T, H, K, V = 4, 8192, 16, 128, 128
    gen = torch.Generator(device="cuda").manual_seed(11)
    mk = lambda *s: torch.randn(*s, generator=gen, device="cuda")  # noqa: E731
    q, k, v = (mk(B, T, H, K).to(torch.bfloat16) for _ in range(3))
    g = (torch.nn.functional.logsigmoid(mk(B, T, H, K)) / 16).to(torch.bfloat16)
    h0 = mk(B, H, K, V) * 0.1
    do = mk(B, T, H, V).to(torch.bfloat16)
    dht = mk(B, H, K, V) * 0.1
    leaves = [x.clone().requires_grad_() for x in (q, k, v, g, h0)]
    o, ht = G.chunk_gla(*leaves[:4], initial_state=leaves[4], output_final_state=True,
                        chunk_size=64)
    torch.autograd.backward([o, ht], [do, dht])
    refs = [x.float().requires_grad_() for x in (q, k, v, g, h0)]
    ro, rht = chunk_gla_torch(*refs, chunk_size=64)
    torch.autograd.backward([ro, rht], [do.float(), dht])
    torch.cuda.synchronize()

    def per_slice(name, got, ref, tok_major):
        dims = (1, 3) if tok_major else (2, 3)   # [B, T, H, D] or [B, H, K, V]
        got, ref = got.detach().float(), ref.detach().float()
        assert torch.isfinite(got).all(), name
        err = (got - ref).abs().amax(dim=dims)
        scale = ref.abs().amax(dim=dims).clamp_min(1e-30)
        worst = float((err / scale).max())
        print(f"{name}: worst slice error/max|ref| {worst:.3e}", flush=True)
        assert worst <= BF16_RTOL_MAX, f"{name}: worst slice error/max|ref| {worst:.3e}"

    per_slice("o", o, ro, True)
    per_slice("ht", ht, rht, False)
    for name, x, r in zip(["dq", "dk", "dv", "dg"], leaves[:4], refs[:4]):
        per_slice(name, x.grad, r.grad, True)
    per_slice("dh0", leaves[4].grad, refs[4].grad, False)


@pytest.mark.parametrize("B,T,H", [(2, 4096, 4), (1, 2412, 2), (1, 2284, 2)],
                         ids=["even", "short-last", "odd"])
def test_segmented_scans_match_sequential(B, T, H):
    """The segment-parallel scans (local states over chunk pairs, then all segments at once,
    each folding its entry state) give the sequential scan's results: tops_gla_chunk_fwd / _bwd with and without the
    workspace. 2412 tokens: 38 chunks (the last partial) in segments of 10, 10, 10, 8 (a
    short last segment); 2284 tokens: 36 chunks (the last partial) in 4 segments of 9, so
    every segment's pairs end with a single chunk."""
    from tops import _lib
    from tops._lib import SeqLayout, call, ptr, stream_of

    K, V, C = 128, 128, 64
    q, k, v, g, s0, do, dht = make_inputs(B, T, H, K, V, 821, gate_div=16.0, h0=True, dht=True,
                                          dtype="bf16")
    d = lambda x: to_dev(x, "bf16")  # noqa: E731
    q, k, v, g, do = (d(x) for x in (q, k, v, g, do))
    h0, dht = to_dev(s0, "state"), to_dev(dht, "state")
    dev = q.device
    seq = SeqLayout(B, T, C, None, dev)
    st = stream_of(dev)
    ws, nws = _lib.seg_workspace(B, T, H, K, V, C, False, torch.bfloat16, dev, backward=True)
    assert nws > 0, "this shape is expected to use sequence segments"
    outs = []
    for w, n in ((None, 0), (ws, nws)):
        o, h = torch.empty_like(v), torch.empty(seq.NC, H, K, V, dtype=q.dtype, device=dev)
        ht = torch.empty_like(h0)
        call("tops_gla_chunk_fwd", ptr(q), ptr(k), ptr(v), ptr(g), ptr(h0), ptr(o), ptr(ht),
             ptr(h), ptr(w), n, K ** -0.5, B, T, H, K, V, C, *seq.args(), _lib.BF16, st)
        dq, dk, dv, dg = (torch.empty_like(x) for x in (q, k, v, g))
        dh0, dh = torch.empty_like(h0), torch.empty_like(h)
        call("tops_gla_chunk_bwd", ptr(q), ptr(k), ptr(v), ptr(g), ptr(h0), ptr(h), ptr(do),
             ptr(dht), ptr(dq), ptr(dk), ptr(dv), ptr(dg), ptr(dh0), None, ptr(dh), ptr(w), n,
             K ** -0.5, B, T, H, K, V, C, *seq.args(), _lib.BF16, st)
        torch.cuda.synchronize()
        outs.append([o, ht, h, dq, dk, dv, dg, dh0])
    names = ["o", "ht", "h", "dq", "dk", "dv", "dg", "dh0"]
    for name, a, b in zip(names, *outs):
        check(name, to_np(b), to_np(a).astype(np.float64), "bf16")


def test_chunk_bwd_misaligned_outputs_take_the_per_chunk_path():
    """Gradient buffers that are not 16-byte aligned (a C caller's offset views) make
    tops_gla_chunk_bwd leave the fused full-head backward, whose vector stores need the
    alignment, and give the same gradients through the per-chunk kernels."""
    from tops import _lib
    from tops._lib import SeqLayout, call, ptr, stream_of

    B, T, H, K, V, C = 1, 320, 2, 128, 128, 64
    q, k, v, g, s0, do, dht = make_inputs(B, T, H, K, V, 841, gate_div=8.0, h0=True, dht=True,
                                          dtype="bf16")
    d = lambda x: to_dev(x, "bf16")  # noqa: E731
    q, k, v, g, do = (d(x) for x in (q, k, v, g, do))
    h0, dht = to_dev(s0, "state"), to_dev(dht, "state")
    dev = q.device
    seq = SeqLayout(B, T, C, None, dev)
    st = stream_of(dev)
    o, h = torch.empty_like(v), torch.empty(seq.NC, H, K, V, dtype=q.dtype, device=dev)
    ht = torch.empty_like(h0)
    call("tops_gla_chunk_fwd", ptr(q), ptr(k), ptr(v), ptr(g), ptr(h0), ptr(o), ptr(ht),
         ptr(h), None, 0, K ** -0.5, B, T, H, K, V, C, *seq.args(), _lib.BF16, st)
    outs = []
    for off in (0, 1):   # element offset 1 = 2 bytes: every gradient buffer misaligned
        bufs = [torch.empty(x.numel() + 8, dtype=x.dtype, device=dev) for x in (q, k, v, g)]
        dq, dk, dv, dg = (b[off:off + x.numel()].view(x.shape) for b, x in
                          zip(bufs, (q, k, v, g)))
        dh0, dh = torch.empty_like(h0), torch.empty_like(h)
        call("tops_gla_chunk_bwd", ptr(q), ptr(k), ptr(v), ptr(g), ptr(h0), ptr(h), ptr(do),
             ptr(dht), ptr(dq), ptr(dk), ptr(dv), ptr(dg), ptr(dh0), None, ptr(dh), None, 0,
             K ** -0.5, B, T, H, K, V, C, *seq.args(), _lib.BF16, st)
        torch.cuda.synchronize()
        outs.append([x.clone() for x in (dq, dk, dv, dg, dh0)])
    for name, a, b in zip(["dq", "dk", "dv", "dg", "dh0"], *outs):
        check(name, to_np(b), to_np(a), "bf16")


# The backward's parts over given intermediates (reference jnp exports chunk.py:504-743).
PART_CASES = [
    dict(B=2, T=64, H=2, K=32, V=64, C=16, seed=901),
    dict(B=1, T=128, H=3, K=96, V=40, C=32, seed=902),
    dict(B=1, T=128, H=2, K=130, V=70, C=64, seed=903),
    dict(B=2, T=64, H=1, K=256, V=512, C=64, seed=904),
]


@pytest.mark.parametrize("cfg", PART_CASES,
                         ids=[f"B{c['B']}T{c['T']}H{c['H']}K{c['K']}V{c['V']}C{c['C']}"
                              for c in PART_CASES])
def test_bwd_parts(cfg):
    G = _gla()
    B, T, H, K, V, C = (cfg[x] for x in ("B", "T", "H", "K", "V", "C"))
    r = np.random.default_rng(cfg["seed"])
    q, k = r.standard_normal((2, B, T, H, K))
    v, do = r.standard_normal((2, B, T, H, V))
    g = -np.logaddexp(0.0, -r.standard_normal((B, T, H, K)))   # logsigmoid
    gc = orc.chunk_local_cumsum(g, C)
    A = r.standard_normal((B, T, H, C))
    dA = np.tril(r.standard_normal((B, T // C, C, H, C)).transpose(0, 1, 3, 2, 4)) \
        .transpose(0, 1, 3, 2, 4).reshape(B, T, H, C)
    h, dh = r.standard_normal((2, B, T // C, H, K, V)) * 0.5
    dq0, dk0 = r.standard_normal((2, B, T, H, K))
    scale = K ** -0.5
    d = lambda x: to_dev(x, "f32")  # noqa: E731
    tol = lambda ref: 1e-4  # noqa: E731

    got = G.chunk_gla_bwd_dA_ref(d(v), d(do), scale, chunk_size=C)
    ref = orc.chunk_gla_bwd_dA(v, do, scale, C)
    check("dA", to_np(got), ref, "f32", atol=tol(ref))

    got = G.chunk_gla_bwd_dv_ref(d(k), d(gc), d(A), d(do), d(h), chunk_size=C)
    ref = orc.chunk_gla_bwd_dv(k, gc, A, do, h, C)
    check("dv", to_np(got), ref, "f32", atol=tol(ref))

    gq, gk = G.chunk_gla_bwd_dqk_intra_ref(d(q), d(k), d(gc), d(dA), chunk_size=C)
    rq, rk = orc.chunk_gla_bwd_dqk_intra(q, k, gc, dA, C)
    check("dq_intra", to_np(gq), rq, "f32", atol=tol(rq))
    check("dk_intra", to_np(gk), rk, "f32", atol=tol(rk))

    out = G.chunk_gla_bwd_dqkg_ref(d(q), d(k), d(v), d(h), d(gc), d(do), d(dh), d(dq0),
                                   d(dk0), scale, chunk_size=C)
    ref = orc.chunk_gla_bwd_dqkg(q, k, v, h, gc, do, dh, dq0, dk0, scale, C)
    for name, a, b in zip(("dq", "dk", "dg"), out, ref):
        check(name, to_np(a), b, "f32", atol=tol(b))


def test_bwd_parts_compose_to_the_fused_backward():
    """dA -> dqk_intra -> dqkg and dv from the forward's A, h and the backward's dh give the
    fused backward's gradients (reference chunk_gla_bwd, chunk.py:815-977)."""
    G = _gla()
    B, T, H, K, V, C = 1, 128, 2, 32, 48, 32
    q, k, v, g, s0, do, dht = make_inputs(B, T, H, K, V, 905, h0=True, dht=True)
    d = lambda x: to_dev(x, "f32")  # noqa: E731
    scale = K ** -0.5
    gc, A, h, _, _ = G.chunk_gla_fwd(d(q), d(k), d(v), d(g), None, None, scale,
                                      to_dev(s0, "state"), True, chunk_size=C)
    from tops.ops.common.chunk_h import chunk_bwd_dh_ref

    dh, _ = chunk_bwd_dh_ref(d(q), None, None, gc, d(do), h0=to_dev(s0, "state"),
                             dht=to_dev(dht, "state"), scale=scale, chunk_size=C)
    dA = G.chunk_gla_bwd_dA_ref(d(v), d(do), scale, chunk_size=C)
    dv = G.chunk_gla_bwd_dv_ref(d(k), gc, A, d(do), dh, chunk_size=C)
    dq, dk = G.chunk_gla_bwd_dqk_intra_ref(d(q), d(k), gc, dA, chunk_size=C)
    dq, dk, dg = G.chunk_gla_bwd_dqkg_ref(d(q), d(k), d(v), h, gc, d(do), dh, dq, dk, scale,
                                          chunk_size=C)
    ref = orc.chunk_gla_bwd(q, k, v, g, None, None, scale, s0, None, None, do, dht,
                            chunk_size=C)
    for name, a, b in zip(("dq", "dk", "dv", "dg"), (dq, dk, dv, dg), ref):
        check(name, to_np(a), b, "f32")


# tops.ops.common.chunk_h (reference tops/ops/common/chunk_h.py:137-697): state scans with
# gk / scalar g / g_gamma gates, chunk sizes above 64 (run as 64-row chunks), split_size.
CH_CASES = [
    dict(B=2, T=128, H=2, K=32, V=64, C=64, gate="gk", seed=911),
    dict(B=1, T=96, H=3, K=64, V=48, C=32, gate="g", seed=912),
    dict(B=2, T=64, H=2, K=32, V=32, C=16, gate="g_gamma", seed=913),
    dict(B=1, T=256, H=2, K=64, V=64, C=128, gate="gk", seed=914),
    dict(B=1, T=256, H=2, K=32, V=64, C=64, S=128, gate="gk", seed=915),
    dict(B=1, T=192, H=2, K=32, V=64, C=64, gate="gk", seed=916, cu=[0, 64, 192]),
    dict(B=1, T=256, H=1, K=128, V=128, C=128, S=256, gate="g_gamma", seed=917),
    # chunk sizes 4 and 8 (the small-chunk kernels)
    dict(B=2, T=64, H=2, K=32, V=64, C=8, gate="gk", seed=918),
    dict(B=1, T=64, H=2, K=16, V=32, C=4, S=16, gate="gk", seed=919),
    dict(B=1, T=64, H=2, K=32, V=48, C=8, gate="g", seed=920, cu=[0, 24, 64]),
]


def _ch_inputs(cfg):
    B, T, H, K, V, C = (cfg[x] for x in ("B", "T", "H", "K", "V", "C"))
    r = np.random.default_rng(cfg["seed"])
    q, k = r.standard_normal((2, B, T, H, K))
    v, do = r.standard_normal((2, B, T, H, V))
    cu = cfg.get("cu")
    N = len(cu) - 1 if cu else B
    h0, dht = r.standard_normal((2, N, H, K, V))
    gate = cfg["gate"]
    kw, gfull = {}, None
    if gate == "gk":
        gfull = orc.chunk_local_cumsum(-np.logaddexp(0.0, -r.standard_normal((B, T, H, K))) / 4,
                                       C, cu_seqlens=cu)
        kw["gk"] = gfull
    elif gate == "g":
        gs = orc.chunk_local_cumsum(-np.logaddexp(0.0, -r.standard_normal((B, T, H, 1))) / 4,
                                    C, cu_seqlens=cu)[..., 0]
        kw["g"] = gs
        gfull = np.repeat(gs[..., None], K, axis=-1)
    else:
        gg = -np.abs(r.standard_normal(H)) / 8
        kw["g_gamma"] = gg
        bounds = cu if cu else [0, T]
        pos = np.concatenate([np.arange(b - a) % C + 1 for a, b in zip(bounds, bounds[1:])])
        gfull = np.broadcast_to(pos[None, :, None, None] * gg[None, None, :, None],
                                (B, T, H, K)).copy()
    return q, k, v, do, h0, dht, kw, gfull, cu


@pytest.mark.parametrize("cfg", CH_CASES, ids=[f"{c['gate']}-C{c['C']}-S{c.get('S', c['C'])}"
                                               f"{'-varlen' if c.get('cu') else ''}"
                                               for c in CH_CASES])
def test_common_chunk_h(cfg):
    from tops.ops.common import chunk_h as CH

    C = cfg["C"]
    S = cfg.get("S", C)
    q, k, v, do, h0, dht, kw, gfull, cu = _ch_inputs(cfg)
    d = lambda x: to_dev(x, "f32")  # noqa: E731
    dkw = {name: d(x) for name, x in kw.items()}
    cut = None if cu is None else torch.tensor(cu)
    tol = lambda ref: 1e-4  # noqa: E731

    h_ref, ht_ref = orc.chunk_fwd_h(k, v, gfull, h0, True, cu_seqlens=cu, chunk_size=C)
    h, ht = CH.chunk_fwd_h_kernel(d(k), d(v), h0=d(h0), output_final_state=True,
                                  cu_seqlens=cut, chunk_size=C, split_size=S, **dkw)
    check("h", to_np(h), h_ref[:, ::S // C], "f32", atol=tol(h_ref))
    check("ht", to_np(ht), ht_ref, "f32", atol=tol(ht_ref))
    if S == C and "gk" in kw:
        h2, ht2 = CH.chunk_fwd_h_ref(d(k), d(v), gk=dkw["gk"], h0=d(h0), output_final_state=True,
                                     cu_seqlens_cpu=cu, chunk_size=C)
        check("h_ref", to_np(h2), h_ref, "f32", atol=tol(h_ref))

    dh_ref, dh0_ref = orc.chunk_bwd_dh(q, gfull, do, h0, dht, 0.5, cu_seqlens=cu, chunk_size=C)
    dh, dh0 = CH.chunk_bwd_dh_kernel(d(q), d(k), d(v), do=d(do), dht=d(dht), scale=0.5,
                                     output_dh0=True, cu_seqlens=cut, chunk_size=C,
                                     split_size=S, **dkw)
    check("dh", to_np(dh), dh_ref[:, ::S // C], "f32", atol=tol(dh_ref))
    check("dh0", to_np(dh0), dh0_ref, "f32", atol=tol(dh0_ref))
    if S == C and "gk" in kw:
        dh2, dh02 = CH.chunk_bwd_dh_ref(d(q), d(k), d(v), dkw["gk"], d(do), h0=d(h0), dht=d(dht),
                                        scale=0.5, cu_seqlens_cpu=cu, chunk_size=C)
        check("dh_ref", to_np(dh2), dh_ref, "f32", atol=tol(dh_ref))
        check("dh0_ref", to_np(dh02), dh0_ref, "f32", atol=tol(dh0_ref))


# ---------------------------------------------------------------------------
# gate ranges beyond the per-element factoring: flagged blocks, recurrent fallback
# ---------------------------------------------------------------------------

STRONG_CASES = [
    # per-token log decays of about 4 (x5 on logsigmoid(randn)): chunk gate ranges near 256,
    # far beyond the factoring's ~138; segmented (2048 tokens: 4 segments) and not
    dict(B=1, T=2048, H=2, K=128, V=128, seed=861, mul=5.0, h0=True, dht=True),
    dict(B=2, T=300, H=2, K=64, V=128, seed=862, mul=5.0, h0=True, dht=True),
    # only one (sequence, head) pair strong: the others keep the chunked results
    dict(B=2, T=512, H=2, K=128, V=128, seed=863, mul=5.0, only=(1, 0), h0=True, dht=True),
    # varlen, an empty sequence, strong gates in the middle sequence only
    dict(B=1, T=400, H=2, K=128, V=64, seed=864, mul=5.0, cu=[0, 100, 100, 300, 400],
         only_seq=2, h0=True, dht=True),
    # just inside the limit (ranges of about 120-130): the chunked kernels themselves
    dict(B=1, T=1024, H=2, K=128, V=128, seed=865, mul=2.4, h0=True, dht=True),
    # no final-state gradient (the fallback's first scan keeps no final state), with and
    # without an initial state; one strong pair among four
    dict(B=2, T=1100, H=2, K=128, V=128, seed=866, mul=5.0, only=(0, 1), h0=True, dht=False),
    dict(B=1, T=700, H=2, K=64, V=64, seed=867, mul=5.0, h0=False, dht=False),
    # float32 inputs: the per-chunk float32 kernels (fused forward / state scan + output,
    # per-chunk backward), checked per chunk by the gate-range kernel
    dict(B=1, T=600, H=2, K=64, V=64, seed=868, mul=5.0, h0=True, dht=True, dtype="f32"),
    dict(B=2, T=400, H=2, K=128, V=128, seed=869, mul=4.0, only=(1, 1), h0=True, dht=True,
         dtype="f32"),
    dict(B=1, T=500, H=2, K=128, V=96, seed=870, mul=4.0, cu=[0, 130, 330, 500], only_seq=1,
         h0=True, dht=False, dtype="f32"),
    # wide heads, fixed length: K = 256, V = 512 (eight 64-column V tiles: the gating kernel's
    # per-chunk flags; the per-chunk backward checked by the same kernel)
    dict(B=1, T=512, H=2, K=256, V=512, seed=871, mul=4.0, h0=True, dht=True),
    dict(B=2, T=320, H=2, K=256, V=512, seed=872, mul=4.0, only=(0, 1), h0=True, dht=True),
    # wide heads, varlen (no gating workspace: the forward's blocks flag themselves)
    dict(B=1, T=450, H=2, K=256, V=192, seed=873, mul=4.0, cu=[0, 200, 450], only_seq=0,
         h0=True, dht=True),
    # K <= 128 with V > 128: full-head forward, per-chunk backward (checked per chunk)
    dict(B=1, T=640, H=2, K=128, V=256, seed=874, mul=5.0, h0=True, dht=True),
    dict(B=2, T=300, H=2, K=64, V=384, seed=875, mul=5.0, only=(1, 0), h0=True, dht=False),
    # a long sequence through the fallback (bf16 dq read back with its rounding residual by
    # the gate gradient's reverse cumsum over 8192 steps)
    dict(B=1, T=8192, H=1, K=64, V=64, seed=876, mul=5.0, h0=True, dht=True),
]


def _strong_inputs(cfg):
    B, T, H, K, V = (cfg[x] for x in "BTHKV")
    cu = cfg.get("cu")
    N = len(cu) - 1 if cu else B
    q, k, v, g, s0, do, dht = make_inputs(B, T, H, K, V, cfg["seed"], h0=cfg.get("h0", False),
                                          dht=cfg.get("dht", False), N=N)
    mul = np.ones_like(g)
    if "only" in cfg:
        b, h = cfg["only"]
        mul[b, :, h] = cfg["mul"]
    elif "only_seq" in cfg:
        i = cfg["only_seq"]
        mul[:, cu[i]:cu[i + 1]] = cfg["mul"]
    else:
        mul[:] = cfg["mul"]
    g = g * mul
    if cfg.get("dtype", "bf16") == "bf16":
        q, k, v, g, do = (round_bf16(x) for x in (q, k, v, g, do))
    return q, k, v, g, s0, do, dht, cu


@pytest.mark.parametrize("cfg", STRONG_CASES, ids=[f"s{c['seed']}" for c in STRONG_CASES])
def test_strong_gates(cfg):
    """chunk_gla forward and backward with per-token decays of 3-5 (chunk gate ranges beyond
    the kernels' per-element factoring), on every chunked path: the full-head kernels, the
    wide heads' gating kernel, the per-chunk bf16 and float32 kernels. The flagged (sequence,
    head) pairs are recomputed by the recurrent scans; everything matches the float64
    oracle at the dtype's bar (float32: max-abs error 1e-4), and stays finite."""
    G = _gla()
    q, k, v, g, s0, do, dht, cu = _strong_inputs(cfg)
    K = cfg["K"]
    dt = cfg.get("dtype", "bf16")
    print(f"strong gates {cfg}", flush=True)
    tq, tk, tv, tg = (to_dev(x, dt).requires_grad_() for x in (q, k, v, g))
    th0 = to_dev(s0, "state") if s0 is not None else None
    if th0 is not None:
        th0.requires_grad_()
    o, ht = G.chunk_gla(tq, tk, tv, tg, initial_state=th0, output_final_state=True,
                        cu_seqlens=None if cu is None else torch.tensor(cu), chunk_size=64)
    loss = (o.float() * to_dev(do, "f32")).sum()
    if dht is not None:
        loss = loss + (ht * to_dev(dht, "state")).sum()
    loss.backward()
    torch.cuda.synchronize()
    on, hn = orc.naive_recurrent_gla(q, k, v, g, initial_state=s0, output_final_state=True,
                                     cu_seqlens=cu)
    errs = {"o": check("o", to_np(o), on, dt), "ht": check("ht", to_np(ht), hn, dt)}
    ref = orc.chunk_gla_bwd(q, k, v, g, None, None, K ** -0.5, s0, None, None, do, dht,
                            cu_seqlens=cu, chunk_size=16)
    for name, x, r in zip(["dq", "dk", "dv", "dg"], (tq, tk, tv, tg), ref):
        errs[name] = check(name, to_np(x.grad), r, dt)
    if th0 is not None:
        errs["dh0"] = check("dh0", to_np(th0.grad), ref[4], dt)
    print(f"  {'max-abs' if dt == 'f32' else 'max-abs / max|ref|'} errors: "
          + ", ".join(f"{n} {e:.2e}" for n, e in errs.items()), flush=True)
