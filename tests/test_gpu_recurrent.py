"""GPU parity: fused_recurrent_gla and naive_recurrent_gla vs the numpy oracle.

Cases mirror ``tests/ops/gla/test_pallas_fused_recurrent.py:24-174``: gate modes gk / gv /
gk+gv / none, reverse, varlen (single-token and unaligned segments), h0, custom scale,
long T, K != V. Output is float32 (the reference convention) for fused_recurrent_gla and the
input dtype for naive_recurrent_gla.
"""

import numpy as np
import pytest
import torch

import oracle as orc
from gla_cases import check, logsigmoid, round_bf16, to_dev, to_np

pytestmark = pytest.mark.gpu

CASES = [
    dict(B=2, T=32, H=4, K=32, V=64, seed=42),
    dict(B=2, T=32, H=4, K=32, V=64, seed=13, h0=True),
    dict(B=1, T=128, H=2, K=64, V=128, seed=7),
    dict(B=2, T=32, H=4, K=16, V=128, seed=20),
    dict(B=2, T=32, H=4, K=128, V=16, seed=21),
    dict(B=1, T=1, H=2, K=32, V=64, seed=30),
    dict(B=2, T=37, H=4, K=16, V=32, seed=40),
    dict(B=2, T=32, H=2, K=8, V=16, seed=71, h0=True),
    dict(B=2, T=32, H=4, K=32, V=64, seed=100, gate="gv"),
    dict(B=2, T=32, H=4, K=32, V=64, seed=101, gate="gk+gv"),
    dict(B=2, T=32, H=4, K=32, V=64, seed=102, gate="none"),
    dict(B=2, T=32, H=4, K=32, V=64, seed=111, reverse=True, h0=True),
    dict(B=1, T=1, H=2, K=16, V=32, seed=112, reverse=True),
    dict(B=2, T=32, H=4, K=32, V=64, seed=200, scale=0.1),
    dict(B=1, T=23, H=2, K=16, V=32, seed=12, cu=[0, 7, 20, 23]),
    dict(B=1, T=48, H=4, K=32, V=64, seed=18, cu=[0, 10, 24, 48], h0=True),
    dict(B=1, T=4, H=2, K=16, V=32, seed=20, cu=[0, 1, 2, 3, 4]),
    dict(B=1, T=23, H=2, K=16, V=32, seed=121, cu=[0, 7, 20, 23], reverse=True),
    dict(B=1, T=32, H=4, K=32, V=64, seed=131, gate="gk+gv", cu=[0, 16, 32]),
    dict(B=1, T=1024, H=2, K=32, V=64, seed=302),
    dict(B=1, T=256, H=4, K=32, V=64, seed=380, gate="gk+gv", h0=True, reverse=True,
         scale=0.1),
    dict(B=1, T=256, H=2, K=256, V=512, seed=2, h0=True, gate_div=16.0),
    dict(B=1, T=64, H=2, K=200, V=70, seed=3),
    # empty sequences keep their initial state; tokens after the last sequence give zeros
    dict(B=1, T=26, H=2, K=16, V=32, seed=122, cu=[0, 0, 7, 7, 23], h0=True),
    # strong gates: 16-step decays beyond e^-60 take the direct (unrescaled) stages, some
    # stages only (gate_mul 5: about -64 per 16 steps) or all of them (gate_mul 12)
    dict(B=1, T=100, H=2, K=32, V=64, seed=140, gate_mul=12.0, h0=True),
    dict(B=1, T=200, H=2, K=64, V=64, seed=141, gate_mul=5.0, h0=True),
    dict(B=1, T=100, H=2, K=32, V=64, seed=142, gate="gv", gate_mul=8.0, h0=True),
    dict(B=1, T=100, H=2, K=32, V=64, seed=143, gate_mul=8.0, h0=True, reverse=True),
    # short scans (fixed length, T <= 64, K <= 128, 256+ blocks: the short-scan kernel): the
    # decode shape B64 T1 H16 K=V=128; partial tiles (K = 96, V = 200, a partial 64-column
    # tile), both gates; unaligned columns (V = 130), reverse, gv only; K = 20 (rows past K
    # in the last row groups), no gate, custom scale
    dict(B=64, T=1, H=16, K=128, V=128, seed=150, h0=True, gate_div=16.0),
    dict(B=16, T=37, H=8, K=96, V=200, seed=151, h0=True, gate="gk+gv"),
    dict(B=32, T=64, H=4, K=64, V=130, seed=152, reverse=True, gate="gv", h0=True),
    dict(B=16, T=5, H=16, K=20, V=64, seed=153, gate="none", scale=0.3),
]


def _cid(c):
    s = f"B{c['B']}T{c['T']}H{c['H']}K{c['K']}V{c['V']}-{c.get('gate', 'gk')}"
    for key in ("h0", "reverse"):
        if c.get(key):
            s += f"-{key}"
    if c.get("cu"):
        s += f"-segs{len(c['cu']) - 1}"
    return s


def _inputs(cfg, dtype):
    r = np.random.default_rng(cfg["seed"])
    B, T, H, K, V = (cfg[x] for x in "BTHKV")
    gate = cfg.get("gate", "gk")
    div = cfg.get("gate_div", 1.0)
    q, k = r.standard_normal((2, B, T, H, K))
    v = r.standard_normal((B, T, H, V))
    mul = cfg.get("gate_mul", 1.0)
    gk = logsigmoid(r.standard_normal((B, T, H, K))) / div * mul if "gk" in gate else None
    gv = logsigmoid(r.standard_normal((B, T, H, V))) / div * mul if "gv" in gate else None
    cu = cfg.get("cu")
    N = len(cu) - 1 if cu else B
    s0 = r.standard_normal((N, H, K, V)) if cfg.get("h0") else None
    if dtype == "bf16":
        q, k, v = (round_bf16(x) for x in (q, k, v))
        gk = None if gk is None else round_bf16(gk)
        gv = None if gv is None else round_bf16(gv)
    return q, k, v, gk, gv, s0, cu


@pytest.mark.parametrize("cfg", CASES, ids=[_cid(c) for c in CASES])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_fused_recurrent(cfg, dtype):
    import tops.ops.gla as G

    q, k, v, gk, gv, s0, cu = _inputs(cfg, dtype)
    d = lambda x: to_dev(x, dtype)  # noqa: E731
    o, ht = G.fused_recurrent_gla(d(q), d(k), d(v), gk=d(gk), gv=d(gv), scale=cfg.get("scale"),
                                  initial_state=to_dev(s0, "state"), output_final_state=True,
                                  reverse=cfg.get("reverse", False),
                                  cu_seqlens=None if cu is None else torch.tensor(cu))
    torch.cuda.synchronize()
    assert o.dtype == torch.float32 and ht.dtype == torch.float32
    on, hn = orc.fused_recurrent_gla(q, k, v, gk=gk, gv=gv, scale=cfg.get("scale"),
                                     initial_state=s0, output_final_state=True,
                                     reverse=cfg.get("reverse", False), cu_seqlens=cu)
    # the recurrent kernel computes in fp32 from the (bf16-rounded) inputs: hold both dtypes
    # to the fp32 bar, relative to the output magnitude for long accumulations
    check("o", to_np(o), on, "f32")
    check("ht", to_np(ht), hn, "f32")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_naive_recurrent(dtype):
    import tops.ops.gla as G

    cfg = dict(B=1, T=50, H=2, K=32, V=64, seed=41, h0=True, cu=[0, 13, 50])
    q, k, v, gk, _, s0, cu = _inputs(cfg, dtype)
    d = lambda x: to_dev(x, dtype)  # noqa: E731
    o, ht = G.naive_recurrent_gla(d(q), d(k), d(v), d(gk), initial_state=to_dev(s0, "state"),
                                  output_final_state=True, cu_seqlens=cu)
    assert o.dtype == (torch.float32 if dtype == "f32" else torch.bfloat16)
    on, hn = orc.naive_recurrent_gla(q, k, v, gk, initial_state=s0, output_final_state=True,
                                     cu_seqlens=cu)
    check("o", to_np(o), on, dtype)
    check("ht", to_np(ht), hn, "f32")


def test_fused_recurrent_c2_all_slices_vs_torch_fp32():
    """C2 at full size (B8 T2048 H4 K256 V512, bf16 inputs, h0, float32 o), all 32 (b, h)
    slices of o and ht against the float32 torch chunked GLA (``tests/torch_ref.py``, pinned
    to the oracle by ``test_torch_ref.py``; the same recurrence in chunk form, 16-token chunks
    so that its gate factors stay small) on the GPU from the same inputs. Bar per slice:
    max-abs error <= 1e-4."""
    import tops.ops.gla as G
    from torch_ref import chunk_gla_torch, slice_errors

    B, T, H, K, V = 8, 2048, 4, 256, 512
    gen = torch.Generator(device="cuda").manual_seed(22)
    mk = lambda *s: torch.randn(*s, generator=gen, device="cuda")  # noqa: E731
    q, k = (mk(B, T, H, K).to(torch.bfloat16) for _ in range(2))
    v = mk(B, T, H, V).to(torch.bfloat16)
    gk = (torch.nn.functional.logsigmoid(mk(B, T, H, K)) / 16).to(torch.bfloat16)
    h0 = mk(B, H, K, V) * 0.1
    o, ht = G.fused_recurrent_gla(q, k, v, gk=gk, initial_state=h0, output_final_state=True)
    assert o.dtype == torch.float32
    with torch.no_grad():
        ro, rht = chunk_gla_torch(q.float(), k.float(), v.float(), gk.float(), h0,
                                  chunk_size=16)
    torch.cuda.synchronize()
    for name, x, r, tm in (("o", o, ro, True), ("ht", ht, rht, False)):
        err, scale = slice_errors(x, r, tm)
        worst = float(err.max())
        print(f"{name}: worst slice max-abs error {worst:.3e} (max |ref| "
              f"{float(scale.max()):.2f})", flush=True)
        assert worst <= 1e-4, name


def test_fused_recurrent_c2_shape_slices():
    """C2 (B8 T2048 H4 K256 V512, bf16, h0, output_final_state): slices vs the oracle."""
    import tops.ops.gla as G

    B, T, H, K, V = 8, 2048, 4, 256, 512
    gen = torch.Generator(device="cuda").manual_seed(2)
    mk = lambda *s: torch.randn(*s, generator=gen, device="cuda")  # noqa: E731
    q, k = (mk(B, T, H, K).to(torch.bfloat16) for _ in range(2))
    v = mk(B, T, H, V).to(torch.bfloat16)
    gk = (torch.nn.functional.logsigmoid(mk(B, T, H, K)) / 16).to(torch.bfloat16)
    h0 = mk(B, H, K, V) * 0.1
    o, ht = G.fused_recurrent_gla(q, k, v, gk=gk, initial_state=h0, output_final_state=True)
    torch.cuda.synchronize()
    assert torch.isfinite(o).all() and torch.isfinite(ht).all()
    for b, h in [(0, 0), (7, 3)]:
        sl = lambda x: to_np(x[b:b + 1, :256, h:h + 1])  # noqa: E731
        on, _ = orc.fused_recurrent_gla(sl(q), sl(k), sl(v), gk=sl(gk),
                                        initial_state=to_np(h0[b:b + 1, h:h + 1]),
                                        output_final_state=False)
        check("o[:256]", sl(o), on, "f32")


# ---------------------------------------------------------------------------
# backward: fused_recurrent_gla_bwd and the autodiff rule of fused_recurrent_gla
# ---------------------------------------------------------------------------

# Mirrors tests/ops/gla/test_pallas_fused_recurrent_bwd.py:25-158 (dht defaults to h0).
BWD_CASES = [
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
    dict(B=8, T=32, H=4, K=32, V=64, seed=50),
    dict(B=2, T=32, H=2, K=8, V=16, seed=71, h0=True),
    dict(B=2, T=32, H=4, K=32, V=64, seed=100, gate="gv"),
    dict(B=2, T=32, H=4, K=32, V=64, seed=101, gate="gk+gv"),
    dict(B=2, T=32, H=4, K=32, V=64, seed=102, gate="none"),
    dict(B=2, T=32, H=4, K=32, V=64, seed=110, reverse=True),
    dict(B=2, T=32, H=4, K=32, V=64, seed=111, reverse=True, h0=True),
    dict(B=1, T=1, H=2, K=16, V=32, seed=112, reverse=True),
    dict(B=2, T=32, H=4, K=32, V=64, seed=200, scale=0.1),
    dict(B=1, T=48, H=4, K=32, V=64, seed=11, cu=[0, 10, 24, 48]),
    dict(B=1, T=23, H=2, K=16, V=32, seed=12, cu=[0, 7, 20, 23]),
    dict(B=1, T=48, H=4, K=32, V=64, seed=18, cu=[0, 10, 24, 48], h0=True),
    dict(B=1, T=4, H=2, K=16, V=32, seed=20, cu=[0, 1, 2, 3, 4]),
    dict(B=1, T=67, H=2, K=32, V=64, seed=25, cu=[0, 3, 67]),
    dict(B=1, T=23, H=2, K=16, V=32, seed=121, cu=[0, 7, 20, 23], reverse=True),
    dict(B=1, T=32, H=4, K=32, V=64, seed=131, gate="gk+gv", cu=[0, 16, 32]),
    dict(B=2, T=32, H=4, K=32, V=64, seed=133, gate="gk+gv", h0=True),
    dict(B=2, T=32, H=4, K=32, V=64, seed=136, gate="gk+gv", reverse=True),
    dict(B=1, T=256, H=2, K=32, V=64, seed=311, gate="gk+gv"),
    dict(B=1, T=256, H=4, K=32, V=64, seed=380, gate="gk+gv", h0=True, reverse=True,
         scale=0.1),
    dict(B=1, T=256, H=4, K=32, V=64, seed=381, gate="gk+gv", h0=True, cu=[0, 64, 180, 256]),
    dict(B=2, T=32, H=4, K=32, V=64, seed=402, dht=True, gate="gk+gv"),
    dict(B=2, T=32, H=4, K=32, V=64, seed=404, dht=True, reverse=True),
    dict(B=2, T=32, H=4, K=32, V=64, seed=411, h0=True, dht=False, gate="gk+gv"),
    dict(B=1, T=48, H=2, K=16, V=32, seed=421, gate="gv", dht=True, cu=[0, 10, 24, 48]),
    dict(B=1, T=48, H=2, K=16, V=32, seed=431, gate="gk+gv", h0=True, cu=[0, 10, 24, 48]),
    # shapes beyond the reference table: wide state (32-column tiles), rows > 256, odd K / V
    dict(B=1, T=64, H=2, K=256, V=512, seed=3, gate="gk+gv", h0=True, gate_div=16.0),
    dict(B=1, T=40, H=2, K=200, V=70, seed=4, gate="gk+gv", h0=True),
    dict(B=2, T=20, H=1, K=512, V=24, seed=5, dht=True),
    # empty sequences: dh0 = dht for them, no gradient through their (absent) tokens
    dict(B=1, T=23, H=2, K=16, V=32, seed=122, cu=[0, 0, 7, 7, 23], h0=True,
         gate="gk+gv"),
    # strong gates: direct stages in every scan (all or some of the stages)
    dict(B=1, T=100, H=2, K=32, V=64, seed=150, gate_mul=12.0, h0=True, dht=True),
    dict(B=1, T=200, H=2, K=64, V=64, seed=151, gate_mul=5.0, h0=True, dht=True),
    dict(B=1, T=100, H=2, K=32, V=64, seed=152, gate="gv", gate_mul=8.0, h0=True, dht=True),
]


def _bwd_inputs(cfg, dtype):
    q, k, v, gk, gv, s0, cu = _inputs(cfg, dtype)
    r = np.random.default_rng(cfg["seed"] + 1000)
    B, T, H, K, V = (cfg[x] for x in "BTHKV")
    N = len(cu) - 1 if cu else B
    do = r.standard_normal((B, T, H, V))
    if dtype == "bf16":
        do = round_bf16(do)
    use_dht = cfg.get("dht", cfg.get("h0", False))
    dht = r.standard_normal((N, H, K, V)) if use_dht else None
    return q, k, v, gk, gv, s0, cu, do, dht


def _close(name, got, ref):
    if ref is None:
        assert got is None, f"{name}: expected None"
        return
    assert got is not None and got.dtype == torch.float32, name
    check(name, to_np(got), ref, "f32")


def _bwd_id(c):
    s = _cid(c)
    if "dht" in c:
        s += "-dht" if c["dht"] else "-nodht"
    return s


@pytest.mark.parametrize("cfg", BWD_CASES, ids=[_bwd_id(c) for c in BWD_CASES])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_fused_recurrent_bwd(cfg, dtype):
    import tops.ops.gla as G

    q, k, v, gk, gv, s0, cu, do, dht = _bwd_inputs(cfg, dtype)
    d = lambda x: to_dev(x, dtype)  # noqa: E731
    cut = None if cu is None else torch.tensor(cu)
    kw = dict(scale=cfg.get("scale"), reverse=cfg.get("reverse", False))
    o = None
    if gv is not None:   # the reference test feeds the kernel's own forward output
        o, _ = G.fused_recurrent_gla(d(q), d(k), d(v), gk=d(gk), gv=d(gv),
                                     initial_state=to_dev(s0, "state"), cu_seqlens=cut, **kw)
    got = G.fused_recurrent_gla_bwd(d(q), d(k), d(v), gk=d(gk), gv=d(gv), o=o, do=d(do),
                                    dht=to_dev(dht, "state"), initial_state=to_dev(s0, "state"),
                                    cu_seqlens=cut, **kw)
    torch.cuda.synchronize()
    ref = orc.fused_recurrent_gla_bwd(q, k, v, gk=gk, gv=gv, do=do, dht=dht, initial_state=s0,
                                      cu_seqlens=cu, **kw)
    for name, g_, r_ in zip(("dq", "dk", "dv", "dgk", "dgv", "dh0"), got, ref):
        _close(name, g_, r_)


def test_fused_recurrent_autograd():
    """Gradients of sum(o * do) + sum(ht * dht) through fused_recurrent_gla's autodiff rule."""
    import tops.ops.gla as G

    cfg = dict(B=1, T=40, H=2, K=32, V=48, seed=77, gate="gk+gv", h0=True, cu=[0, 15, 40])
    q, k, v, gk, gv, s0, cu, do, dht = _bwd_inputs(cfg, "f32")
    leaf = lambda x: to_dev(x, "f32").requires_grad_(True)  # noqa: E731
    tq, tk, tv, tgk, tgv, th0 = (leaf(x) for x in (q, k, v, gk, gv, s0))
    o, ht = G.fused_recurrent_gla(tq, tk, tv, gk=tgk, gv=tgv, initial_state=th0,
                                  output_final_state=True, cu_seqlens=cu)
    loss = (o * to_dev(do, "f32")).sum() + (ht * to_dev(dht, "f32")).sum()
    loss.backward()
    ref = orc.fused_recurrent_gla_bwd(q, k, v, gk=gk, gv=gv, do=do, dht=dht, initial_state=s0,
                                      cu_seqlens=cu)
    for name, t, r_ in zip(("dq", "dk", "dv", "dgk", "dgv", "dh0"),
                           (tq, tk, tv, tgk, tgv, th0), ref):
        _close(name, t.grad, r_)


def test_fused_recurrent_bwd_c2_shape_slices():
    """Backward at the C2 shape (B8 T2048 H4 K256 V512, bf16, h0, dht): finite everywhere,
    and the full-length gradients of two (b, h) slices against the oracle."""
    import tops.ops.gla as G

    B, T, H, K, V = 8, 2048, 4, 256, 512
    gen = torch.Generator(device="cuda").manual_seed(5)
    mk = lambda *s: torch.randn(*s, generator=gen, device="cuda")  # noqa: E731
    q, k = (mk(B, T, H, K).to(torch.bfloat16) for _ in range(2))
    v, do = (mk(B, T, H, V).to(torch.bfloat16) for _ in range(2))
    gk = (torch.nn.functional.logsigmoid(mk(B, T, H, K)) / 16).to(torch.bfloat16)
    h0 = mk(B, H, K, V) * 0.1
    dht = mk(B, H, K, V) * 0.1
    got = G.fused_recurrent_gla_bwd(q, k, v, gk=gk, do=do, dht=dht, initial_state=h0)
    torch.cuda.synchronize()
    for g_ in got:
        assert g_ is None or torch.isfinite(g_).all()
    for b, h in [(0, 0), (7, 3)]:
        sl = lambda x: to_np(x[b:b + 1, :, h:h + 1])  # noqa: E731
        st = lambda x: to_np(x[b:b + 1, h:h + 1])  # noqa: E731
        # float32 oracle: its per-step gated states of one slice then take 1 GiB
        ref = orc.fused_recurrent_gla_bwd(sl(q), sl(k), sl(v), gk=sl(gk), do=sl(do),
                                          dht=st(dht), initial_state=st(h0), dtype=np.float32)
        for name, g_, r_ in zip(("dq", "dk", "dv", "dgk", "dgv", "dh0"), got, ref):
            if r_ is not None:
                gs = st(g_) if name == "dh0" else sl(g_)
                # dgk: a reverse cumsum over 2048 steps of terms of order 10
                check(name, gs, r_, "f32",
                      rel_f32="reverse cumsum over 2048 steps" if name == "dgk" else None)


def test_non_contiguous_inputs():
    """Strided views (the layer's split projections) as inputs: the host layer's contiguous
    copies must stay alive until the kernels are enqueued (regression: temporaries passed as
    device pointers were freed and their memory reused by the next copy)."""
    import tops.ops.gla as G

    r = np.random.default_rng(77)
    B, T, H, K, V = 2, 40, 2, 16, 32
    big = r.standard_normal((B, T, H, 2 * K + V + K)).astype(np.float32)
    q, k, v, gk = (big[..., :K], big[..., K:2 * K], big[..., 2 * K:2 * K + V],
                   logsigmoid(big[..., 2 * K + V:]))
    s0 = r.standard_normal((B, H, K, V))
    d = torch.tensor(big).cuda()
    dq, dk, dv = d[..., :K], d[..., K:2 * K], d[..., 2 * K:2 * K + V]
    dg = torch.nn.functional.logsigmoid(d[..., 2 * K + V:])
    assert not dq.is_contiguous()
    o, ht = G.fused_recurrent_gla(dq, dk, dv, gk=dg, initial_state=to_dev(s0, "state"),
                                  output_final_state=True)
    torch.cuda.synchronize()
    on, hn = orc.fused_recurrent_gla(q, k, v, gk=gk, initial_state=s0, output_final_state=True)
    check("o", to_np(o), on, "f32")
    check("ht", to_np(ht), hn, "f32")
