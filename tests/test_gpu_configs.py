"""GPU parity at the benchmark configurations' full sizes (BASELINE configs C3 and C5), and
the reference-written layer fixtures on the HIP layer.

* C3: ``chunk_gla`` forward, bf16, B8 T4096 H4 K256 V512, chunk 64, h0 ~ N(0, 0.1^2)
  (reference ``tops/ops/gla/chunk.py:1083-1179``): every output finite at full size, two
  full-length (b, h) slices of o and ht against the oracle.
* C5: ``GatedLinearAttention`` forward + backward, bf16, B2 T16384, hidden 2048, 4 heads,
  expand_k 0.5 (K = 256), expand_v 1 (V = 512), gate rank 16, normalizer 16, weights ~ N(0,
  0.02), x ~ N(0, 1), loss = sum(out * probe) (reference ``tops/layers/gla.py:208-345``): every
  output and parameter gradient finite; the output on a causal prefix of 512 tokens against
  the layer oracle on the same weights; the attention core's dq / dk / dv / dg on two (b, h)
  slices against the oracle's ``chunk_gla_bwd`` given the core's own inputs and upstream
  gradient (captured from the layer run), and the core's o, dq, dk, dv, dg on all 8 slices
  against the float32 torch chunked GLA (``tests/torch_ref.py``) from the same inputs; the
  whole layer at full size (output, input gradient and every parameter gradient) against
  a float32 reference on the GPU: the layer oracle's composition (``oracle/layer.py``) with
  the chunked torch recurrence in place of its step loop, from the same bf16 weights.
* Reference fixtures (``tests/golden/gla_layer.npz``, written by the reference's torch CPU
  layer): the float32 HIP layer's output and gradients.

Bars: bf16 max-abs error / max |ref| <= 2e-2; float32 max-abs error <= 1e-4.
"""

import os
import sys

import numpy as np
import pytest
import torch

import oracle as orc
from gla_cases import check, to_np

pytestmark = pytest.mark.gpu

torch.backends.cuda.matmul.allow_tf32 = False

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))


def _say(*a):
    print(*a, flush=True)


def test_c3_chunk_gla_fwd_full_size():
    import tops.ops.gla as G

    B, T, H, K, V = 8, 4096, 4, 256, 512
    _say(f"C3 chunk_gla fwd B{B} T{T} H{H} K{K} V{V}")
    gen = torch.Generator(device="cuda").manual_seed(3)
    mk = lambda *s: torch.randn(*s, generator=gen, device="cuda")  # noqa: E731
    q, k = (mk(B, T, H, K).to(torch.bfloat16) for _ in range(2))
    v = mk(B, T, H, V).to(torch.bfloat16)
    g = (torch.nn.functional.logsigmoid(mk(B, T, H, K)) / 16).to(torch.bfloat16)
    h0 = mk(B, H, K, V) * 0.1
    o, ht = G.chunk_gla(q, k, v, g, initial_state=h0, output_final_state=True, chunk_size=64)
    torch.cuda.synchronize()
    assert o.shape == (B, T, H, V) and o.dtype == torch.bfloat16
    assert ht.shape == (B, H, K, V) and ht.dtype == torch.float32
    assert torch.isfinite(o.float()).all() and torch.isfinite(ht).all()
    for b, h in [(0, 0), (7, 3), (4, 1)]:
        sl = lambda x: to_np(x[b:b + 1, :, h:h + 1])  # noqa: E731
        on, hn = orc.chunk_gla(sl(q), sl(k), sl(v), sl(g), initial_state=to_np(h0[b:b + 1, h:h + 1]),
                               output_final_state=True, chunk_size=64, dtype=np.float32)
        check(f"o[{b},{h}]", sl(o), on, "bf16")
        check(f"ht[{b},{h}]", to_np(ht[b:b + 1, h:h + 1]), hn, "bf16")
        _say(f"  slice ({b}, {h}) ok")


def test_c3_all_slices_vs_torch_fp32():
    """C3 at full size, all 32 (b, h) slices of o and ht against the float32 torch chunked
    GLA (``tests/torch_ref.py``, pinned to the oracle by ``test_torch_ref.py``) on the GPU from
    the same bf16 inputs. Bar per slice: max-abs error / max |ref| <= 2e-2."""
    import tops.ops.gla as G
    from gla_cases import BF16_RTOL_MAX
    from torch_ref import chunk_gla_torch, slice_errors

    B, T, H, K, V = 8, 4096, 4, 256, 512
    _say(f"C3 chunk_gla fwd B{B} T{T} H{H} K{K} V{V}, all slices vs torch fp32")
    gen = torch.Generator(device="cuda").manual_seed(33)
    mk = lambda *s: torch.randn(*s, generator=gen, device="cuda")  # noqa: E731
    q, k = (mk(B, T, H, K).to(torch.bfloat16) for _ in range(2))
    v = mk(B, T, H, V).to(torch.bfloat16)
    g = (torch.nn.functional.logsigmoid(mk(B, T, H, K)) / 16).to(torch.bfloat16)
    h0 = mk(B, H, K, V) * 0.1
    o, ht = G.chunk_gla(q, k, v, g, initial_state=h0, output_final_state=True, chunk_size=64)
    with torch.no_grad():
        ro, rht = chunk_gla_torch(q.float(), k.float(), v.float(), g.float(), h0,
                                  chunk_size=64)
    torch.cuda.synchronize()
    for name, x, r, tm in (("o", o, ro, True), ("ht", ht, rht, False)):
        err, scale = slice_errors(x, r, tm)
        worst = float((err / scale.clamp_min(1e-30)).max())
        _say(f"  {name}: worst slice error/max|ref| {worst:.3e}")
        assert worst <= BF16_RTOL_MAX, name


def test_c5_layer_fwd_bwd_full_size():
    from oracle import layer as L
    from tops.layers import GatedLinearAttention
    import tops.layers.gla as layer_mod

    B, T, D, H = 2, 16384, 2048, 4
    cfg = dict(hidden_size=D, num_heads=H, expand_k=0.5, expand_v=1.0, gate_low_rank_dim=16,
               gate_logit_normalizer=16)
    _say(f"C5 GatedLinearAttention fwd+bwd B{B} T{T} hidden {D} heads {H}")
    m = GatedLinearAttention(rngs=5, dtype=torch.bfloat16, **cfg).cuda()
    gen = torch.Generator(device="cuda").manual_seed(5)
    with torch.no_grad():
        for _, p in m.named_parameters():
            p.copy_(torch.randn(p.shape, generator=gen, device="cuda") * 0.02)
    x = torch.randn(B, T, D, generator=gen, device="cuda").to(torch.bfloat16)
    probe = torch.randn(B, T, D, generator=gen, device="cuda")
    core = {}
    real = layer_mod.chunk_gla

    def spy(q, k, v, g, **kw):   # the attention core's inputs and output, gradients kept
        for name, t in (("q", q), ("k", k), ("v", v), ("g", g)):
            t.retain_grad()
            core[name] = t
        o, s = real(q, k, v, g, **kw)
        o.retain_grad()
        core["o"], core["chunk_size"] = o, kw.get("chunk_size")
        return o, s

    layer_mod.chunk_gla = spy
    try:
        xd = x.clone().requires_grad_(True)
        out, _, _ = m(xd)
        (out.float() * probe).sum().backward()
    finally:
        layer_mod.chunk_gla = real
    torch.cuda.synchronize()
    assert "o" in core, "the layer did not run the chunked core"
    assert out.shape == (B, T, D)
    assert torch.isfinite(out.float()).all() and torch.isfinite(xd.grad.float()).all()
    for n, p in m.named_parameters():
        assert p.grad is not None and torch.isfinite(p.grad.float()).all(), n
    _say("  full-size outputs and gradients finite")
    # causal prefix against the layer oracle (float64, same bf16 weights and input)
    P = 512
    params = {n: p.detach().to("cpu", torch.float64) for n, p in m.named_parameters()}
    oref, _ = L.gla_layer(params, x[:, :P].to("cpu", torch.float64), cfg)
    check("out[:, :512]", to_np(out[:, :P]), oref.numpy(), "bf16")
    _say("  prefix output ok")
    # the core's gradients on two (b, h) slices
    K, V = D // 2 // H, D // H
    for b, h in [(0, 0), (1, 3)]:
        sl = lambda x: to_np(x[b:b + 1, :, h:h + 1])  # noqa: E731
        qn, kn, vn, gn = (sl(core[n]) for n in ("q", "k", "v", "g"))
        don = sl(core["o"].grad)
        ref = orc.chunk_gla_bwd(qn, kn, vn, gn, None, None, K ** -0.5, None, None, None, don,
                                None, chunk_size=64, dtype=np.float32)
        for name, r in zip(["q", "k", "v", "g"], ref):
            check(f"d{name}[{b},{h}]", sl(core[name].grad), r, "bf16")
        _say(f"  core slice ({b}, {h}) ok")
    assert core["q"].shape == (B, T, H, K) and core["v"].shape == (B, T, H, V)
    # the core's output and gradients on all 8 (b, h) slices against the float32 torch
    # chunked GLA (tests/torch_ref.py) from the same inputs and upstream gradient
    from gla_cases import BF16_RTOL_MAX
    from torch_ref import chunk_gla_torch, slice_errors

    refs = [core[n].detach().float().requires_grad_() for n in ("q", "k", "v", "g")]
    ro, _ = chunk_gla_torch(*refs, chunk_size=64)
    ro.backward(core["o"].grad.float())
    pairs = [("o", core["o"], ro)] + [(f"d{n}", core[n].grad, r.grad)
                                      for n, r in zip(("q", "k", "v", "g"), refs)]
    for name, got, r in pairs:
        err, scale = slice_errors(got, r, True)
        worst = float((err / scale.clamp_min(1e-30)).max())
        _say(f"  core {name}, all slices: worst error/max|ref| {worst:.3e}")
        assert worst <= BF16_RTOL_MAX, name
    del refs, ro, pairs
    # the whole layer at full size against a float32 reference on the GPU (the oracle's
    # composition with the chunked torch recurrence, pinned by tests/test_torch_ref.py):
    # output, input gradient and every parameter gradient, each at the bf16 bar
    def chunk_recurrence(q, k, v, g, scale, initial_state=None, cu_seqlens=None):
        assert cu_seqlens is None
        return chunk_gla_torch(q, k, v, g, initial_state, scale=scale, chunk_size=64)

    refp = {n: p.detach().float().requires_grad_() for n, p in m.named_parameters()}
    xr = x.detach().float().requires_grad_()
    oref_full, _ = L.gla_layer(refp, xr, cfg, recurrence_fn=chunk_recurrence)
    (oref_full * probe).sum().backward()
    torch.cuda.synchronize()
    full = [("out", out, oref_full), ("d_x", xd.grad, xr.grad)] + [
        (f"d_{n}", p.grad, refp[n].grad) for n, p in m.named_parameters()]
    for name, got, r in full:
        err = float((got.detach().float() - r.detach()).abs().max())
        scale = float(r.detach().abs().max())
        _say(f"  full layer {name}: error/max|ref| {err / max(scale, 1e-30):.3e}")
        assert err <= BF16_RTOL_MAX * scale, name


def _layer_cases():
    from layer_cases import CASES

    return list(CASES)


@pytest.mark.parametrize("case", _layer_cases())
def test_layer_matches_reference_fixture(case):
    from layer_cases import CASES, full_kwargs, make_io, make_params
    from tops.layers import GatedLinearAttention

    kw, B, T, seed, grads, cu = CASES[case]
    ckw = full_kwargs(kw)
    fx = np.load(os.path.join(HERE, "golden", "gla_layer.npz"))
    m = GatedLinearAttention(**ckw).cuda()
    shapes = {n: tuple(p.shape) for n, p in m.named_parameters()}
    vals = make_params(seed, shapes)
    with torch.no_grad():
        for n, p in m.named_parameters():
            p.copy_(torch.from_numpy(vals[n]))
    x, probe = make_io(seed, B, T, ckw["hidden_size"])
    xd = torch.from_numpy(x).cuda().requires_grad_(grads)
    out, _, _ = m(xd, cu_seqlens=cu)

    def close(name, got, ref):
        # parameter gradients sum over every token of the batch (projections on hipBLASLt)
        check(name, to_np(got), ref, "f32",
              rel_f32="sum over the batch's tokens" if name.startswith("d_") and
              name != "d_x" else None)

    close("out", out, fx[f"{case}/out"])
    if grads:
        (out * torch.from_numpy(probe).cuda()).sum().backward()
        close("d_x", xd.grad, fx[f"{case}/d_x"])
        for n, p in m.named_parameters():
            close(f"d_{n}", p.grad, fx[f"{case}/d_{n}"])
