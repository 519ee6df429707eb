"""GPU parity: the GLA layer and its modules vs the float64 torch restatement in
``oracle/layer.py`` (forward and, through autograd, every gradient).

Mirrors ``tests/layers/test_gla.py`` (layer configs: hidden 64..256, heads 2..4, GQA, short
conv, output gate on / off, fused / unfused norm, feature map, clamp_min, affine on / off;
RMSNorm / FusedRMSNormGated / ShortConvolution checks), adding the backward the reference
does not test. Tolerances: float32 max-abs <= 2e-3 x max(1, |ref|) for the layer (the
reference's layer bar is 5e-4..2e-3), 1e-5 for the modules; bfloat16 relative 2e-2.
"""

import numpy as np
import pytest
import torch

from gla_cases import check

pytestmark = pytest.mark.gpu

torch.backends.cuda.matmul.allow_tf32 = False


def _f64(t):
    return t.detach().to("cpu", torch.float64)


def _close(name, got, ref, tol):
    got = got.detach().double().cpu().numpy()
    ref = ref.detach().double().cpu().numpy()
    check(name, got, ref, "f32", atol=tol * max(1.0, float(np.abs(ref).max())))


# D: rows of one 512-feature piece in registers, of two, and in 1024-feature slabs (the
# backward's three builds)
@pytest.mark.parametrize("D", [64, 768, 1536])
@pytest.mark.parametrize("affine", [True, False])
@pytest.mark.parametrize("gated", [True, False])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rmsnorm_gated(affine, gated, dtype, D):
    from oracle import layer as L
    from tops.modules import FusedRMSNormGated, RMSNorm

    gen = torch.Generator().manual_seed(5)
    x = torch.randn(3, 37, D, generator=gen)
    g = torch.randn(3, 37, D, generator=gen)
    dy = torch.randn(3, 37, D, generator=gen)
    m = (FusedRMSNormGated(D, affine) if gated else RMSNorm(D, affine)).cuda()
    if affine:
        with torch.no_grad():
            m.weight.copy_(torch.rand(D, generator=gen) + 0.5)
    xd = x.to(dtype).cuda().requires_grad_(True)
    gd = g.to(dtype).cuda().requires_grad_(True)
    y = m(xd, gd) if gated else m(xd)
    y.backward(dy.to(dtype).cuda())
    xr = _f64(xd).requires_grad_(True)
    gr = _f64(gd).requires_grad_(True)
    wr = _f64(m.weight).requires_grad_(True) if affine else None
    yr = L.rms_norm(xr, wr, 1e-5, gr if gated else None)
    yr.backward(_f64(dy.to(dtype)))
    if dtype == torch.float32:
        tol = 1e-5
        _close("y", y, yr, tol)
        _close("dx", xd.grad, xr.grad, tol)
        if gated:
            _close("dg", gd.grad, gr.grad, tol)
        if affine:
            _close("dw", m.weight.grad, wr.grad, 1e-4)
    else:
        check("y", y.detach().float().cpu().numpy(), yr.detach().numpy(), "bf16")
        check("dx", xd.grad.float().cpu().numpy(), xr.grad.numpy(), "bf16")
        if gated:
            check("dg", gd.grad.float().cpu().numpy(), gr.grad.numpy(), "bf16")
        if affine:
            check("dw", m.weight.grad.cpu().numpy(), wr.grad.numpy(), "bf16")


@pytest.mark.parametrize("clamp", [None, -0.05])
def test_gate_logsigmoid(clamp):
    from oracle import layer as L
    from tops.modules._norm import GateLogSigmoidFn

    gen = torch.Generator().manual_seed(6)
    x = torch.randn(4, 33, 3, 16, generator=gen) * 4
    dy = torch.randn(4, 33, 3, 16, generator=gen)
    xd = x.cuda().requires_grad_(True)
    y = GateLogSigmoidFn.apply(xd, 16, clamp)
    y.backward(dy.cuda())
    xr = x.double().requires_grad_(True)
    yr = L.gate_logsigmoid(xr, 16, clamp)
    yr.backward(dy.double())
    _close("y", y, yr, 1e-6)
    _close("dx", xd.grad, xr.grad, 1e-6)


@pytest.mark.parametrize("case", [
    dict(D=64, W=4, T=50, B=2, bias=False, act="silu"),
    dict(D=32, W=4, T=16, B=1, bias=True, act=None),
    dict(D=96, W=3, T=23, B=1, bias=True, act="silu", cu=[0, 7, 20, 23]),
    dict(D=128, W=8, T=70, B=3, bias=False, act="silu"),
])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_short_conv(case, dtype):
    from oracle import layer as L
    from tops.modules import ShortConvolution

    D, W, T, B = case["D"], case["W"], case["T"], case["B"]
    cu = case.get("cu")
    gen = torch.Generator().manual_seed(7)
    m = ShortConvolution(D, W, bias=case["bias"], activation=case["act"], rngs=3).cuda()
    x = torch.randn(B, T, D, generator=gen)
    dy = torch.randn(B, T, D, generator=gen)
    xd = x.to(dtype).cuda().requires_grad_(True)
    y, fs = m(xd, output_final_state=True, cu_seqlens=cu)
    y.backward(dy.to(dtype).cuda())
    xr = _f64(xd).requires_grad_(True)
    wr = _f64(m.weight).requires_grad_(True)
    br = _f64(m.bias).requires_grad_(True) if case["bias"] else None
    yr = L.short_conv(xr, wr, br, case["act"], cu)
    yr.backward(_f64(dy.to(dtype)))
    if dtype == torch.float32:
        _close("y", y, yr, 1e-5)
        _close("dx", xd.grad, xr.grad, 1e-5)
        _close("dw", m.weight.grad, wr.grad, 1e-4)
        if case["bias"]:
            _close("db", m.bias.grad, br.grad, 1e-4)
    else:
        check("y", y.detach().float().cpu().numpy(), yr.detach().numpy(), "bf16")
        check("dx", xd.grad.float().cpu().numpy(), xr.grad.numpy(), "bf16")
        check("dw", m.weight.grad.float().cpu().numpy(), wr.grad.numpy(), "bf16")
    segs = [(0, a, b) for a, b in zip(cu, cu[1:])] if cu else [(i, 0, T) for i in range(B)]
    for i, (b, a, e) in enumerate(segs):   # last W inputs of each sequence, zero padded
        want = torch.zeros(W, D)
        n = min(W, e - a)
        want[W - n:] = x[b, e - n:e].to(dtype).float()
        assert torch.equal(fs[i].float().cpu(), want)


LAYER_CASES = [
    dict(B=2, T=100, hidden_size=128, num_heads=4),
    dict(B=2, T=40, hidden_size=128, num_heads=4),                    # q_len <= 64: recurrent
    dict(B=1, T=96, hidden_size=128, num_heads=4, num_kv_heads=2),
    dict(B=1, T=80, hidden_size=128, num_heads=2, use_short_conv=True, conv_bias=True),
    dict(B=1, T=72, hidden_size=64, num_heads=2, use_output_gate=False),
    dict(B=1, T=72, hidden_size=64, num_heads=2, fuse_norm=False, gate_fn="swish"),
    dict(B=1, T=90, hidden_size=64, num_heads=2, feature_map="relu", clamp_min=-0.1),
    dict(B=1, T=70, hidden_size=128, num_heads=4, elementwise_affine=False),
    dict(B=1, T=3, hidden_size=64, num_heads=2),
    dict(B=1, T=130, hidden_size=128, num_heads=4, mode="fused_chunk", cu=[0, 50, 130]),
]


def _layer_id(c):
    return "-".join(f"{k}{v}" for k, v in c.items() if k not in ("B",)).replace(" ", "")


@pytest.mark.parametrize("cfg", LAYER_CASES, ids=[_layer_id(c) for c in LAYER_CASES])
def test_gla_layer_fwd_bwd(cfg):
    from oracle import layer as L
    from tops.layers import GatedLinearAttention

    cfg = dict(cfg)
    B, T = cfg.pop("B"), cfg.pop("T")
    cu = cfg.pop("cu", None)
    m = GatedLinearAttention(rngs=11, **cfg).cuda()
    gen = torch.Generator().manual_seed(12)
    with torch.no_grad():   # non-trivial norm weights and gate biases
        for name, p in m.named_parameters():
            if name.endswith("norm_swish_gate.weight") or name.endswith("g_norm.weight") \
                    or name.endswith(".bias"):
                p.copy_(torch.rand(p.shape, generator=gen) + 0.5)
    x = torch.randn(B, T, cfg["hidden_size"], generator=gen)
    probe = torch.randn(B, T, cfg["hidden_size"], generator=gen)
    xd = x.cuda().requires_grad_(True)
    o, _, _ = m(xd, cu_seqlens=cu)
    (o * probe.cuda()).sum().backward()
    params = {n: _f64(p).requires_grad_(True) for n, p in m.named_parameters()}
    xr = x.double().requires_grad_(True)
    orf, _ = L.gla_layer(params, xr, cfg, cu_seqlens=cu)
    (orf * probe.double()).sum().backward()
    tol = 2e-3
    _close("o", o, orf, tol)
    _close("dx", xd.grad, xr.grad, tol)
    for n, p in m.named_parameters():
        _close("d" + n, p.grad, params[n].grad, tol)


def test_gla_layer_bf16_full_head_path():
    """bf16 layer (head dims 64 / 128: the full-head chunk kernels) against the float64
    restatement on the same bf16 parameters and input."""
    from oracle import layer as L
    from tops.layers import GatedLinearAttention

    cfg = dict(hidden_size=256, num_heads=2)
    m = GatedLinearAttention(rngs=13, dtype=torch.bfloat16, **cfg).cuda()
    gen = torch.Generator().manual_seed(14)
    x = torch.randn(2, 256, 256, generator=gen).to(torch.bfloat16)
    probe = torch.randn(2, 256, 256, generator=gen)
    xd = x.cuda().requires_grad_(True)
    o, _, _ = m(xd)
    (o.float() * probe.cuda()).sum().backward()
    params = {n: _f64(p).requires_grad_(True) for n, p in m.named_parameters()}
    xr = x.double().requires_grad_(True)
    orf, _ = L.gla_layer(params, xr, cfg)
    (orf * probe.double()).sum().backward()
    check("o", o.detach().float().cpu().numpy(), orf.detach().numpy(), "bf16")
    check("dx", xd.grad.float().cpu().numpy(), xr.grad.numpy(), "bf16")
    for n, p in m.named_parameters():
        check("d" + n, p.grad.float().cpu().numpy(), params[n].grad.numpy(), "bf16")


def test_gla_layer_cache_decode():
    """use_cache: a prefill then single-token steps equal one pass over the whole sequence
    (recurrent state and short-conv windows carried in the cache)."""
    from tops.layers import GatedLinearAttention
    from tops.layers.gla import LayerCache

    m = GatedLinearAttention(hidden_size=64, num_heads=2, use_short_conv=True, layer_idx=0,
                             rngs=15).cuda()
    gen = torch.Generator().manual_seed(16)
    x = torch.randn(2, 12, 64, generator=gen).cuda()
    with torch.no_grad():
        full, _, _ = m(x)
        cache = LayerCache()
        first, _, cache = m(x[:, :9], past_key_values=cache, use_cache=True)
        steps = [first]
        for t in range(9, 12):
            y, _, cache = m(x[:, t:t + 1], past_key_values=cache, use_cache=True)
            steps.append(y)
    _close("o", torch.cat(steps, 1), full, 1e-4)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_concat_cols_matches_torch_cat(dtype):
    """The library's row-wise concatenation (the layer's grouped projection backward) against
    torch.cat: widths of 8 / 16-byte multiples, one to eight sources, a partial last block."""
    from tops.layers.gla import _concat_cols

    gen = torch.Generator(device="cuda").manual_seed(3)
    w8 = 8 if dtype == torch.bfloat16 else 4    # 16 bytes
    for widths in ([1024, 1024, 2048, 2048], [w8], [w8 * k for k in range(1, 9)]):
        ts = [torch.randn(1237, w, generator=gen, device="cuda").to(dtype) for w in widths]
        got = _concat_cols(ts)
        assert torch.equal(got, torch.cat(ts, 1))
    # a width that is no 16-byte multiple takes torch.cat
    ts = [torch.randn(5, 3, device="cuda").to(dtype), torch.randn(5, w8, device="cuda").to(dtype)]
    assert torch.equal(_concat_cols(ts), torch.cat(ts, 1))
