"""Host-side pieces of the GLA layer that need no GPU: the fan-out projection node against
separate ``F.linear`` calls (forward values and every gradient, float64 on the CPU)."""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "pallas-kernel_amd"))


@pytest.mark.parametrize("widths", [(16, 32, 40, 4), (96, 16, 80, 128)])
@pytest.mark.parametrize("unused", [None, 1])
def test_fanout_linear_matches_separate_linears(unused, widths):
    import torch
    import torch.nn.functional as F

    from tops.layers.gla import _FanOutLinear

    gen = torch.Generator().manual_seed(0)
    x = torch.randn(3, 7, 32, generator=gen, dtype=torch.float64, requires_grad=True)
    # output widths below, at and above the input's (the narrow ones take the transposed
    # weight-gradient product; widths above 64 form the concatenated group)
    ws = [torch.randn(o, 32, generator=gen, dtype=torch.float64, requires_grad=True)
          for o in widths]
    ys = _FanOutLinear.apply(x, *ws)
    ref = [F.linear(x, w) for w in ws]
    for y, r in zip(ys, ref):
        assert torch.equal(y, r)
    keep = [i for i in range(len(ws)) if i != unused]   # an output left out of the loss
    dys = [torch.randn(ys[i].shape, generator=gen, dtype=torch.float64) for i in keep]
    got = torch.autograd.grad([ys[i] for i in keep], [x] + ws, dys, allow_unused=True)
    exp = torch.autograd.grad([ref[i] for i in keep], [x] + ws, dys, allow_unused=True)
    for i, (g, e) in enumerate(zip(got, exp)):
        if e is None:
            assert g is None or not g.abs().max() > 0, i
            continue
        assert torch.allclose(g, e, rtol=1e-12, atol=1e-12), i


@pytest.mark.parametrize("bias", [True, False])
@pytest.mark.parametrize("rows", [48, 32 * 512])
def test_narrow_linear_matches_linear(bias, rows):
    """The low-rank gate's second matrix: values and gradients against F.linear (float64);
    rows = 32 x 512 takes the split product over the rows, 48 the GEMM."""
    import torch
    import torch.nn.functional as F

    from tops.layers.gla import _NarrowLinear, _skinny_at_b

    gen = torch.Generator().manual_seed(1)
    x = torch.randn(rows, 16, generator=gen, dtype=torch.float64, requires_grad=True)
    w = torch.randn(40, 16, generator=gen, dtype=torch.float64, requires_grad=True)
    b = torch.randn(40, generator=gen, dtype=torch.float64, requires_grad=True) if bias else None
    y = _NarrowLinear.apply(x, w, b)
    r = F.linear(x, w, b)
    assert torch.allclose(y, r, rtol=1e-12, atol=1e-12)
    dy = torch.randn(y.shape, generator=gen, dtype=torch.float64)
    ins = [x, w] + ([b] if bias else [])
    got = torch.autograd.grad(y, ins, dy)
    exp = torch.autograd.grad(r, ins, dy)
    for g, e in zip(got, exp):
        assert torch.allclose(g, e, rtol=1e-10, atol=1e-10)
    assert (_skinny_at_b(x.detach(), dy) is None) == (rows == 48)


def test_fanout_narrow_output_split_product():
    """A fan-out output of 16 features over 32 x 512 rows takes the split product for its
    weight gradient."""
    import torch
    import torch.nn.functional as F

    from tops.layers.gla import _FanOutLinear

    gen = torch.Generator().manual_seed(2)
    x = torch.randn(32 * 512, 24, generator=gen, dtype=torch.float64, requires_grad=True)
    ws = [torch.randn(o, 24, generator=gen, dtype=torch.float64, requires_grad=True)
          for o in (16, 40)]
    ys = _FanOutLinear.apply(x, *ws)
    dys = [torch.randn(y.shape, generator=gen, dtype=torch.float64) for y in ys]
    got = torch.autograd.grad(ys, [x] + ws, dys)
    exp = torch.autograd.grad([F.linear(x, w) for w in ws], [x] + ws, dys)
    for g, e in zip(got, exp):
        assert torch.allclose(g, e, rtol=1e-10, atol=1e-10)
