"""GPU: chunked GLA on tensors past 2^31 elements (4 GiB of bf16 per tensor).

The C ABI takes up to 2^31 - 1 tokens, so q, k, v, g and the per-chunk states may hold many
more than 2^31 elements; every kernel forms its global offsets from 64-bit bases. Here a
varlen batch of filler sequences places one test sequence across the 2^31-element offset
of q (and of the per-chunk states behind it). The test sequence's output, final state and
every gradient (dq, dk, dv, dg, dh0) must equal, bit for bit, a call over copies of that
sequence alone: the same chunks run through the same kernels, and a block's arithmetic does
not depend on where its sequence sits. Three paths: the fused full-head kernels (K = V = 128),
the wide heads' per-chunk backward (K = 256) and the recurrent scans (float32 output and
gradients, 8 GiB each). Skipped where the GPU lacks the memory.
"""

import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu

CASES = [
    # H, K, V; filler sequences; test sequence length; GiB of device memory needed
    dict(op="chunk", H=8, K=128, V=128, nfill=64, tlen=300, need=64),
    dict(op="chunk", H=2, K=256, V=256, nfill=64, tlen=300, need=112),
    dict(op="recurrent", H=8, K=128, V=128, nfill=64, tlen=300, need=112),
]


@pytest.fixture(autouse=True)
def _release_cache():
    """Hand the cached blocks back after each case (tens of GiB), for the tests after it."""
    yield
    torch.cuda.empty_cache()


def _cid(c):
    return f"{c['op']}-H{c['H']}K{c['K']}V{c['V']}"


def _inputs(T, H, K, V, N, gen, do_dtype):
    dev = torch.device("cuda:0")
    bf = torch.bfloat16

    def rn(*shape, dtype=bf):
        return torch.randn(*shape, dtype=dtype, device=dev, generator=gen)

    q, k, v = rn(1, T, H, K), rn(1, T, H, K), rn(1, T, H, V)
    g = F.logsigmoid(rn(1, T, H, K)) / 16
    h0 = rn(N, H, K, V, dtype=torch.float32)
    do, dht = rn(1, T, H, V, dtype=do_dtype), rn(N, H, K, V, dtype=torch.float32)
    return q, k, v, g, h0, do, dht


def _run(op, q, k, v, g, h0, do, dht, cu):
    import tops.ops.gla as G

    xs = [t.requires_grad_(True) for t in (q, k, v, g, h0)]
    if op == "chunk":
        o, ht = G.chunk_gla(*xs[:4], initial_state=xs[4], output_final_state=True,
                            cu_seqlens=torch.tensor(cu), chunk_size=64)
    else:
        o, ht = G.fused_recurrent_gla(*xs[:3], gk=xs[3], initial_state=xs[4],
                                      output_final_state=True, cu_seqlens=torch.tensor(cu))
    grads = torch.autograd.grad((o, ht), xs, (do, dht))
    torch.cuda.synchronize()
    return [o.detach(), ht.detach()] + list(grads)


@pytest.mark.parametrize("c", CASES, ids=[_cid(c) for c in CASES])
def test_past_2_31_elements(c):
    H, K, V = c["H"], c["K"], c["V"]
    torch.cuda.empty_cache()   # blocks cached by earlier tests count as used
    free, _ = torch.cuda.mem_get_info(0)
    if free < c["need"] * 2**30:
        pytest.skip(f"needs {c['need']} GiB of free device memory, {free / 2**30:.0f} free")
    tb = 2**31 // (H * K)          # first token whose q elements start at or past 2^31
    start = tb - 100               # the test sequence begins 100 tokens before it
    L = start // c["nfill"]
    lens = [L] * (c["nfill"] - 1) + [start - L * (c["nfill"] - 1)]
    cu = [0]
    for n in lens + [c["tlen"]]:
        cu.append(cu[-1] + n)
    T, N = cu[-1], len(cu) - 1
    assert cu[-2] == start and (T - 1) * H * K >= 2**31
    gen = torch.Generator(device="cuda:0").manual_seed(2024)
    # the recurrent scans write a float32 output, so its gradient comes in float32
    do_dtype = torch.bfloat16 if c["op"] == "chunk" else torch.float32
    q, k, v, g, h0, do, dht = _inputs(T, H, K, V, N, gen, do_dtype)
    big = _run(c["op"], q, k, v, g, h0, do, dht, cu)
    a, b, n = start, T, c["tlen"]
    # the test sequence's slices: tokens [a, b) of the per-token tensors, the last state
    tok = lambda t: t[:, a:b].clone()
    last = lambda t: t[N - 1:].clone()
    # the check runs COPIES copies of the sequence, so that the launchers that size their
    # tiles by the grid (the recurrent scans: 64-column tiles from 256 blocks up, 32-column
    # ones below, with another order of the output's fp32 sums) pick the big call's; the
    # first copy is compared
    COPIES = 32
    rep = lambda t: t.repeat(1, COPIES, 1, 1)
    rep_s = lambda t: t.repeat(COPIES, 1, 1, 1)
    small = _run(c["op"], rep(tok(q)), rep(tok(k)), rep(tok(v)), rep(tok(g)), rep_s(last(h0)),
                 rep(tok(do)), rep_s(last(dht)), [i * n for i in range(COPIES + 1)])
    names = ["o", "ht", "dq", "dk", "dv", "dg", "dh0"]
    picks = [tok, last, tok, tok, tok, tok, last]
    firsts = [lambda t: t[:, :n]] + [lambda t: t[:1]] + [lambda t: t[:, :n]] * 4 + [lambda t: t[:1]]
    for name, pick, first, x, y in zip(names, picks, firsts, big, small):
        xs, ys = pick(x), first(y)
        assert torch.isfinite(xs.float()).all(), name
        assert torch.equal(xs, ys), (name, (xs.float() - ys.float()).abs().max().item())


FIXED = [
    # H, K, V; GiB of device memory needed (both calls' outputs and one call's workspaces)
    dict(H=8, K=128, V=128, need=96),    # fused full-head kernels
    dict(H=2, K=256, V=512, need=200),   # wide heads: the per-chunk gating workspace path
]


@pytest.mark.parametrize("c", FIXED, ids=[f"H{c['H']}K{c['K']}V{c['V']}" for c in FIXED])
def test_past_2_31_elements_fixed_length(c):
    """The fixed-length call (segmented: every (sequence, head) cut into segments whose entry
    states come from a segment pass; wide heads also stream the per-chunk gating workspace) on
    one sequence whose q, k, g pass 2^31 elements by 300 tokens, against the same sequence as a
    varlen call (one segment walked in order; wide heads gate in every V tile's block): the
    entry states are summed in another order and the wide forward takes another factoring, so
    the two agree to the bf16 bar (max-abs error / max |ref| <= 2e-2) and, for the float32
    final state and dh0, to 1e-4 relative."""
    H, K, V = c["H"], c["K"], c["V"]
    torch.cuda.empty_cache()   # blocks cached by earlier tests count as used
    free, _ = torch.cuda.mem_get_info(0)
    if free < c["need"] * 2**30:
        pytest.skip(f"needs {c['need']} GiB of free device memory, {free / 2**30:.0f} free")
    T = 2**31 // (H * K) + 300
    gen = torch.Generator(device="cuda:0").manual_seed(2025)
    q, k, v, g, h0, do, dht = _inputs(T, H, K, V, 1, gen, torch.bfloat16)
    import tops.ops.gla as G

    def run(cu):
        xs = [t.detach().requires_grad_(True) for t in (q, k, v, g, h0)]
        o, ht = G.chunk_gla(*xs[:4], initial_state=xs[4], output_final_state=True,
                            cu_seqlens=None if cu is None else torch.tensor(cu), chunk_size=64)
        grads = torch.autograd.grad((o, ht), xs, (do, dht))
        torch.cuda.synchronize()
        return [o.detach(), ht.detach()] + list(grads)

    fixed = run(None)
    ref = run([0, T])
    names = ["o", "ht", "dq", "dk", "dv", "dg", "dh0"]
    for name, x, y in zip(names, fixed, ref):
        assert torch.isfinite(x.float()).all(), name
        err = (x.float() - y.float()).abs().max().item() / y.float().abs().max().item()
        bar = 1e-4 if x.dtype == torch.float32 else 2e-2
        print(f"{name}: error / max |ref| {err:.2e} (bar {bar})", flush=True)
        assert err <= bar, (name, err)
