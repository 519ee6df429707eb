"""tops_gla_chunk_fwd_noalloc (the segment workspace in the library's static device scratch)
against tops_gla_chunk_fwd with a caller workspace, through the C ABI: calls in a row, the
second on a smaller input (fewer sequences, heads and chunks: another segment plan in the
same scratch), the third with gates strong enough that every (sequence, head) pair takes
the gate-range fallback, whose flags live in the scratch (checked against the oracle too).
Both run the same kernels on the same segment plan, so the outputs (o, ht, the per-chunk
states h) are bit-identical."""

import pytest
import torch

import oracle as orc
from gla_cases import check, make_inputs, round_bf16, to_dev, to_np

pytestmark = pytest.mark.gpu


def _run(B, T, H, K, V, seed, gate_mul=None):
    from tops import _lib
    from tops._lib import SeqLayout, call, ptr, stream_of

    C = 64
    q, k, v, g, s0, _, _ = make_inputs(B, T, H, K, V, seed, gate_div=16.0, h0=True,
                                       dtype="bf16")
    if gate_mul is not None:   # per-token decays of about 4: every pair flagged
        g = round_bf16(g * 16.0 * gate_mul)
    qn, kn, vn, gn = q, k, v, g
    q, k, v, g = (to_dev(x, "bf16") for x in (q, k, v, g))
    h0 = to_dev(s0, "state")
    dev = q.device
    seq = SeqLayout(B, T, C, None, dev)
    st = stream_of(dev)
    ws, nws = _lib.seg_workspace(B, T, H, K, V, C, False, torch.bfloat16, dev)
    assert nws > 0, "the case must use sequence segments"
    outs = []
    for noalloc in (False, True):
        o = torch.full_like(v, float("nan"))
        ht = torch.full_like(h0, float("nan"))
        h = torch.full((seq.NC, H, K, V), float("nan"), dtype=q.dtype, device=dev)
        if noalloc:
            call("tops_gla_chunk_fwd_noalloc", ptr(q), ptr(k), ptr(v), ptr(g), ptr(h0), ptr(o),
                 ptr(ht), ptr(h), K ** -0.5, B, T, H, K, V, C, *seq.args(), _lib.BF16, st)
        else:
            call("tops_gla_chunk_fwd", ptr(q), ptr(k), ptr(v), ptr(g), ptr(h0), ptr(o),
                 ptr(ht), ptr(h), ptr(ws), nws, K ** -0.5, B, T, H, K, V, C, *seq.args(),
                 _lib.BF16, st)
        torch.cuda.synchronize()
        outs.append((o, ht, h))
    # the per-chunk states of flagged pairs are not meaningful (the gate-range fallback
    # rewrites o and ht only)
    names = ("o", "ht") if gate_mul is not None else ("o", "ht", "h")
    for name, a, b in zip(names, *outs):
        assert torch.isfinite(a.float()).all(), name
        assert torch.equal(a, b), f"{name}: max diff {(a.float() - b.float()).abs().max()}"
    if gate_mul is not None:
        on, hn = orc.naive_recurrent_gla(qn, kn, vn, gn, initial_state=s0,
                                         output_final_state=True)
        check("o", to_np(outs[1][0]), on, "bf16")
        check("ht", to_np(outs[1][1]), hn, "bf16")


def test_noalloc_forward_matches_workspace_forward_twice():
    print("noalloc case 1: B2 T4096 H4 K=V=128 (8 segments)", flush=True)
    _run(2, 4096, 4, 128, 128, 951)
    print("noalloc case 2: B1 T2000 H2 K64 V128 (smaller, partial last chunk)", flush=True)
    _run(1, 2000, 2, 64, 128, 952)
    print("noalloc case 3: B2 T1024 H2 K=V=128, per-token decays near 4 (gate-range "
          "fallback through the scratch's flags) against the oracle", flush=True)
    _run(2, 1024, 2, 128, 128, 953, gate_mul=5.0)
