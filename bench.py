#!/usr/bin/env python3
"""Benchmarks of the GLA hot path on one MI355X (the headline configurations C1-C5).

Default (the headline metric, configs[3], "C4"): ``chunk_gla`` forward + backward, B=4 T=8192
H=16 K=V=128, bf16, chunk 64, h0 and dht. One step = forward (o, ht) + backward (dq, dk, dv,
dg, dh0) through autograd on synthetic inputs already resident in HBM (numpy
default_rng(seed=4), draw order q, k, v, g_raw, h0, do, dht; g = logsigmoid(g_raw) / 16;
h0, dht ~ N(0, 0.1^2)).

Other legs (``--op``; not the headline, same JSON fields):
  fused_recurrent : configs[1] "C2", fused_recurrent_gla forward with final state, B8 T2048
                    H4 K256 V512 bf16, h0 fp32, o fp32 (the reference's convention);
  chunk_fwd_c3    : configs[2] "C3", chunk_gla forward, B8 T4096 H4 K256 V512 bf16, h0;
  layer_c5        : configs[4] "C5", GatedLinearAttention forward + backward, bf16, B2
                    T16384 hidden 2048, 4 heads (K 256, V 512), weights ~ N(0, 0.02), the
                    output's gradient a fixed random probe (flops / bytes: the GLA core's);
  simple_gla      : the C4 shape with a per-head constant log-decay (chunk_gla(g_gamma=...));
  decode_t1 / _t64: fused_recurrent_gla forward at a decode shape, B64 H16 K=V=128, T = 1 / 64:
                    the recurrent kernel where HBM, not VALU, bounds it.

The default run (``--op chunk_gla``) first measures the other configurations, C2, C3 and C5,
and the two decode shapes (the legs above, fixed warmup and step counts each), and reports
them compactly under
``legs`` in the headline's line: ms per step, tokens/s, the step's HBM fraction, and the
dominant kernel's roofline fraction (C2: fp32 VALU, with its HBM fraction beside it). They
run before the headline's warmup, so its timed steps also start at the GPU's steady clocks.

The JSON line carries the driver's fields plus
  tflops, mfma_frac   : the step's flops (per token-head: forward 4KV + 2C(K+V), backward
                        twice that) / time, / bf16 dense peak;
  step_hbm_frac       : the step's algorithmic bytes (every input read once, every output
                        written once) / time / 8 TB/s;
  roofline            : the dominant kernel of the step, timed inside the timed steps with
                        HIP events the library records on the launch stream (torch's current
                        stream) around every launch of it, against its binding roofline with
                        its algorithmic bytes (every input read once, every output written
                        once; the per-chunk state residual h / dh is
                        implementation traffic, reported apart) -- or, for the recurrent
                        kernel, its fp32 VALU lane-ops against the non-packed VALU peak with
                        the HBM fraction beside it; ``traffic`` = its HBM bytes per launch
                        from the copy-calibrated rocprofv3 FETCH_SIZE / WRITE_SIZE summary
                        (profiles/hbm_traffic.json);
  kernels             : every timed kernel of the step (average ms, algorithmic GB/s);
  cpu_baseline        : the float32 numpy oracle (the reference's jnp algorithm restated) on
                        a sample of the workload's batch rows (every head at full length),
                        its (batch, head) slices spread over one single-threaded process per
                        host core (rank 0, N = 1 only).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "pallas-kernel_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK = 2.517e15
# fp32 VALU without packed-fp32 instructions (disabled in this build): 256 CUs x 4 SIMDs x 16
# lanes per clock x 2.4 GHz lane-ops per second
VALU_LANE_OPS_PEAK = 256 * 64 * 2.4e9
BF = 2      # bf16 bytes
F4 = 4      # fp32 bytes
METRIC = "chunk_gla fwd+bwd tokens/s & % bf16 MFMA peak, B4 T8192 H16 K=V=128"
KT_HEAD_FWD, KT_HEAD_BWD, KT_REC_FWD, KT_BWD_DQKG = 0, 1, 2, 3


def _flops(T_tok, H, K, V, C, fwd=True, bwd=False):
    """Flops per token-head: forward 4KV + 2C(K+V) (state and chunk products), backward
    twice that."""
    per = (4 * K * V + 2 * C * (K + V)) * (int(fwd) + 2 * int(bwd))
    return T_tok * H * per


def _rng_inputs(shape_qk, V, seed, h0=True, do=False, dht=False, gate_div=16.0):
    import numpy as np

    r = np.random.default_rng(seed)
    f = np.float32
    B, T, H, K = shape_qk
    out = {"q": r.standard_normal((B, T, H, K), dtype=f),
           "k": r.standard_normal((B, T, H, K), dtype=f),
           "v": r.standard_normal((B, T, H, V), dtype=f)}
    graw = r.standard_normal((B, T, H, K), dtype=f)
    if h0:
        out["h0"] = r.standard_normal((B, H, K, V), dtype=f) * 0.1
    if do:
        out["do"] = r.standard_normal((B, T, H, V), dtype=f)
    if dht:
        out["dht"] = r.standard_normal((B, H, K, V), dtype=f) * 0.1
    out["g"] = (-np.logaddexp(0, -graw) / gate_div).astype(f)
    out["_rng"] = r
    return out


def _to_dev(x, dev, states=("h0", "dht")):
    import torch

    d = {}
    for n, a in x.items():
        if n.startswith("_"):
            continue
        t = torch.from_numpy(a).to(dev)
        d[n] = t if n in states else t.to(torch.bfloat16)
    return d


# ---------------------------------------------------------------------------
# legs
# ---------------------------------------------------------------------------


def leg_chunk_gla(dev, simple=False):
    """C4: chunk_gla forward + backward (the headline)."""
    import numpy as np
    import torch

    import tops.ops.gla as G

    B, T, H, K, V, C = 4, 8192, 16, 128, 128, 64
    raw = _rng_inputs((B, T, H, K), V, 4, do=True, dht=True)
    # simple_gla: a per-head constant log-decay drawn after the main inputs
    gamma = (-np.logaddexp(0, -raw["_rng"].standard_normal(H, dtype=np.float32))).astype(
        np.float32)
    x = _to_dev(raw, dev)
    lq, lk, lv, lg, lh0 = (x[n].clone().requires_grad_() for n in ("q", "k", "v", "g", "h0"))
    tok = B * T * H
    states = 2 * B * H * K * V * F4
    resid = (T // C) * B * H * K * V * BF    # bf16 per-chunk states h (forward -> backward)
    if simple:
        gg = torch.from_numpy(gamma).to(dev).reshape(H, 1)

        def step():
            o, ht = G.chunk_gla(lq, lk, lv, g_gamma=gg, initial_state=lh0,
                                output_final_state=True, chunk_size=C)
            return torch.autograd.grad((o, ht), (lq, lk, lv, lh0), (x["do"], x["dht"]))

        fwd_b, bwd_b = tok * (2 * K + 2 * V) * BF + states, tok * (4 * K + 3 * V) * BF + states
        metric = "chunk_gla g_gamma (simple GLA) fwd+bwd tokens/s, B4 T8192 H16 K=V=128"
        flops = None   # the per-element flop count does not describe the scalar-gate form
        workload = "chunk_gla fwd+bwd, per-head g_gamma, BASELINE configs[3] shape"
    else:
        def step():
            o, ht = G.chunk_gla(lq, lk, lv, lg, initial_state=lh0, output_final_state=True,
                                chunk_size=C)
            return torch.autograd.grad((o, ht), (lq, lk, lv, lg, lh0), (x["do"], x["dht"]))

        fwd_b, bwd_b = tok * (3 * K + 2 * V) * BF + states, tok * (6 * K + 3 * V) * BF + states
        metric = METRIC
        flops = _flops(B * T, H, K, V, C, fwd=True, bwd=True)
        workload = "chunk_gla fwd+bwd (BASELINE configs[3])"
    return dict(
        metric=metric, tokens=B * T, flops=flops, bytes=fwd_b + bwd_b, step=step,
        config={"workload": workload, "B": B, "T": T, "H": H, "K": K, "V": V,
                "chunk_size": C, "h0": True, "dht": True, "global_batch": B, "seq_len": T,
                "parallelism": "single-gpu"},
        kernels={"head_fwd_kernel": dict(slot=KT_HEAD_FWD, bytes=fwd_b, residual=resid),
                 "head_bwd_kernel": dict(slot=KT_HEAD_BWD, bytes=bwd_b, residual=resid)},
        bound="hbm",
        cpu=None if simple else dict(fn="chunk_gla_fwd_bwd", shape=(B, T, H, K, V, C), seed=4,
                                     rows=B),
        stages=(lambda: _c4_stages(x, simple, B, T, H, K, V, C, gamma)),
    )


def leg_fused_recurrent(dev):
    """C2: fused_recurrent_gla forward with final state (fp32 o, the reference's default)."""
    import torch

    import tops.ops.gla as G

    B, T, H, K, V = 8, 2048, 4, 256, 512
    raw = _rng_inputs((B, T, H, K), V, 2)
    x = _to_dev(raw, dev)

    def step():
        with torch.no_grad():
            return G.fused_recurrent_gla(x["q"], x["k"], x["v"], gk=x["g"],
                                         initial_state=x["h0"], output_final_state=True)

    tok = B * T * H
    nbytes = tok * (3 * K + V) * BF + tok * V * F4 + 2 * B * H * K * V * F4
    lane_ops = 3 * tok * K * V   # decay multiply, rank-1 FMA, output FMA per state element
    return dict(
        metric="fused_recurrent_gla fwd tokens/s, B8 T2048 H4 K256 V512 (BASELINE configs[1])",
        tokens=B * T, flops=None, bytes=nbytes, step=step,
        config={"workload": "fused_recurrent_gla fwd + final state (BASELINE configs[1])",
                "B": B, "T": T, "H": H, "K": K, "V": V, "h0": True, "o_dtype": "f32",
                "global_batch": B, "seq_len": T, "parallelism": "single-gpu"},
        kernels={"rec_scan_kernel": dict(slot=KT_REC_FWD, bytes=nbytes, residual=0,
                                         lane_ops=lane_ops)},
        bound="valu",
        cpu=dict(fn="fused_recurrent_fwd", shape=(B, T, H, K, V), seed=2, rows=B),
        stages=None,
    )


def leg_recurrent_decode(dev, T):
    """fused_recurrent_gla forward at a decode shape: B64 H16 K=V=128,
    T = 1 or 64 tokens, bf16 inputs, h0 and the final state fp32, o fp32 -- the shape where
    the recurrent kernel is bound by HBM (state in and out) rather than by its VALU work."""
    import torch

    import tops.ops.gla as G

    B, H, K, V = 64, 16, 128, 128
    raw = _rng_inputs((B, T, H, K), V, 6 + T)
    x = _to_dev(raw, dev)

    def step():
        with torch.no_grad():
            return G.fused_recurrent_gla(x["q"], x["k"], x["v"], gk=x["g"],
                                         initial_state=x["h0"], output_final_state=True)

    tok = B * T * H
    nbytes = tok * (3 * K + V) * BF + tok * V * F4 + 2 * B * H * K * V * F4
    return dict(
        metric=f"fused_recurrent_gla fwd (decode) tokens/s, B64 T{T} H16 K=V=128",
        tokens=B * T, flops=None, bytes=nbytes, step=step,
        config={"workload": f"fused_recurrent_gla fwd + final state, decode shape T={T}",
                "B": B, "T": T, "H": H, "K": K, "V": V, "h0": True, "o_dtype": "f32",
                "global_batch": B, "seq_len": T, "parallelism": "single-gpu"},
        kernels={"rec_scan_kernel": dict(slot=KT_REC_FWD, bytes=nbytes, residual=0,
                                         lane_ops=3 * tok * K * V)},
        bound="hbm", cpu=None, stages=None,
    )


def leg_chunk_fwd_c3(dev):
    """C3: chunk_gla forward, wide heads."""
    import torch

    import tops.ops.gla as G

    B, T, H, K, V, C = 8, 4096, 4, 256, 512, 64
    raw = _rng_inputs((B, T, H, K), V, 3)
    x = _to_dev(raw, dev)

    def step():
        with torch.no_grad():
            return G.chunk_gla(x["q"], x["k"], x["v"], x["g"], initial_state=x["h0"],
                               output_final_state=True, chunk_size=C)

    tok = B * T * H
    nbytes = tok * (3 * K + 2 * V) * BF + 2 * B * H * K * V * F4
    return dict(
        metric="chunk_gla fwd tokens/s, B8 T4096 H4 K256 V512 (BASELINE configs[2])",
        tokens=B * T, flops=_flops(B * T, H, K, V, C), bytes=nbytes, step=step,
        config={"workload": "chunk_gla fwd (BASELINE configs[2])", "B": B, "T": T, "H": H,
                "K": K, "V": V, "chunk_size": C, "h0": True, "global_batch": B,
                "seq_len": T, "parallelism": "single-gpu"},
        # the work is split over the gating kernel (q, k, g in; gated tiles out), the segment
        # pass and head_fwd_kernel (gated tiles, v in; o out): the roofline is the step's
        kernels={"head_fwd_kernel": dict(slot=KT_HEAD_FWD, bytes=nbytes, residual=0)},
        bound="hbm", roofline_on_step=True,
        cpu=dict(fn="chunk_gla_fwd", shape=(B, T, H, K, V, C), seed=3, rows=B),
        stages=None,
    )


def leg_layer_c5(dev):
    """C5: the GLA layer forward + backward (flops / bytes of the attention core only)."""
    import torch

    from tops.layers import GatedLinearAttention

    B, T, D, H = 2, 16384, 2048, 4
    K, V, C = D // 2 // H, D // H, 64
    m = GatedLinearAttention(hidden_size=D, num_heads=H, expand_k=0.5, expand_v=1.0,
                             gate_low_rank_dim=16, gate_logit_normalizer=16, rngs=5,
                             dtype=torch.bfloat16).to(dev)
    gen = torch.Generator(device=dev).manual_seed(5)
    with torch.no_grad():
        for _, p in m.named_parameters():
            p.copy_(torch.randn(p.shape, generator=gen, device=dev) * 0.02)
    x = torch.randn(B, T, D, generator=gen, device=dev).to(torch.bfloat16).requires_grad_()
    probe = torch.randn(B, T, D, generator=gen, device=dev).to(torch.bfloat16)
    params = [p for p in m.parameters()]

    def step():
        out, _, _ = m(x)
        # the output gradient handed to the backward (as the C4 leg does): the layer's forward
        # and backward only, no loss reduction of the output
        return torch.autograd.grad(out, [x] + params, probe)

    tok = B * T * H
    fwd_b = tok * (3 * K + 2 * V) * BF
    bwd_b = tok * (6 * K + 3 * V) * BF
    dqkg_b = tok * (6 * K + 2 * V) * BF   # q, k, g, v, do in; dq, dk, dg out
    resid = (T // C) * B * H * K * V * BF * 2   # h and dh tiles it reads
    return dict(
        metric="GatedLinearAttention fwd+bwd tokens/s, B2 T16384 hidden 2048 (BASELINE "
               "configs[4])",
        tokens=B * T, flops=_flops(B * T, H, K, V, C, fwd=True, bwd=True),
        bytes=fwd_b + bwd_b, step=step,
        config={"workload": "GatedLinearAttention fwd+bwd (BASELINE configs[4])", "B": B,
                "T": T, "hidden": D, "heads": H, "K": K, "V": V, "chunk_size": C,
                "global_batch": B, "seq_len": T, "parallelism": "single-gpu",
                "counted": "GLA core flops/bytes (projections are hipBLASLt GEMMs, not counted)"},
        kernels={"head_fwd_kernel": dict(slot=KT_HEAD_FWD, bytes=fwd_b, residual=resid // 2),
                 "head_dqkg_kernel": dict(slot=KT_BWD_DQKG, bytes=dqkg_b, residual=resid)},
        bound="hbm", cpu=None, stages=None,
    )


LEGS = {"chunk_gla": leg_chunk_gla, "simple_gla": lambda d: leg_chunk_gla(d, simple=True),
        "fused_recurrent": leg_fused_recurrent, "chunk_fwd_c3": leg_chunk_fwd_c3,
        "layer_c5": leg_layer_c5,
        "decode_t1": lambda d: leg_recurrent_decode(d, 1),
        "decode_t64": lambda d: leg_recurrent_decode(d, 64)}


# ---------------------------------------------------------------------------
# the C4 entry points on their own (segment preparation vs fused kernel)
# ---------------------------------------------------------------------------


def _c4_stages(x, simple, B, T, H, K, V, C, gamma, reps=25):
    """tops_gla_chunk_fwd / _bwd (or the scalar-gate pair) called back to back through the C
    ABI: whole entry point timed with torch events on the launch stream, the fused kernel
    with the library's HIP events; their difference is the segment preparation."""
    import torch

    from tops import _lib
    from tops._lib import SeqLayout, call, ptr, stream_of

    lib = _lib.load()
    dev = x["q"].device
    seq = SeqLayout(B, T, C, None, dev)
    st = stream_of(dev)
    sc = K ** -0.5
    h = torch.empty(seq.NC, H, K, V, dtype=torch.bfloat16, device=dev)
    dh = torch.empty_like(h)
    o, dq, dk, dv, dg = (torch.empty_like(x[n]) for n in ("v", "q", "k", "v", "g"))
    ht, dh0 = torch.empty_like(x["h0"]), torch.empty_like(x["h0"])
    q, k, v, g, h0, do, dht = (x[n] for n in ("q", "k", "v", "g", "h0", "do", "dht"))
    lay = (B, T, H, K, V, C, *seq.args(), _lib.BF16, st)
    ws, nws = _lib.seg_workspace(B, T, H, K, V, C, False, torch.bfloat16, dev, backward=True)
    gs = torch.from_numpy(gamma).to(dev)
    if simple:
        runs = [("simple_chunk_fwd", KT_HEAD_FWD, lambda: call(
                    "tops_gla_simple_chunk_fwd", ptr(q), ptr(k), ptr(v), ptr(gs), 0, ptr(h0),
                    ptr(o), ptr(ht), ptr(h), ptr(ws), nws, sc, *lay)),
                ("simple_chunk_bwd", KT_HEAD_BWD, lambda: call(
                    "tops_gla_simple_chunk_bwd", ptr(q), ptr(k), ptr(v), ptr(gs), 0, ptr(h0),
                    ptr(h), ptr(do), ptr(dht), ptr(dq), ptr(dk), ptr(dv), None, ptr(dh0), None,
                    ptr(ws), nws, sc, *lay))]
    else:
        runs = [("chunk_fwd", KT_HEAD_FWD, lambda: call(
                    "tops_gla_chunk_fwd", ptr(q), ptr(k), ptr(v), ptr(g), ptr(h0), ptr(o),
                    ptr(ht), ptr(h), ptr(ws), nws, sc, *lay)),
                ("chunk_bwd", KT_HEAD_BWD, lambda: call(
                    "tops_gla_chunk_bwd", ptr(q), ptr(k), ptr(v), ptr(g), ptr(h0), ptr(h),
                    ptr(do), ptr(dht), ptr(dq), ptr(dk), ptr(dv), ptr(dg), ptr(dh0), None,
                    ptr(dh), ptr(ws), nws, sc, *lay))]
    stages = {}
    cur = torch.cuda.current_stream(dev)
    for entry, slot, fn in runs:
        fn()  # warm (the forward also produces the states the backward reads)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(cur)
        for _ in range(reps):
            fn()
        e1.record(cur)
        torch.cuda.synchronize(dev)
        ems = e0.elapsed_time(e1) / reps
        call("tops_gla_kernel_timing", 1)
        for _ in range(reps):
            fn()
        kms = float(lib.tops_gla_kernel_ms(slot))
        call("tops_gla_kernel_timing", 0)
        stages[entry] = dict(ms=round(ems, 4), segment_prep_ms=round(ems - kms, 4))
    return stages


# ---------------------------------------------------------------------------
# CPU baseline: the numpy oracle over the workload's (batch, head) slices
# ---------------------------------------------------------------------------


def _cpu_slice(job):
    """One (batch, head) slice of a CPU-baseline workload, single-threaded (runs in a
    spawned process: no GPU state, BLAS pinned to one thread)."""
    os.environ.update(OMP_NUM_THREADS="1", OPENBLAS_NUM_THREADS="1", MKL_NUM_THREADS="1")
    import numpy as np

    import oracle as orc

    fn, shape, seed, b, h = job
    r = np.random.default_rng([seed, b, h])
    f = np.float32
    T, K, V = shape[1], shape[3], shape[4]
    q, k = (r.standard_normal((1, T, 1, K), dtype=f) for _ in range(2))
    v = r.standard_normal((1, T, 1, V), dtype=f)
    g = (-np.logaddexp(0, -r.standard_normal((1, T, 1, K), dtype=f)) / 16).astype(f)
    h0 = r.standard_normal((1, 1, K, V), dtype=f) * 0.1
    t0 = time.perf_counter()
    if fn == "fused_recurrent_fwd":
        orc.fused_recurrent_gla(q, k, v, gk=g, initial_state=h0, output_final_state=True,
                                dtype=f)
    else:
        C = shape[5]
        orc.chunk_gla(q, k, v, g, initial_state=h0, output_final_state=True, chunk_size=C,
                      dtype=f)
        if fn == "chunk_gla_fwd_bwd":
            do = r.standard_normal((1, T, 1, V), dtype=f)
            dht = r.standard_normal((1, 1, K, V), dtype=f) * 0.1
            orc.chunk_gla_bwd(q, k, v, g, None, None, K ** -0.5, h0, None, None, do, dht,
                              chunk_size=C, dtype=f)
    return time.perf_counter() - t0


def _cpu_baseline(spec, max_procs=None):
    """The float32 numpy oracle on the (batch, head) slices of ``spec["rows"]`` batch rows of
    the workload (every head at full length), spread over one single-threaded spawned process
    per available host core; tokens/s of those rows."""
    import multiprocessing as mp

    cores = len(os.sched_getaffinity(0))
    if max_procs:
        cores = min(cores, max_procs)
    B, T, H = spec["shape"][:3]
    rows = spec["rows"]
    jobs = [(spec["fn"], spec["shape"], spec["seed"], b, h) for b in range(rows)
            for h in range(H)]
    ctx = mp.get_context("spawn")
    t0 = time.perf_counter()
    with ctx.Pool(min(cores, len(jobs))) as pool:
        busy = pool.map(_cpu_slice, jobs, chunksize=1)
    wall = time.perf_counter() - t0
    return dict(value=round(rows * T / wall, 1), unit="tokens/s", cores=min(cores, len(jobs)),
                kind="port",
                sample=f"float32 numpy oracle ({spec['fn']}) on {rows} of the workload's {B} "
                       f"batch rows ({len(jobs)} (batch, head) slices at full length) over "
                       f"{min(cores, len(jobs))} single-threaded processes: {wall:.1f} s wall, "
                       f"{sum(busy):.1f} s of slice compute",
                affinity_cpus=len(os.sched_getaffinity(0)), os_cpu_count=os.cpu_count())


def _measured_traffic(kernel, op):
    """HBM bytes per launch of `kernel` in leg `op` from the committed, copy-calibrated
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (profiles/hbm_traffic.json), or None."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    try:
        with open(path) as f:
            d = json.load(f)["bytes_per_launch"]
    except (OSError, ValueError, KeyError):
        return None
    return d.get(op, {}).get(kernel)


def _measure(leg, steps, warmup, timing):
    """W untimed steps, then K steps timed with torch events on the launch stream (bracketed
    by synchronizations); with ``timing`` another K steps follow with the library's HIP events
    around every launch of the leg's timed kernels. Those events cost host time per launch
    (measured: a short step such as the T = 1 decode, 27 -> 33 us), so they stay out of the
    step's own timed region. Returns (ms per step, {kernel: ms})."""
    import torch

    from tops import _lib

    dev = torch.device("cuda:0")
    step = leg["step"]
    for _ in range(warmup):
        step()
    torch.cuda.synchronize(dev)
    cur = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(cur)
    for _ in range(steps):
        step()
    e1.record(cur)
    torch.cuda.synchronize(dev)
    ms = e0.elapsed_time(e1) / steps
    kms = {}
    if timing:   # HIP events around every timed-kernel launch of K more steps
        _lib.call("tops_gla_kernel_timing", 1)
        for _ in range(steps):
            step()
        torch.cuda.synchronize(dev)
        lib = _lib.load()
        for name, kd in leg["kernels"].items():
            x = float(lib.tops_gla_kernel_ms(kd["slot"]))
            if x > 0:
                kms[name] = x
        _lib.call("tops_gla_kernel_timing", 0)
    return ms, kms


def _report(leg, ms, kms, op):
    """The leg's figures: throughput, flop and byte fractions, the dominant kernel's
    roofline (or the step's, where the work is split over kernels)."""
    sec = ms * 1e-3
    out = {"value": round(leg["tokens"] / sec, 1), "ms_per_step": round(ms, 4)}
    if leg["flops"]:
        out["tflops"] = round(leg["flops"] / sec / 1e12, 2)
        out["mfma_frac"] = round(leg["flops"] / sec / MFMA_BF16_PEAK, 4)
    out["step_hbm_frac"] = round(leg["bytes"] / sec / 1e9 / HBM_PEAK_GBS, 4)
    out["step_algorithmic_bytes"] = int(leg["bytes"])
    kernels = {}
    for name, x in kms.items():
        kd = leg["kernels"][name]
        kernels[name] = dict(ms=round(x, 4), bytes=int(kd["bytes"]),
                             gbs=round(kd["bytes"] / (x * 1e-3) / 1e9, 1))
        if kd.get("residual"):
            kernels[name]["residual_bytes"] = int(kd["residual"])
    if kernels and leg.get("roofline_on_step"):
        gbs = leg["bytes"] / sec / 1e9
        out["roofline"] = {
            "bound": "hbm", "kernel": "step (every kernel of the op)", "achieved": round(gbs, 1),
            "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": None}
    elif kernels:
        dom = max(kernels, key=lambda n: kernels[n]["ms"])
        d, kd = kernels[dom], leg["kernels"][dom]
        if leg["bound"] == "valu":
            achieved = kd["lane_ops"] / (d["ms"] * 1e-3) / 1e12
            peak = VALU_LANE_OPS_PEAK / 1e12
            out["roofline"] = {
                "bound": "valu", "kernel": dom, "achieved": round(achieved, 2),
                "peak": round(peak, 2), "unit": "T fp32 lane-ops/s (non-packed)",
                "frac": round(achieved / peak, 4),
                "traffic": _measured_traffic(dom, op),
                "hbm_achieved_gbs": d["gbs"], "hbm_frac": round(d["gbs"] / HBM_PEAK_GBS, 4)}
        else:
            res = int(kd.get("residual", 0))
            out["roofline"] = {
                "bound": "hbm", "kernel": dom, "achieved": d["gbs"], "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(d["gbs"] / HBM_PEAK_GBS, 4),
                "traffic": _measured_traffic(dom, op),
                "residual_bytes": res,
                # the same launch with its per-chunk state traffic counted as well
                "frac_with_residual": round((kd["bytes"] + res) / (d["ms"] * 1e-3) / 1e9 /
                                            HBM_PEAK_GBS, 4)}
    if kernels:
        out["kernels"] = kernels
    return out


# the other BASELINE configurations, measured before the headline leg and reported in its
# line (compact), in this order: (key, leg name, warmup, timed steps). Every leg's inputs are
# made first, so the measurements follow one another with the GPU busy throughout (C5's ten
# warmup steps, about 60 ms, bring it to its steady clocks).
SIDE_LEGS = (("D1", "decode_t1", 5, 50), ("D64", "decode_t64", 5, 50),
             ("C5", "layer_c5", 10, 10), ("C3", "chunk_fwd_c3", 5, 20),
             ("C2", "fused_recurrent", 5, 20))


def _side_leg(leg, op, warmup, steps, timing):
    """One BASELINE configuration other than the headline's, as a compact dict."""
    ms, kms = _measure(leg, steps, warmup, timing)
    r = _report(leg, ms, kms, op)
    d = {"ms_per_step": r["ms_per_step"], "tokens_per_s": r["value"], "steps": steps,
         "warmup": warmup, "step_hbm_frac": r["step_hbm_frac"]}
    if "tflops" in r:
        d["tflops"] = r["tflops"]
    rf = r.get("roofline")
    if rf:
        d["roofline"] = {"kernel": rf["kernel"], "bound": rf["bound"], "frac": rf["frac"]}
        if rf["bound"] == "valu":
            d["roofline"]["hbm_frac"] = rf["hbm_frac"]
        if rf.get("residual_bytes"):
            d["roofline"]["frac_with_residual"] = rf["frac_with_residual"]
        if rf["bound"] == "hbm" and rf["unit"] == "GB/s" and rf["kernel"] in r.get("kernels", {}):
            d["roofline"]["gbs"] = rf["achieved"]
        if rf["kernel"] in r.get("kernels", {}):
            d["roofline"]["kernel_ms"] = r["kernels"][rf["kernel"]]["ms"]
    return d


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # the GPU reaches its steady clocks after about 40 ms of this load: 5 warmup steps alone
    # leave the timed steps 6 % slower than 50 or 200 do (the other configurations' legs,
    # which run first by default, are such a load as well)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--op", choices=tuple(LEGS), default="chunk_gla")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-kernel-profile", action="store_true")
    ap.add_argument("--no-legs", action="store_true",
                    help="skip the C2 / C3 / C5 legs the default headline run reports")
    ap.add_argument("--cpu-procs", type=int, default=0, help="cap on CPU-baseline processes")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a 512 MiB device copy (HBM counter calibration point)")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the GLA path shards over batch and "
              "heads with no communication); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    # torch.autograd.grad with grad_outputs imports this module (and sympy) on its first call,
    # about 0.2 s of host time; imported here, the first step does not leave the GPU idle
    # between the measurements (after such a gap the step time settles over ~50 steps)
    import torch.fx.experimental.symbolic_shapes  # noqa: F401

    dev = torch.device("cuda:0")
    timing = not a.no_kernel_profile
    leg = LEGS[a.op](dev)
    legs = {}
    if a.op == "chunk_gla" and not a.no_legs:
        side = [(key, op, w, k, LEGS[op](dev)) for key, op, w, k in SIDE_LEGS]
        for key, op, w, k, sl in side:
            legs[key] = _side_leg(sl, op, w, k, timing)
        order = [key for key, *_ in SIDE_LEGS]
        legs = {key: legs[key] for key in sorted(order)}
    # the C4 entry points timed on their own: a measurement of the same work, made right before
    # the headline's warmup (the step time falls for about 30 steps of this work after other
    # work or idle: measured, 0.69-0.87 -> 0.64 ms)
    stages = leg["stages"]() if timing and leg["stages"] is not None else None
    ms, kms = _measure(leg, a.steps, a.warmup, timing)
    out = {
        "metric": leg["metric"],
        "value": None,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": leg["config"],
    }
    out.update(_report(leg, ms, kms, a.op))
    if stages is not None:
        out["stages"] = stages
    if legs:
        out["legs"] = legs
    if a.calibrate_copy:
        n = 512 * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize(dev)
    if not a.no_cpu_baseline and leg["cpu"] is not None:
        out["cpu_baseline"] = _cpu_baseline(leg["cpu"], a.cpu_procs or None)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
