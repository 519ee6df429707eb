#!/usr/bin/env python3
"""North-star benchmark: chunk_gla forward + backward, B=4 T=8192 H=16 K=V=128, bf16,
chunk 64, h0 and dht (its headline metric).

One step = chunk_gla forward (o, ht) + backward (dq, dk, dv, dg, dh0) on synthetic inputs
already resident in HBM (the benchmark's input recipe: numpy default_rng(seed=4), draw order
q, k, v, g_raw, h0, do, dht; g = logsigmoid(g_raw) / 16; h0, dht ~ N(0, 0.1^2)).

Prints ONE JSON line with the driver's fields plus
  roofline     : the dominant kernel of a step (largest share of its time), timed in the
                 timed steps themselves with HIP events the library records on the launch
                 stream (torch's current stream) right around every launch of that kernel
                 (average over the timed steps), against the HBM roofline with its
                 algorithmic bytes per launch, and the copy-calibrated rocprofv3
                 FETCH_SIZE + WRITE_SIZE bytes per launch (profiles/hbm_traffic.json);
  cpu_baseline : the numpy oracle (float32, one thread) on a bounded sample of the same
                 workload (1 batch row, all 16 heads, full T), scaled to tokens/s of
                 the whole workload;
  kernels      : the fused forward / backward kernels in the timed steps: average
                 duration, achieved GB/s;
  stages       : the chunk_fwd / chunk_bwd entry points called on their own, back to back
                 (segment local states + fused kernel), and the part before the
                 fused kernel (timed the same way).
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

B, T, H, K, V, C = 4, 8192, 16, 128, 128, 64
SEED = 4
METRIC = "chunk_gla fwd+bwd tokens/s & % bf16 MFMA peak, B4 T8192 H16 K=V=128"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK = 2.517e15
# algorithmic flops per token-head (full C x C tiles, no recompute): fwd 4KV + 2C(K+V), bwd
# twice that
FLOPS_STEP = B * T * H * (12 * K * V + 6 * C * (K + V))
# state traffic (h/dht fp32) counted once per use
STATE_BYTES = B * H * K * V * 4
BF = 2  # bf16 bytes


def _inputs(device):
    import numpy as np
    import torch

    r = np.random.default_rng(SEED)
    f = np.float32
    q = r.standard_normal((B, T, H, K), dtype=f)
    k = r.standard_normal((B, T, H, K), dtype=f)
    v = r.standard_normal((B, T, H, V), dtype=f)
    graw = r.standard_normal((B, T, H, K), dtype=f)
    h0 = r.standard_normal((B, H, K, V), dtype=f) * 0.1
    do = r.standard_normal((B, T, H, V), dtype=f)
    dht = r.standard_normal((B, H, K, V), dtype=f) * 0.1
    g = (-np.logaddexp(0, -graw) / 16).astype(f)
    # --op simple_gla: a per-head constant log-decay (logsigmoid(randn(H)), drawn last so the
    # main workload's inputs are unchanged)
    gamma = (-np.logaddexp(0, -r.standard_normal(H, dtype=f))).astype(f)
    bf = lambda x: torch.from_numpy(x).to(device).to(torch.bfloat16)  # noqa: E731
    fp = lambda x: torch.from_numpy(x).to(device)  # noqa: E731
    return dict(q=bf(q), k=bf(k), v=bf(v), g=bf(g), h0=fp(h0), do=bf(do), dht=fp(dht),
                gamma=fp(gamma))


def _copy_calibration(device, mib=512, reps=3):
    """Plain device copy of a known size: the HBM-counter calibration point for rocprofv3
    --pmc FETCH_SIZE / WRITE_SIZE runs (bytes read = bytes written = mib MiB per dispatch)."""
    import torch

    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device=device)
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize(device)


def _kernel_bytes(op="chunk_gla"):
    """Algorithmic HBM bytes per launch of the fused forward / backward kernels: every input
    read once and every output written once (tok = B*T*H token-heads; h / dh per chunk bf16;
    h0 / ht or dht / dh0 fp32)."""
    tok = B * T * H
    hbytes = (T // C) * B * H * K * V * BF
    if op == "simple_gla":   # scalar gates: no [.., K] gate tensor in or out
        return {"head_fwd_kernel": tok * (2 * K + 2 * V) * BF + STATE_BYTES * 2 + hbytes,
                "head_bwd_kernel": tok * (4 * K + 3 * V) * BF + STATE_BYTES * 2 + hbytes}
    return {"head_fwd_kernel": tok * (3 * K + 2 * V) * BF + STATE_BYTES * 2 + hbytes,
            "head_bwd_kernel": tok * (6 * K + 3 * V) * BF + STATE_BYTES * 2 + hbytes}


def _kernel_profile(x, reps=10, op="chunk_gla"):
    """The step's two entry points called on their own through the C ABI, back to back:
    whole entry point (segment local states + fused kernel) timed with torch
    events on the launch stream, the fused kernel with the library's HIP events around it
    (tops_gla_kernel_ms), their difference = the segment preparation."""
    import torch

    from tops import _lib
    from tops._lib import SeqLayout, call, ptr, stream_of

    lib = _lib.load()
    dev = x["q"].device
    seq = SeqLayout(B, T, C, None, dev)
    st = stream_of(dev)
    sc = K ** -0.5
    bf = _lib.BF16
    h = torch.empty(seq.NC, H, K, V, dtype=torch.bfloat16, device=dev)
    dh = torch.empty_like(h)
    o, dq, dk, dv, dg = (torch.empty_like(x[n]) for n in ("v", "q", "k", "v", "g"))
    ht, dh0 = torch.empty_like(x["h0"]), torch.empty_like(x["h0"])
    q, k, v, g, h0, do, dht = (x[n] for n in ("q", "k", "v", "g", "h0", "do", "dht"))
    lay = (B, T, H, K, V, C, *seq.args(), bf, st)
    ws, nws = _lib.seg_workspace(B, T, H, K, V, C, False, torch.bfloat16, dev)
    gs = x["gamma"]
    # (entry point, kernel name, timing slot)
    runs = [
        ("simple_chunk_fwd",
         lambda: call("tops_gla_simple_chunk_fwd", ptr(q), ptr(k), ptr(v), ptr(gs), 0, ptr(h0),
                      ptr(o), ptr(ht), ptr(h), ptr(ws), nws, sc, *lay),
         "head_fwd_kernel", 0),
        ("simple_chunk_bwd",
         lambda: call("tops_gla_simple_chunk_bwd", ptr(q), ptr(k), ptr(v), ptr(gs), 0, ptr(h0),
                      ptr(h), ptr(do), ptr(dht), ptr(dq), ptr(dk), ptr(dv), None, ptr(dh0),
                      None, ptr(ws), nws, sc, *lay),
         "head_bwd_kernel", 1),
    ] if op == "simple_gla" else [
        ("chunk_fwd",
         lambda: call("tops_gla_chunk_fwd", ptr(q), ptr(k), ptr(v), ptr(g), ptr(h0), ptr(o),
                      ptr(ht), ptr(h), ptr(ws), nws, sc, *lay),
         "head_fwd_kernel", 0),
        ("chunk_bwd",
         lambda: call("tops_gla_chunk_bwd", ptr(q), ptr(k), ptr(v), ptr(g), ptr(h0), ptr(h),
                      ptr(do), ptr(dht), ptr(dq), ptr(dk), ptr(dv), ptr(dg), ptr(dh0), None,
                      ptr(dh), ptr(ws), nws, sc, *lay),
         "head_bwd_kernel", 1),
    ]
    stages = {}
    cur = torch.cuda.current_stream(dev)
    for entry, fn, kname, slot in runs:
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


def _measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed, copy-calibrated rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (profiles/hbm_traffic.json), or None."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    try:
        with open(path) as f:
            return json.load(f)["bytes_per_launch"].get(kernel)
    except (OSError, ValueError, KeyError):
        return None


def _cpu_baseline(heads=16):
    """Float32 numpy oracle (single thread) on B=1, `heads` heads, full T; scaled to the
    whole workload's tokens/s."""
    import numpy as np

    import oracle as orc

    try:
        from threadpoolctl import threadpool_limits
    except ImportError:  # pragma: no cover
        threadpool_limits = None
    r = np.random.default_rng(SEED)
    f = np.float32
    q, k, v = (r.standard_normal((1, T, heads, d), dtype=f) for d in (K, K, V))
    g = (-np.logaddexp(0, -r.standard_normal((1, T, heads, K), dtype=f)) / 16).astype(f)
    h0 = r.standard_normal((1, heads, K, V), dtype=f) * 0.1
    do = r.standard_normal((1, T, heads, V), dtype=f)
    dht = r.standard_normal((1, heads, K, V), dtype=f) * 0.1

    def run():
        orc.chunk_gla(q, k, v, g, initial_state=h0, output_final_state=True, chunk_size=C,
                      dtype=np.float32)
        orc.chunk_gla_bwd(q, k, v, g, None, None, K ** -0.5, h0, None, None, do, dht,
                          chunk_size=C, dtype=np.float32)

    ctx = threadpool_limits(limits=1) if threadpool_limits else None
    t0 = time.perf_counter()
    if ctx:
        with ctx:
            run()
    else:
        run()
    dt = time.perf_counter() - t0
    frac = heads / (B * H)  # share of the workload's (batch, head) slices
    tokens_per_s = B * T / (dt / frac)
    return dict(value=round(tokens_per_s, 1), unit="tokens/s", cores=1, kind="port",
                sample=f"numpy float32 oracle chunk_gla fwd+bwd on B=1 T={T} H={heads} "
                       f"K=V={K} (={frac:.3f} of the workload), {dt:.1f} s, scaled",
                affinity_cpus=len(os.sched_getaffinity(0)))


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # the GPU reaches its steady clocks after about 40 ms of this load: 5 warmup steps leave
    # the timed steps 6 % slower than 50 or 200 do
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-kernel-profile", action="store_true")
    ap.add_argument("--cpu-heads", type=int, default=16)
    ap.add_argument("--profile-reps", type=int, default=10)
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a 512 MiB device copy (counter calibration)")
    ap.add_argument("--op", choices=("chunk_gla", "simple_gla"), default="chunk_gla",
                    help="simple_gla: the same shape with a per-head constant log-decay "
                         "(chunk_gla(g_gamma=...), the scalar-gate kernels); not the headline "
                         "metric, no CPU baseline")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the GLA path shards over batch and "
              "heads with no communication); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    import tops.ops.gla as G
    from tops import _lib

    dev = torch.device("cuda:0")
    x = _inputs(dev)
    lq, lk, lv, lg, lh0 = (x[n].clone().requires_grad_() for n in ("q", "k", "v", "g", "h0"))

    def step():
        o, ht = G.chunk_gla(lq, lk, lv, lg, initial_state=lh0, output_final_state=True,
                            chunk_size=C)
        return torch.autograd.grad((o, ht), (lq, lk, lv, lg, lh0), (x["do"], x["dht"]))

    if a.op == "simple_gla":
        gg = x["gamma"].reshape(H, 1)

        def step():  # noqa: F811
            o, ht = G.chunk_gla(lq, lk, lv, g_gamma=gg, initial_state=lh0,
                                output_final_state=True, chunk_size=C)
            return torch.autograd.grad((o, ht), (lq, lk, lv, lh0), (x["do"], x["dht"]))

    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize(dev)
    cur = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    timing = not a.no_kernel_profile
    if timing:   # HIP events around every fused-kernel launch of the timed steps
        _lib.call("tops_gla_kernel_timing", 1)
    e0.record(cur)
    for _ in range(a.steps):
        step()
    e1.record(cur)
    torch.cuda.synchronize(dev)
    ms = e0.elapsed_time(e1) / a.steps
    kernels = {}
    if timing:
        lib = _lib.load()
        for slot, (kname, nbytes) in enumerate(_kernel_bytes(a.op).items()):
            kms = float(lib.tops_gla_kernel_ms(slot))
            kernels[kname] = dict(ms=round(kms, 4), bytes=int(nbytes),
                                  gbs=round(nbytes / (kms * 1e-3) / 1e9, 1))
        _lib.call("tops_gla_kernel_timing", 0)
    tokens_s = B * T / (ms * 1e-3)

    simple = a.op == "simple_gla"
    out = {
        "metric": METRIC if not simple else
        "chunk_gla g_gamma (simple GLA) fwd+bwd tokens/s, B4 T8192 H16 K=V=128",
        "value": round(tokens_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "chunk_gla fwd+bwd (BASELINE configs[3])" if not simple else
                   "chunk_gla fwd+bwd, per-head g_gamma, BASELINE configs[3] shape",
                   "B": B, "T": T,
                   "H": H, "K": K, "V": V, "chunk_size": C, "h0": True, "dht": True,
                   "global_batch": B, "seq_len": T, "parallelism": "single-gpu"},
        "tflops": round(FLOPS_STEP / (ms * 1e-3) / 1e12, 2),
        "mfma_frac": round(FLOPS_STEP / (ms * 1e-3) / MFMA_BF16_PEAK, 4),
    }
    if simple:   # the flop count of the per-element form does not describe this op
        del out["tflops"], out["mfma_frac"]
    if timing:
        prof = kernels
        stages = _kernel_profile(x, max(1, a.profile_reps), a.op)
        dom = max(prof, key=lambda n: prof[n]["ms"])
        d = prof[dom]
        out["roofline"] = {"bound": "hbm", "kernel": dom, "achieved": d["gbs"],
                           "peak": HBM_PEAK_GBS, "unit": "GB/s",
                           "frac": round(d["gbs"] / HBM_PEAK_GBS, 4),
                           "traffic": None if simple else _measured_traffic(dom)}
        out["kernels"] = prof
        out["stages"] = stages
    if a.calibrate_copy:
        _copy_calibration(dev)
    if not a.no_cpu_baseline and not simple:
        out["cpu_baseline"] = _cpu_baseline(a.cpu_heads)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
