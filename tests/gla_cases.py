"""Shared input generation and tolerance checks for the GLA tests."""

from __future__ import annotations

import numpy as np
import torch

FP32_ATOL = 1e-4     # north-star bar for float32 inputs: max-abs error
BF16_RTOL_MAX = 2e-2  # north-star bar for bfloat16 inputs: max-abs error / max |ref|


def logsigmoid(x):
    return -np.logaddexp(0.0, -x)


def make_inputs(B, T, H, K, V, seed, gate_div=1.0, h0=False, dht=False, N=None, dtype="f32",
                h_std=1.0):
    """Seeded inputs in the reference's draw order (q, k, v, g, h0, do, dht).

    Returns float64 numpy arrays already rounded to ``dtype`` (so the oracle sees exactly
    what the kernel sees).
    """
    r = np.random.default_rng(seed)
    N = B if N is None else N
    q = r.standard_normal((B, T, H, K))
    k = r.standard_normal((B, T, H, K))
    v = r.standard_normal((B, T, H, V))
    g = logsigmoid(r.standard_normal((B, T, H, K))) / gate_div
    s0 = r.standard_normal((N, H, K, V)) * h_std if h0 else None
    do = r.standard_normal((B, T, H, V))
    sdt = r.standard_normal((N, H, K, V)) * h_std if dht else None
    out = [q, k, v, g, s0, do, sdt]
    if dtype == "bf16":
        out = [None if x is None else round_bf16(x) if i not in (4, 6) else x
               for i, x in enumerate(out)]
    return out


def round_bf16(x):
    return torch.tensor(x, dtype=torch.float32).to(torch.bfloat16).to(torch.float64).numpy()


def to_dev(x, dtype, device="cuda"):
    if x is None:
        return None
    tdt = {"f32": torch.float32, "bf16": torch.bfloat16, "state": torch.float32}[dtype]
    return torch.tensor(np.asarray(x), dtype=torch.float32).to(tdt).to(device).contiguous()


def to_np(t):
    return None if t is None else t.detach().float().cpu().numpy().astype(np.float64)


def check(name, got, ref, dtype, atol=None, rel_f32=None):
    """Assert the north-star tolerance; returns the measured error.

    float32: max-abs error <= 1e-4 (or ``atol``). ``rel_f32`` (a reason) names an output whose
    values are far from order one (sums over long sequences or wide heads, the unmasked
    intra matrix): it is held to 1e-4 x max(1, max |ref|) instead, and both errors are
    printed."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, f"{name}: shape {got.shape} vs {ref.shape}"
    assert np.isfinite(got).all(), f"{name}: non-finite values"
    err = float(np.abs(got - ref).max()) if got.size else 0.0
    if dtype == "f32":
        tol = FP32_ATOL if atol is None else atol
        if rel_f32 is not None:
            big = max(1.0, float(np.abs(ref).max()) if ref.size else 1.0)
            tol = FP32_ATOL * big
            print(f"  {name}: max-abs error {err:.2e}, max |ref| {big:.1f}, error / max(1, "
                  f"max|ref|) {err / big:.2e} ({rel_f32})", flush=True)
        assert err <= tol, f"{name}: max-abs error {err:.3e} > {tol:.1e}"
        return err
    scale = float(np.abs(ref).max()) if ref.size else 1.0
    rel = err / max(scale, 1e-30)
    assert rel <= BF16_RTOL_MAX, f"{name}: error/max|ref| {rel:.3e} > {BF16_RTOL_MAX}"
    return rel
