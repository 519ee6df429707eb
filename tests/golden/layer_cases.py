"""Layer fixture cases and their deterministic inputs (shared by the fixture writer and the
tests that read ``gla_layer.npz``).

Cases follow the reference's layer-test table (``tests/layers/test_gla.py:2153-2295, 2414,
2950`` and ``run_test_layer_cu_seqlens`` ``:785-846``): hidden 128, 4 heads unless noted. T <= 64
runs the layer's fused-recurrent mode and T > 64 its chunked mode (``tops/layers/gla.py:224``).

Parameters and inputs are drawn with numpy's PCG64 (stable across machines and versions), one
stream per (case seed, parameter name): Linear weights and biases ~ U(-1/sqrt(fan_in),
1/sqrt(fan_in)) (torch's nn.Linear range), norm weights 1 + 0.1 N(0, 1) (so the affine weight
matters), x ~ N(0, 1), probe ~ N(0, 1). The loss is ``sum(out * probe)``.
"""

from __future__ import annotations

import zlib

import numpy as np

# name -> (constructor kwargs, B, T, seed, gradients stored, cu_seqlens)
CASES = {
    "basic": (dict(), 2, 32, 101, True, None),                                  # :2157
    "no_fuse": (dict(fuse_norm=False), 2, 32, 102, False, None),                 # :2161
    "mqa": (dict(num_kv_heads=2), 2, 32, 103, False, None),                      # :2204
    "no_gate": (dict(use_output_gate=False, fuse_norm=False), 2, 32, 104, True, None),  # :2249
    "chunk_T128": (dict(), 1, 128, 105, True, None),                           # :2414
    "chunk_T65": (dict(), 1, 65, 106, False, None),                             # :2950
    "T1": (dict(hidden_size=64, num_heads=2), 1, 1, 107, True, None),          # :2288
    "clamp": (dict(clamp_min=-0.5), 2, 32, 108, False, None),                   # :2268
    "normalizer8": (dict(gate_logit_normalizer=8), 2, 32, 109, False, None),    # :2274
    "expand_v2": (dict(expand_v=2.0), 2, 32, 110, False, None),                 # :2235
    "cu_seqlens": (dict(), 1, 48, 111, False, [0, 16, 32, 48]),                 # :785-846
    "chunk_mqa_nofuse": (dict(num_kv_heads=2, fuse_norm=False), 1, 130, 112, True, None),
}


def full_kwargs(kw):
    """The constructor arguments of a case (the reference table's defaults filled in)."""
    out = dict(mode="chunk", hidden_size=128, num_heads=4, expand_k=0.5, expand_v=1.0)
    out.update(kw)
    return out


def _rng(seed, name):
    return np.random.default_rng([seed, zlib.crc32(name.encode())])


def make_params(seed, shapes):
    """``{name: float32 array}`` for the parameter names and shapes of a layer."""
    out = {}
    for name, shape in shapes.items():
        r = _rng(seed, name)
        if "norm" in name:
            out[name] = (1.0 + 0.1 * r.standard_normal(shape)).astype(np.float32)
            continue
        # Linear [out, in] weight, or the bias of a Linear whose weight is `<module>.weight`
        fan_in = shapes[name.rsplit(".", 1)[0] + ".weight"][1]
        lim = 1.0 / np.sqrt(fan_in)
        out[name] = r.uniform(-lim, lim, size=shape).astype(np.float32)
    return out


def make_io(seed, B, T, hidden):
    """(x, probe) float32 ``[B, T, hidden]``."""
    x = _rng(seed, "x").standard_normal((B, T, hidden)).astype(np.float32)
    probe = _rng(seed, "probe").standard_normal((B, T, hidden)).astype(np.float32)
    return x, probe
