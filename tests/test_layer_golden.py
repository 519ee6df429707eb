"""The layer oracle (``oracle/layer.py::gla_layer``) against fixtures written by the
reference's own torch CPU layer (``tests/src/layers/gla.py:53``; ``tests/golden/
make_layer_fixtures.py``): forward on every case of ``tests/golden/layer_cases.py`` and, where
stored, the gradients of ``sum(out * probe)`` w.r.t. x and every parameter.

The oracle computes in float64 and the fixtures are float32 from a float32 run, so the bar is
max-abs error <= 2e-5 x max(1, |ref|).
"""

import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))

from layer_cases import CASES, full_kwargs, make_io, make_params  # noqa: E402

FIX = os.path.join(HERE, "golden", "gla_layer.npz")
TOL = 2e-5


def _fixture():
    return np.load(FIX)


def param_shapes(ckw):
    """Parameter names and shapes of the layer for constructor kwargs ``ckw`` (the same names
    as the torch modules: ``q_proj.weight`` [out, in], ...)."""
    hidden, H = ckw["hidden_size"], ckw["num_heads"]
    Hkv = ckw.get("num_kv_heads") or H
    G = H // Hkv
    kd, vd = int(hidden * ckw["expand_k"]), int(hidden * ckw["expand_v"])
    s = {"q_proj.weight": (kd, hidden), "k_proj.weight": (kd // G, hidden),
         "v_proj.weight": (vd // G, hidden)}
    gate = ckw.get("use_output_gate", True)
    if gate:
        s["g_proj.weight"] = (vd, hidden)
    s["gk_proj.0.weight"] = (ckw.get("gate_low_rank_dim", 16), hidden)
    s["gk_proj.1.weight"] = (kd // G, ckw.get("gate_low_rank_dim", 16))
    s["gk_proj.1.bias"] = (kd // G,)
    s["o_proj.weight"] = (hidden, vd)
    fused = ckw.get("gate_fn", "swish") == "swish" and ckw.get("fuse_norm", True) and gate
    s["g_norm_swish_gate.weight" if fused else "g_norm.weight"] = (vd // H,)
    return s


def _close(name, got, ref):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    assert got.shape == ref.shape, f"{name}: {got.shape} vs {ref.shape}"
    err = float(np.abs(got - ref).max())
    assert err <= TOL * max(1.0, float(np.abs(ref).max())), f"{name}: max-abs error {err:.2e}"


def test_fixture_covers_every_case():
    fx = _fixture()
    for name, (kw, B, T, seed, grads, cu) in CASES.items():
        ckw = full_kwargs(kw)
        assert fx[f"{name}/out"].shape == (B, T, ckw["hidden_size"])
        if grads:
            for p, shp in param_shapes(ckw).items():
                assert fx[f"{name}/d_{p}"].shape == shp, (name, p)


@pytest.mark.parametrize("case", list(CASES))
def test_oracle_layer_matches_reference_fixture(case):
    import torch

    from oracle import layer as L

    kw, B, T, seed, grads, cu = CASES[case]
    ckw = full_kwargs(kw)
    fx = _fixture()
    shapes = param_shapes(ckw)
    params = {n: torch.tensor(a, dtype=torch.float64, requires_grad=grads)
              for n, a in make_params(seed, shapes).items()}
    x, probe = make_io(seed, B, T, ckw["hidden_size"])
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=grads)
    o, _ = L.gla_layer(params, xt, ckw, cu_seqlens=cu)
    _close("out", o.detach().numpy(), fx[f"{case}/out"])
    if grads:
        (o * torch.tensor(probe, dtype=torch.float64)).sum().backward()
        _close("d_x", xt.grad.numpy(), fx[f"{case}/d_x"])
        for n, p in params.items():
            _close(f"d_{n}", p.grad.numpy(), fx[f"{case}/d_{n}"])


def test_fixture_detects_a_planted_mistake():
    """A plausible slip in the oracle's composition (the GQA repeat interleaving heads the
    other way round) fails against the fixture."""
    import torch

    from oracle import layer as L

    kw, B, T, seed, _, cu = CASES["mqa"]
    ckw = full_kwargs(kw)
    params = {n: torch.tensor(a, dtype=torch.float64)
              for n, a in make_params(seed, param_shapes(ckw)).items()}
    x, _ = make_io(seed, B, T, ckw["hidden_size"])
    # swap the kv-head blocks of k / v / gk: what a (g h) instead of (h g) repeat would give
    for n in ("k_proj.weight", "v_proj.weight", "gk_proj.1.weight", "gk_proj.1.bias"):
        w = params[n]
        params[n] = torch.cat(list(reversed(w.chunk(2, 0))), 0)
    o, _ = L.gla_layer(params, torch.tensor(x, dtype=torch.float64), ckw, cu_seqlens=cu)
    err = float(np.abs(o.numpy() - _fixture()["mqa/out"]).max())
    assert err > 100 * TOL, err
