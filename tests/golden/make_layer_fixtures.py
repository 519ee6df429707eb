"""Writes ``gla_layer.npz``: the reference's own torch CPU GLA layer
(``tests/src/layers/gla.py:53``, importable with torch + einops) run on the cases of
``layer_cases.py``.

Runs only in the build container, where the reference tree is mounted (``/root/reference``,
or ``$TOPS_REFERENCE``); nothing from it is copied: the file holds, per case, the layer output
and (where ``CASES`` asks) the gradients of ``sum(out * probe)`` w.r.t. x and every parameter,
all float32. Parameters and inputs are regenerated from the case seed by ``layer_cases``.

    python tests/golden/make_layer_fixtures.py
"""

from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

from layer_cases import CASES, full_kwargs, make_io, make_params  # noqa: E402


def main():
    ref = os.environ.get("TOPS_REFERENCE", "/root/reference")
    sys.path.insert(0, ref)
    import torch

    from tests.src.layers.gla import GatedLinearAttention as RefGLA  # the reference layer

    torch.set_grad_enabled(True)
    out = {}
    for name, (kw, B, T, seed, grads, cu) in CASES.items():
        ckw = full_kwargs(kw)
        model = RefGLA(**ckw)   # float32, as the reference's own layer tests run it
        shapes = {n: tuple(p.shape) for n, p in model.named_parameters()}
        params = make_params(seed, shapes)
        with torch.no_grad():
            for n, p in model.named_parameters():
                p.copy_(torch.from_numpy(params[n]))
        x, probe = make_io(seed, B, T, ckw["hidden_size"])
        xt = torch.from_numpy(x).requires_grad_(grads)
        extra = {} if cu is None else {"cu_seqlens": torch.LongTensor(cu)}
        o, _, _ = model(xt, **extra)
        out[f"{name}/out"] = o.detach().float().numpy()
        if grads:
            (o * torch.from_numpy(probe)).sum().backward()
            out[f"{name}/d_x"] = xt.grad.float().numpy()
            for n, p in model.named_parameters():
                out[f"{name}/d_{n}"] = p.grad.float().numpy()
        print(f"{name}: out {tuple(o.shape)} max|out| {o.abs().max().item():.3f}", flush=True)
    path = os.path.join(HERE, "gla_layer.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()
