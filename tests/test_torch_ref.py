"""The torch chunked GLA used by the full-size GPU parity test, pinned to the numpy oracle.

Forward (o, final state) against ``oracle.chunk_gla`` and autograd gradients (dq, dk, dv,
dg, dh0) against ``oracle.chunk_gla_bwd``, in float64 on the CPU, on ragged lengths (a
partial last chunk), an initial state and a final-state gradient.
"""

import numpy as np
import pytest
import torch

import oracle as orc
from gla_cases import make_inputs
from torch_ref import chunk_gla_torch


@pytest.mark.parametrize("B,T,H,K,V,C,seed", [
    (1, 200, 2, 16, 32, 64, 3),
    (2, 64, 1, 32, 16, 64, 5),
    (1, 77, 3, 8, 8, 16, 9),
])
def test_torch_ref_matches_oracle(B, T, H, K, V, C, seed):
    q, k, v, g, s0, do, dht = make_inputs(B, T, H, K, V, seed, gate_div=16.0, h0=True,
                                          dht=True)
    t = lambda x: torch.tensor(x, dtype=torch.float64, requires_grad=True)  # noqa: E731
    tq, tk, tv, tg, th0 = t(q), t(k), t(v), t(g), t(s0)
    o, ht = chunk_gla_torch(tq, tk, tv, tg, th0, chunk_size=C)
    on, hn = orc.chunk_gla(q, k, v, g, initial_state=s0, output_final_state=True,
                           chunk_size=C)
    np.testing.assert_allclose(o.detach().numpy(), on, rtol=0, atol=1e-9)
    np.testing.assert_allclose(ht.detach().numpy(), hn, rtol=0, atol=1e-9)
    torch.autograd.backward([o, ht], [torch.tensor(do), torch.tensor(dht)])
    ref = orc.chunk_gla_bwd(q, k, v, g, None, None, K ** -0.5, s0, None, None, do, dht,
                            chunk_size=C)
    for name, x, r in zip(["dq", "dk", "dv", "dg", "dh0"], (tq, tk, tv, tg, th0), ref):
        np.testing.assert_allclose(x.grad.numpy(), r, rtol=0, atol=1e-8, err_msg=name)
