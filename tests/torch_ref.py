"""Chunked GLA in plain torch (float32 / float64), differentiable by torch autograd.

Test infrastructure only: it lets a GPU test check every (batch, head) slice of a
full-size workload, where the numpy oracle would take minutes. It is pinned to the oracle
(``oracle.chunk_gla``, ``oracle.chunk_gla_bwd``) on small inputs by
``tests/test_torch_ref.py``; the gradients are torch autograd's, not a second restatement.

Algorithm: the chunk form of the reference's forward (``tops/ops/gla/chunk.py``: in-chunk
gate cumsum, intra-chunk attention A, inter-chunk state recurrence, output combine). The
gates are factored around the chunk's first position (``q e^{gc}``, ``k e^{-gc}``), as the
reference's jnp path does (``chunk.py:329-332``), so a chunk's cumulative log gate must stay
well inside the float range: use it with weak gates (the tests' ``logsigmoid(x) / 16``).
"""

import torch


def chunk_gla_torch(q, k, v, g, h0=None, scale=None, chunk_size=64):
    """o [B, T, H, V] and the final state [B, H, K, V] for q, k, g [B, T, H, K], v [B, T, H, V]
    (all of one floating dtype), h0 [B, H, K, V] or None; scale defaults to K ** -0.5."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    C = chunk_size
    scale = K ** -0.5 if scale is None else scale
    NC = (T + C - 1) // C
    pad = NC * C - T
    if pad:
        zp = lambda x: torch.nn.functional.pad(x, (0, 0, 0, 0, 0, pad))  # noqa: E731
        q, k, v, g = zp(q), zp(k), zp(v), zp(g)   # zero k, v: no state change; g 0: factor 1

    def chunks(x):   # [B, NC*C, H, D] -> [B, H, NC, C, D]
        return x.reshape(B, NC, C, H, -1).permute(0, 3, 1, 2, 4)

    q, k, v, g = chunks(q), chunks(k), chunks(v), chunks(g)
    gc = g.cumsum(-2)
    qe = q * scale * torch.exp(gc)
    ke = k * torch.exp(-gc)
    A = qe @ ke.transpose(-1, -2).contiguous()
    A = A * torch.tril(torch.ones(C, C, dtype=A.dtype, device=A.device))
    glast = gc[..., -1, :]                              # [B, H, NC, K]
    kd = k * torch.exp(glast.unsqueeze(-2) - gc)        # k decayed to the chunk's end
    h = torch.zeros(B, H, K, V, dtype=q.dtype, device=q.device) if h0 is None else h0
    outs = []
    for n in range(NC):
        outs.append(qe[:, :, n] @ h + A[:, :, n] @ v[:, :, n])
        h = torch.exp(glast[:, :, n]).unsqueeze(-1) * h + \
            kd[:, :, n].transpose(-1, -2).contiguous() @ v[:, :, n]
    o = torch.stack(outs, 2)                            # [B, H, NC, C, V]
    o = o.permute(0, 2, 3, 1, 4).reshape(B, NC * C, H, V)[:, :T]
    return o, h


def slice_errors(got, ref, tok_major):
    """Per (batch, head) slice: max |got - ref| and max |ref|, as [B, H] tensors, for outputs
    laid out [B, T, H, D] (tok_major) or states [B, H, K, V]."""
    dims = (1, 3) if tok_major else (2, 3)
    got, ref = got.detach().float(), ref.detach().float()
    assert torch.isfinite(got).all()
    return (got - ref).abs().amax(dim=dims), ref.abs().amax(dim=dims)
