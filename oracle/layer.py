"""CPU restatement of the GLA layer and its modules, in float64 torch (differentiable, so
that the layer's gradients come from autograd). Test infrastructure only: imported by
``tests/`` and nothing on the product path.

Follows:
* ``GatedLinearAttention.__call__``, ``tops/layers/gla.py:224-345`` (projections, optional
  short convolutions, head split / GQA repeat ``:49-66``, ``log_sigmoid(gk) / normalizer``
  and clamp ``:286-288``, feature map, the recurrence, output norm and gate, o_proj);
* ``FusedRMSNormGated.__call__``, ``tops/modules/fused_norm_gate.py:28-37``;
  ``RMSNorm.__call__``, ``tops/modules/layernorm.py:28-35``;
* ``ShortConvolution._causal_conv1d``, ``tops/modules/convolution.py:46-78``;
* the step recurrence of ``naive_recurrent_gla``, ``tops/ops/gla/naive.py:5-99`` (every mode
  of the layer computes it: chunked, fused-chunk and fused-recurrent are the same function).

Parameters come in as a dict of float64 tensors keyed by the torch module's parameter names
(``q_proj.weight`` [out, in], ``gk_proj.1.bias``, ``q_conv1d.weight`` [D, 1, W], ...).

Pinning: ``recurrence`` against the pinned numpy ``naive_recurrent_gla``; ``rms_norm``,
``gate_logsigmoid`` and ``short_conv`` by closed forms and brute-force taps
(``tests/test_oracle.py``); ``gla_layer`` (the composition: projections, GQA repeat, gate,
norm and output gate, out-projection; output and every gradient) against fixtures written
by the reference's own torch CPU layer, ``tests/src/layers/gla.py:53``, on twelve cases of
the reference's layer-test table (``tests/test_layer_golden.py``, ``tests/golden/``).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

ACT = {"swish": F.silu, "silu": F.silu, "gelu": F.gelu, "relu": F.relu,
       "sigmoid": torch.sigmoid, "tanh": torch.tanh}


def rms_norm(x, weight=None, eps=1e-5, gate=None):
    """x rsqrt(mean(x^2) + eps) [* weight] [* silu(gate)] over the last axis
    (``fused_norm_gate.py:28-37``, ``layernorm.py:28-35``)."""
    y = x * torch.rsqrt((x * x).mean(-1, keepdim=True) + eps)
    if weight is not None:
        y = y * weight
    if gate is not None:
        y = y * F.silu(gate)
    return y


def gate_logsigmoid(x, normalizer, clamp_min=None):
    """``log_sigmoid(x) / normalizer``, clipped below at clamp_min (``gla.py:286-288``)."""
    y = F.logsigmoid(x) / normalizer
    return y if clamp_min is None else torch.clamp(y, min=clamp_min)


def short_conv(x, weight, bias=None, activation="silu", cu_seqlens=None):
    """Causal depthwise conv (``convolution.py:46-78``): per sequence, left zero padding of
    W - 1 rows, then the depthwise taps; optional SiLU. x [B, T, D], weight [D, 1, W]."""
    W = weight.shape[-1]

    def one(seg):   # [1, L, D]
        xp = F.pad(seg.transpose(1, 2), (W - 1, 0))
        return F.conv1d(xp, weight, bias, groups=weight.shape[0]).transpose(1, 2)

    if cu_seqlens is not None:
        y = torch.cat([one(x[:, a:b]) for a, b in zip(cu_seqlens, cu_seqlens[1:])], dim=1)
    else:
        y = one(x) if x.shape[0] == 1 else torch.cat([one(x[i:i + 1]) for i in
                                                        range(x.shape[0])], 0)
    return F.silu(y) if activation in ("silu", "swish") else y


def recurrence(q, k, v, gk, scale, initial_state=None, cu_seqlens=None):
    """``S_t = diag(e^{gk_t}) S_{t-1} + k_t^T v_t``, ``o_t = scale q_t S_t`` per sequence
    (``naive.py:89-96``). q, k, gk [B, T, H, K], v [B, T, H, V]; returns (o, final states)."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    segs = ([(b, 0, T) for b in range(B)] if cu_seqlens is None else
            [(0, a, e) for a, e in zip(cu_seqlens, cu_seqlens[1:])])
    outs = [None] * T if cu_seqlens is not None else None
    o_rows, finals = [], []
    for i, (b, bos, eos) in enumerate(segs):
        S = torch.zeros(H, K, V, dtype=q.dtype)
        if initial_state is not None:
            S = S + initial_state[i]
        rows = []
        for t in range(bos, eos):
            S = torch.exp(gk[b, t])[:, :, None] * S + k[b, t][:, :, None] * v[b, t][:, None, :]
            rows.append(scale * torch.einsum("hk,hkv->hv", q[b, t], S))
        finals.append(S)
        if cu_seqlens is None:
            o_rows.append(torch.stack(rows) if rows else torch.zeros(0, H, V, dtype=q.dtype))
        else:
            for t, r in zip(range(bos, eos), rows):
                outs[t] = r
    if cu_seqlens is None:
        o = torch.stack(o_rows)
    else:
        o = torch.stack(outs)[None]
    return o, torch.stack(finals)


def gla_layer(params, x, cfg, cu_seqlens=None, initial_state=None, recurrence_fn=None):
    """The layer's forward (``gla.py:224-345``) for config ``cfg`` (the constructor's keyword
    arguments). Returns (o [B, T, hidden], final recurrent state). ``recurrence_fn`` (same
    arguments and results as ``recurrence``) replaces the step recurrence, e.g. by a chunked
    form for full-length sequences on the GPU."""
    hidden = cfg.get("hidden_size", 1024)
    H = cfg.get("num_heads", 4)
    Hkv = cfg.get("num_kv_heads") or H
    G = H // Hkv
    key_dim = int(hidden * cfg.get("expand_k", 0.5))
    value_dim = int(hidden * cfg.get("expand_v", 1.0))
    dk, dv = key_dim // H, value_dim // H
    lin = lambda name, t: F.linear(t, params[name + ".weight"],  # noqa: E731
                                   params.get(name + ".bias"))
    q, k, v = lin("q_proj", x), lin("k_proj", x), lin("v_proj", x)
    if cfg.get("use_short_conv", False):
        conv = lambda name, t: short_conv(t, params[name + ".weight"],  # noqa: E731
                                          params.get(name + ".bias"), "silu", cu_seqlens)
        q, k, v = conv("q_conv1d", q), conv("k_conv1d", k), conv("v_conv1d", v)
    gk = lin("gk_proj.1", lin("gk_proj.0", x))

    def heads(t, d, groups):
        t = t.reshape(*t.shape[:-1], t.shape[-1] // d, d)
        if groups > 1:
            t = t.unsqueeze(-2).expand(*t.shape[:-1], groups, d).reshape(
                *t.shape[:-2], t.shape[-2] * groups, d)
        return t

    q = heads(q, dk, 1)
    k, gk, v = heads(k, dk, G), heads(gk, dk, G), heads(v, dv, G)
    gk = gate_logsigmoid(gk, cfg.get("gate_logit_normalizer", 16), cfg.get("clamp_min"))
    fm = cfg.get("feature_map")
    if fm is not None:
        q, k = ACT[fm](q), ACT[fm](k)
    o, ht = (recurrence_fn or recurrence)(q, k, v, gk, dk ** -0.5, initial_state, cu_seqlens)
    eps = cfg.get("norm_eps", 1e-5)
    affine = cfg.get("elementwise_affine", True)
    use_gate = cfg.get("use_output_gate", True)
    fused = cfg.get("gate_fn", "swish") == "swish" and cfg.get("fuse_norm", True) and use_gate
    if fused:
        g = heads(lin("g_proj", x), dv, 1)
        w = params["g_norm_swish_gate.weight"] if affine else None
        o = rms_norm(o, w, eps, g).reshape(*o.shape[:-2], value_dim)
    else:
        w = params["g_norm.weight"] if affine else None
        o = rms_norm(o, w, eps).reshape(*o.shape[:-2], value_dim)
        if use_gate:
            o = o * ACT[cfg.get("gate_fn", "swish")](lin("g_proj", x))
    return lin("o_proj", o), ht
