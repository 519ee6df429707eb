"""Gated Linear Attention layer on the MI355X kernels.

Reference: ``GatedLinearAttention``, ``tops/layers/gla.py:71-345`` (a Flax NNX module); this
is the same layer as a ``torch.nn.Module`` with the same constructor arguments, call
signature and return convention ``(o, None, past_key_values)``. The attention core runs on
the HIP kernels (``chunk_gla`` / ``fused_chunk_gla``, ``fused_recurrent_gla`` for q_len <= 64),
the key-wise gate activation and the output RMSNorm * SiLU gate on their own HIP kernels,
the projections on hipBLASLt through ``torch.nn.functional.linear``.
"""

from __future__ import annotations

import math
from typing import Any

import torch
import torch.nn.functional as F

from .._lib import require
from ..modules import FusedRMSNormGated, RMSNorm
from ..modules._norm import GateLogSigmoidFn
from ..modules.convolution import ShortConvolution
from ..ops.gla import chunk_gla, fused_chunk_gla, fused_recurrent_gla

__all__ = ["GatedLinearAttention", "LayerCache"]

ACT2FN = {
    "swish": F.silu,
    "silu": F.silu,
    "gelu": F.gelu,
    "relu": F.relu,
    "sigmoid": torch.sigmoid,
    "tanh": torch.tanh,
}


class Linear(torch.nn.Module):
    """Dense layer with Flax's conventions: default init lecun-normal (truncated normal,
    std 1/sqrt(fan_in)), zero bias, and jnp-style dtype promotion of input and weight."""

    def __init__(self, in_features, out_features, use_bias=False, *, generator=None,
                 device=None, dtype=torch.float32):
        super().__init__()
        self.in_features, self.out_features = in_features, out_features
        w = torch.empty(out_features, in_features, dtype=torch.float32)
        std = 1.0 / math.sqrt(in_features) / 0.87962566103423978   # variance-preserving
        torch.nn.init.trunc_normal_(w, std=std, a=-2 * std, b=2 * std, generator=generator)
        self.weight = torch.nn.Parameter(w.to(device=device, dtype=dtype))
        if use_bias:
            self.bias = torch.nn.Parameter(torch.zeros(out_features, device=device, dtype=dtype))
        else:
            self.register_parameter("bias", None)

    def forward(self, x):
        dt = torch.promote_types(x.dtype, self.weight.dtype)
        b = None if self.bias is None else self.bias.to(dt)
        return F.linear(x.to(dt), self.weight.to(dt), b)


def _concat_cols(ts):
    """``torch.cat(ts, 1)`` of row-major [rows, w_i] tensors; on the GPU through the
    library's row-wise concatenation (every destination row written as one contiguous run:
    about twice torch.cat's rate into the row slices of a wider tensor here)."""
    rows = ts[0].shape[0]
    ok = (ts[0].is_cuda and ts[0].dtype in (torch.bfloat16, torch.float32) and len(ts) <= 8
          and all(t.dtype == ts[0].dtype and t.shape[0] == rows and t.is_contiguous()
                  and (t.shape[1] * t.element_size()) % 16 == 0 and t.data_ptr() % 16 == 0
                  for t in ts))
    if not ok:
        return torch.cat(ts, 1)
    import ctypes

    from .._lib import call, dtype_code, stream_of

    out = torch.empty(rows, sum(t.shape[1] for t in ts), dtype=ts[0].dtype,
                      device=ts[0].device)
    srcs = (ctypes.c_void_p * len(ts))(*[t.data_ptr() for t in ts])
    widths = (ctypes.c_int64 * len(ts))(*[t.shape[1] for t in ts])
    call("tops_gla_concat_cols", srcs, widths, len(ts), rows, ctypes.c_void_p(out.data_ptr()),
         dtype_code(out.dtype), stream_of(out.device))
    return out


def _skinny_at_b(a, b, ones=False):
    """``a^T b`` for a tall ``a`` [N, r] with few columns and a tall ``b`` [N, c], in float32:
    a split over the rows (``bmm`` of S row blocks, then the S partial products summed).
    With ``ones`` a row of column sums of ``b`` is appended (the bias gradient of a layer
    whose output gradient is ``b``). A single GEMM of this shape has no parallelism to spare
    in its output (r x c) and walks the N rows in one pass: hipBLASLt took 104 us for
    [32768, 1024]^T [32768, 16] and 71 us for [32768, 16]^T [32768, 2048], the split form
    47 and 41 us. Summed in float32 (or the inputs' wider type). Returns None when N does
    not split (the caller then uses a GEMM)."""
    N = a.shape[0]
    S = 32
    if N % S != 0 or N < S * 512:
        return None
    if ones:
        a = torch.cat([a, torch.ones(N, 1, dtype=a.dtype, device=a.device)], 1)
    n = N // S
    # both bmm operands row-major and contiguous (the left one is [S, r, n], a small copy)
    lhs = a.reshape(S, n, a.shape[1]).transpose(1, 2).contiguous()
    p = torch.bmm(lhs, b.reshape(S, n, b.shape[1]))
    return p.to(torch.promote_types(p.dtype, torch.float32)).sum(0)


class _NarrowLinear(torch.autograd.Function):
    """``x W^T + bias`` for an input with few features (the low-rank gate's second matrix:
    16 -> key dim). The weight and bias gradients come from one split product over the rows
    (``_skinny_at_b`` with the column sums appended) instead of a GEMM over all rows plus a
    separate reduction for the bias."""

    @staticmethod
    def forward(ctx, x, weight, bias):
        ctx.save_for_backward(x, weight)
        ctx.has_bias = bias is not None
        return F.linear(x, weight, bias)

    @staticmethod
    def backward(ctx, dy):
        x, weight = ctx.saved_tensors
        x2 = x.reshape(-1, x.shape[-1])
        dy2 = dy.reshape(-1, dy.shape[-1])
        dx = (dy2 @ weight).view(x.shape) if ctx.needs_input_grad[0] else None
        dw = db = None
        if ctx.needs_input_grad[1] or (ctx.has_bias and ctx.needs_input_grad[2]):
            p = _skinny_at_b(x2, dy2, ones=ctx.has_bias)   # [r (+1), out]
            if p is None:
                dw = dy2.t() @ x2
                db = dy2.sum(0) if ctx.has_bias else None
            else:
                dw = p[:x2.shape[1]].t().to(weight.dtype)
                db = p[x2.shape[1]].to(weight.dtype) if ctx.has_bias else None
        return dx, dw, db


class _FanOutLinear(torch.autograd.Function):
    """``[x W_i^T for W_i in weights]``: bias-free projections of one input, forward as
    separate GEMMs, backward with the input gradient accumulated inside the GEMMs
    (``dx = dy_0 W_0``, then ``dx += dy_i W_i`` as the GEMMs' own accumulate). Autograd over
    separate ``F.linear`` calls instead sums the five contributions of the layer's hidden
    states with four elementwise adds of a [B, T, hidden] tensor (at B2 T16384 hidden 2048:
    4 x 60 us a step)."""

    @staticmethod
    def forward(ctx, x, *weights):
        ctx.set_materialize_grads(False)   # unused outputs: no gradient products
        ctx.save_for_backward(x, *weights)
        return tuple(F.linear(x, w) for w in weights)

    @staticmethod
    def backward(ctx, *dys):
        x, *weights = ctx.saved_tensors
        x2 = x.reshape(-1, x.shape[-1])
        dx2 = None
        dws = [None] * len(weights)
        want = [dy is not None and ctx.needs_input_grad[1 + i] for i, dy in enumerate(dys)]
        # the wide projections as one pair of GEMMs over their concatenated output gradient
        # Y = [dy_0 | dy_1 | ...]: dx = Y W_cat and dW_cat = Y^T x (K = 6144 and an output of
        # 6144 x 2048 at C5 instead of four GEMMs of 1024-2048 columns each)
        wide = [i for i, dy in enumerate(dys) if want[i] and dy.shape[-1] > 64]
        if len(wide) > 1:
            Y = _concat_cols([dys[i].reshape(-1, dys[i].shape[-1]).contiguous() for i in wide])
            W = torch.cat([weights[i] for i in wide], 0)
            if ctx.needs_input_grad[0]:
                dx2 = Y @ W
            dW = Y.t() @ x2
            o = 0
            for i in wide:
                n = weights[i].shape[0]
                dws[i] = dW[o:o + n]
                o += n
        else:
            wide = []
        for i, (w, dy) in enumerate(zip(weights, dys)):
            if dy is None or i in wide:
                continue
            dy2 = dy.reshape(-1, dy.shape[-1])
            if ctx.needs_input_grad[0]:
                dx2 = dy2 @ w if dx2 is None else dx2.addmm_(dy2, w)
            if ctx.needs_input_grad[1 + i]:
                # very narrow outputs (the low-rank gate): the split product over the rows;
                # narrow ones: x^T dy, transposed, a faster GEMM build than dy^T x (hipBLASLt,
                # [32768, 2048] x [32768, 1024]: 235 against 304 us)
                p = _skinny_at_b(dy2, x2) if dy2.shape[1] <= 64 else None
                if p is not None:
                    dws[i] = p.to(w.dtype)
                elif dy2.shape[1] < x2.shape[1]:
                    dws[i] = (x2.t() @ dy2).t()
                else:
                    dws[i] = dy2.t() @ x2
        dx = None
        if ctx.needs_input_grad[0]:
            dx = dx2.view(x.shape) if dx2 is not None else torch.zeros_like(x)
        return (dx, *dws)


def _to_heads(x, head_dim):
    """... (h d) -> ... h d"""
    return x.reshape(*x.shape[:-1], x.shape[-1] // head_dim, head_dim)


def _from_heads(x):
    """... h d -> ... (h d)"""
    return x.reshape(*x.shape[:-2], x.shape[-2] * x.shape[-1])


def _repeat_kv(x, groups, head_dim):
    """... (h d) -> ... (h g) d (reference ``_repeat_kv``, gla.py:49-66)."""
    x = _to_heads(x, head_dim)
    return x.unsqueeze(-2).expand(*x.shape[:-1], groups, head_dim).reshape(
        *x.shape[:-2], x.shape[-2] * groups, head_dim)


class LayerCache:
    """Minimal per-layer cache with the interface the layer uses (``len``, indexing by
    layer_idx, ``update(recurrent_state=, conv_state=, layer_idx=, offset=)``)."""

    def __init__(self):
        self.states: list[dict] = []
        self.seen_tokens = 0

    def __len__(self):
        return len(self.states)

    def __getitem__(self, i):
        return self.states[i]

    def update(self, recurrent_state=None, conv_state=None, layer_idx=0, offset=1):
        while len(self.states) <= layer_idx:
            self.states.append({"recurrent_state": None, "conv_state": None})
        self.states[layer_idx] = {"recurrent_state": recurrent_state, "conv_state": conv_state}
        if layer_idx == 0:
            self.seen_tokens += offset


class GatedLinearAttention(torch.nn.Module):
    r"""Gated Linear Attention (https://arxiv.org/abs/2312.06635).

    Arguments mirror ``tops/layers/gla.py:81-103``. ``rngs`` (keyword) may be an int seed or
    a ``torch.Generator`` for the weight init; ``device`` and ``dtype`` (parameter dtype,
    default float32 like Flax) are torch additions.
    """

    def __init__(self, mode="chunk", hidden_size=1024, expand_k=0.5, expand_v=1.0,
                 num_heads=4, num_kv_heads=None, feature_map=None, use_short_conv=False,
                 conv_size=4, conv_bias=False, use_output_gate=True, gate_fn="swish",
                 elementwise_affine=True, norm_eps=1e-5, gate_logit_normalizer=16,
                 gate_low_rank_dim=16, clamp_min=None, fuse_norm=True, layer_idx=None, *,
                 rngs=None, device=None, dtype=torch.float32):
        super().__init__()
        gen = rngs if isinstance(rngs, torch.Generator) else torch.Generator().manual_seed(
            0 if rngs is None else int(rngs))
        self.mode = mode
        self.hidden_size = hidden_size
        self.expand_k = expand_k
        self.expand_v = expand_v
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads if num_kv_heads is not None else num_heads
        self.num_kv_groups = self.num_heads // self.num_kv_heads
        self.feature_map_fn = ACT2FN[feature_map] if feature_map is not None else None
        self.use_short_conv = use_short_conv
        self.conv_size = conv_size
        self.conv_bias = conv_bias
        self.use_output_gate = use_output_gate
        self.key_dim = int(hidden_size * expand_k)
        self.value_dim = int(hidden_size * expand_v)
        self.key_dim_per_group = self.key_dim // self.num_kv_groups
        self.value_dim_per_group = self.value_dim // self.num_kv_groups
        self.clamp_min = clamp_min
        self.layer_idx = layer_idx

        require(mode in ["chunk", "fused_recurrent", "fused_chunk"],
                f"Not supported mode `{mode}`.")
        require(self.key_dim % num_heads == 0,
                f"key dim must be divisible by num_heads of {num_heads}")
        require(self.value_dim % num_heads == 0,
                f"value dim must be divisible by num_heads of {num_heads}")
        self.head_k_dim = self.key_dim // num_heads
        self.head_v_dim = self.value_dim // num_heads

        lin = lambda i, o, b=False: Linear(i, o, b, generator=gen, device=device,  # noqa: E731
                                           dtype=dtype)
        self.q_proj = lin(hidden_size, self.key_dim)
        self.k_proj = lin(hidden_size, self.key_dim_per_group)
        self.v_proj = lin(hidden_size, self.value_dim_per_group)
        if self.use_output_gate:
            self.g_proj = lin(hidden_size, self.value_dim)
        if use_short_conv:
            conv = lambda d: ShortConvolution(d, conv_size, bias=conv_bias,  # noqa: E731
                                              activation="silu", rngs=gen, device=device,
                                              dtype=dtype)
            self.q_conv1d = conv(self.key_dim)
            self.k_conv1d = conv(self.key_dim_per_group)
            self.v_conv1d = conv(self.value_dim_per_group)
        self.gk_proj = torch.nn.Sequential(lin(hidden_size, gate_low_rank_dim),
                                           lin(gate_low_rank_dim, self.key_dim_per_group, True))
        self.o_proj = lin(self.value_dim, hidden_size)
        if gate_fn == "swish" and fuse_norm and use_output_gate:
            self.g_norm_swish_gate = FusedRMSNormGated(self.head_v_dim, elementwise_affine,
                                                       norm_eps, device=device)
            self.fuse_norm_and_gate = True
        else:
            self.fuse_norm_and_gate = False
            self.g_norm = RMSNorm(self.head_v_dim, elementwise_affine, norm_eps, device=device)
            self.gate_fn_act = ACT2FN[gate_fn]
        self.gate_logit_normalizer = gate_logit_normalizer

    def forward(self, hidden_states, attention_mask=None, past_key_values: Any | None = None,
                use_cache=False, output_attentions=False, **kwargs):
        """Reference: ``GatedLinearAttention.__call__``, ``tops/layers/gla.py:224-345``."""
        if attention_mask is not None:
            require(attention_mask.dim() == 2,
                    "Expected attention_mask as a 0-1 matrix with shape [batch_size, seq_len].")
        batch_size, q_len, _ = hidden_states.shape
        mode = "fused_recurrent" if q_len <= 64 else self.mode

        last_state = None
        if past_key_values is not None and len(past_key_values) > self.layer_idx:
            last_state = past_key_values[self.layer_idx]
        cu_seqlens = kwargs.get("cu_seqlens")
        chunk_size = 16

        # the projections of the hidden states: one autograd node when they share its dtype
        # (the input gradient then accumulates inside the GEMMs)
        lins = [self.q_proj, self.k_proj, self.v_proj, self.gk_proj[0]]
        if self.use_output_gate:
            lins.append(self.g_proj)
        g = None
        if (torch.is_grad_enabled()
                and all(m.bias is None and m.weight.dtype == hidden_states.dtype for m in lins)):
            ys = _FanOutLinear.apply(hidden_states, *[m.weight for m in lins])
            up = self.gk_proj[1]
            q, k, v = ys[0], ys[1], ys[2]
            gk = (_NarrowLinear.apply(ys[3], up.weight, up.bias)
                  if up.weight.dtype == hidden_states.dtype and (
                      up.bias is None or up.bias.dtype == up.weight.dtype)
                  else up(ys[3]))
            if self.use_output_gate:
                g = ys[4]
        else:
            q = self.q_proj(hidden_states)
            k = self.k_proj(hidden_states)
            v = self.v_proj(hidden_states)
            gk = self.gk_proj(hidden_states)

        conv_state_q = conv_state_k = conv_state_v = None
        if self.use_short_conv:
            if last_state is not None and last_state.get("conv_state") is not None:
                conv_state_q, conv_state_k, conv_state_v = last_state["conv_state"]
            q, conv_state_q = self.q_conv1d(q, cache=conv_state_q, output_final_state=use_cache,
                                            cu_seqlens=cu_seqlens)
            k, conv_state_k = self.k_conv1d(k, cache=conv_state_k, output_final_state=use_cache,
                                            cu_seqlens=cu_seqlens)
            v, conv_state_v = self.v_conv1d(v, cache=conv_state_v, output_final_state=use_cache,
                                            cu_seqlens=cu_seqlens)

        q = _to_heads(q, self.head_k_dim)
        if self.num_kv_groups > 1:
            k = _repeat_kv(k, self.num_kv_groups, self.head_k_dim)
            gk = _repeat_kv(gk, self.num_kv_groups, self.head_k_dim)
            v = _repeat_kv(v, self.num_kv_groups, self.head_v_dim)
        else:
            k = _to_heads(k, self.head_k_dim)
            gk = _to_heads(gk, self.head_k_dim)
            v = _to_heads(v, self.head_v_dim)

        gk = GateLogSigmoidFn.apply(gk, self.gate_logit_normalizer, self.clamp_min)

        if self.feature_map_fn is not None:
            q = self.feature_map_fn(q)
            k = self.feature_map_fn(k)

        recurrent_state = last_state["recurrent_state"] if last_state is not None else None
        if mode == "fused_recurrent":
            o, recurrent_state = fused_recurrent_gla(q=q, k=k, v=v, gk=gk,
                                                     initial_state=recurrent_state,
                                                     output_final_state=use_cache,
                                                     cu_seqlens=cu_seqlens)
        elif mode == "fused_chunk":
            o, recurrent_state = fused_chunk_gla(q=q, k=k, v=v, g=gk,
                                                 initial_state=recurrent_state,
                                                 output_final_state=use_cache,
                                                 cu_seqlens=cu_seqlens)
        elif mode == "chunk":
            o, recurrent_state = chunk_gla(q=q, k=k, v=v, g=gk, initial_state=recurrent_state,
                                           output_final_state=use_cache, cu_seqlens=cu_seqlens,
                                           chunk_size=chunk_size)
        else:
            raise NotImplementedError(f"Not supported mode `{mode}`.")

        if past_key_values is not None:
            past_key_values.update(
                recurrent_state=recurrent_state,
                conv_state=(conv_state_q, conv_state_k, conv_state_v)
                if self.use_short_conv else None,
                layer_idx=self.layer_idx, offset=q_len)

        if self.use_output_gate:
            if g is None:
                g = self.g_proj(hidden_states)
            if self.fuse_norm_and_gate:
                g = _to_heads(g, self.head_v_dim)
                o = _from_heads(self.g_norm_swish_gate(o, g))
            else:
                o = _from_heads(self.g_norm(o))
                o = o * self.gate_fn_act(g)
        else:
            o = _from_heads(self.g_norm(o))
        o = self.o_proj(o)
        return o, None, past_key_values
