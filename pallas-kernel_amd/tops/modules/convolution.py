"""Causal depthwise short convolution. Reference: ``tops/modules/convolution.py:6-197``.

The prefill / training path runs on the ``tops_gla_short_conv_*`` kernels (forward and
backward); the single-token decode step (a roll of the cached window and one dot product per
channel) is host glue over torch ops, as in the reference.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from .. import _lib
from .._lib import call, check_device, dtype_code, ptr, stream_of


def _io_dtype(x):
    return x.dtype if x.dtype in (torch.float32, torch.bfloat16) else torch.float32


class _ShortConvFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w, bias, silu, cu):
        B, T, D = x.shape
        W = w.shape[-1]
        dev = check_device(x, w, bias)
        dt = _io_dtype(x)
        xx = x.to(dt).contiguous()
        ww = w.reshape(D, W).to(torch.float32).contiguous()
        bb = None if bias is None else bias.to(torch.float32).contiguous()
        seq = _lib.SeqLayout(B, T, 1, cu, dev)
        max_len = T if cu is None else max(b - a for a, b in zip(cu, cu[1:]))
        y = torch.empty_like(xx)
        call("tops_gla_short_conv_fwd", ptr(xx), ptr(ww), ptr(bb), ptr(y), B, T, D, W, int(silu),
             ptr(seq.cu), seq.N, max_len, dtype_code(dt), stream_of(dev))
        ctx.save_for_backward(xx, ww, bb)
        ctx.meta = (x.dtype, w.shape, w.dtype, silu, cu, seq, max_len)
        return y.to(x.dtype)

    @staticmethod
    def backward(ctx, dy):
        xx, ww, bb = ctx.saved_tensors
        xdt, wshape, wdt, silu, cu, seq, max_len = ctx.meta
        B, T, D = xx.shape
        W = ww.shape[-1]
        dev = xx.device
        dd = dy.to(xx.dtype).contiguous()
        dx = torch.empty_like(xx)
        want_w = ctx.needs_input_grad[1] or ctx.needs_input_grad[2]
        dwb = torch.empty((W + 1) * D, dtype=torch.float32, device=dev) if want_w else None
        nws = int(_lib.load().tops_gla_short_conv_ws_bytes(B, T, D, W, seq.N, max_len,
                                                          int(cu is not None))) if want_w else 0
        ws = torch.empty(nws, dtype=torch.uint8, device=dev) if nws else None
        call("tops_gla_short_conv_bwd", ptr(xx), ptr(ww), ptr(bb), ptr(dd), ptr(dx), ptr(dwb),
             ptr(ws), nws, B, T, D, W, int(silu), ptr(seq.cu), seq.N, max_len,
             dtype_code(xx.dtype), stream_of(dev))
        dw = db = None
        if want_w:
            dw = dwb[:D * W].reshape(wshape).to(wdt)
            db = dwb[D * W:].to(wdt) if bb is not None else None
        return dx.to(xdt), dw, db, None, None


class ShortConvolution(torch.nn.Module):
    """Depthwise causal conv1d (kernel ``conv_size``, groups = hidden_size) with optional bias
    and SiLU. ``weight`` is ``[D, 1, W]`` (torch Conv1d layout; the reference's Flax kernel is
    ``[W, 1, D]``). ``rngs``: int seed or ``torch.Generator`` for the init (uniform in
    +-1/sqrt(W), torch's Conv1d default scale)."""

    def __init__(self, hidden_size, kernel_size, bias=False, activation="silu", *, rngs=None,
                 device=None, dtype=torch.float32):
        super().__init__()
        self.hidden_size = hidden_size
        self.kernel_size = kernel_size
        self.activation = activation
        gen = rngs if isinstance(rngs, torch.Generator) else torch.Generator().manual_seed(
            0 if rngs is None else int(rngs))
        bound = 1.0 / math.sqrt(kernel_size)
        w = (torch.rand(hidden_size, 1, kernel_size, generator=gen) * 2 - 1) * bound
        self.weight = torch.nn.Parameter(w.to(device=device, dtype=dtype))
        if bias:
            b = (torch.rand(hidden_size, generator=gen) * 2 - 1) * bound
            self.bias = torch.nn.Parameter(b.to(device=device, dtype=dtype))
        else:
            self.register_parameter("bias", None)

    def _silu(self):
        return self.activation in ("silu", "swish")

    def step(self, x, cache, output_final_state=False, cu_seqlens=None):
        """Single-token decode. Reference: ``tops/modules/convolution.py:76-118``.
        x ``[B, 1, D]`` (or ``[1, N, D]`` with cu_seqlens); cache ``[N, W, D]``."""
        W, D = self.kernel_size, self.hidden_size
        N = x.shape[0] if cu_seqlens is None else len(_lib.to_list(cu_seqlens)) - 1
        if output_final_state and cache is None:
            cache = torch.zeros(N, W, D, dtype=x.dtype, device=x.device)
        x_step = x[0] if cu_seqlens is not None else x[:, 0, :]
        w = self.weight[:, 0, :].t()   # [W, D]
        if cache is not None:
            cache = torch.roll(cache, shifts=-1, dims=1)
            cache[:, -1, :] = x_step
            y = (cache * w).sum(dim=1)
        else:
            y = x_step * w[-1]
        if self.bias is not None:
            y = y + self.bias
        if self._silu():
            y = F.silu(y)
        return y.reshape(x.shape), cache

    def forward(self, x, cache=None, output_final_state=False, cu_seqlens=None, **kwargs):
        """Reference: ``tops/modules/convolution.py:120-197``. Returns ``(y, final_state)``,
        final_state ``[N, W, D]`` (the last W inputs of each sequence, zero-padded) or None."""
        B, T, D = x.shape
        cu = None if cu_seqlens is None else _lib.to_list(cu_seqlens)
        N = B if cu is None else len(cu) - 1
        W = self.kernel_size
        if B * T == N:
            return self.step(x, cache, output_final_state, cu_seqlens)
        y = _ShortConvFn.apply(x, self.weight, self.bias, self._silu(), cu)
        final_state = None
        if output_final_state:
            if cu is not None:
                segs = [x[0, a:b] for a, b in zip(cu, cu[1:])]
            else:
                segs = list(x)
            final_state = torch.stack(
                [F.pad(s, (0, 0, max(0, W - s.shape[0]), 0))[-W:] for s in segs])
        return y, final_state
