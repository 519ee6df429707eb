"""Autograd functions over the norm / gate kernels of ``tops_gla_rmsnorm_gated_*`` and
``tops_gla_gate_logsigmoid_*``."""

from __future__ import annotations

import torch

from .. import _lib
from .._lib import call, check_device, dtype_code, ptr, stream_of


def _io_dtype(x):
    return x.dtype if x.dtype in (torch.float32, torch.bfloat16) else torch.float32


class RMSNormGatedFn(torch.autograd.Function):
    """y = x rsqrt(mean(x^2) + eps) [* w] [* silu(g)] over the last dimension, computed in
    float32, returned in x's dtype."""

    @staticmethod
    def forward(ctx, x, g, w, eps):
        dev = check_device(x, g, w)
        dt = _io_dtype(x)
        D = x.shape[-1]
        xx = x.to(dt).contiguous()
        gg = None if g is None else g.to(dt).contiguous()
        ww = None if w is None else w.to(torch.float32).contiguous()
        rows = xx.numel() // D if D else 0
        y = torch.empty_like(xx)
        rstd = torch.empty(rows, dtype=torch.float32, device=dev)
        call("tops_gla_rmsnorm_gated_fwd", ptr(xx), ptr(gg), ptr(ww), ptr(y), ptr(rstd), rows, D,
             float(eps), dtype_code(dt), stream_of(dev))
        ctx.save_for_backward(xx, gg, ww, rstd)
        ctx.meta = (x.dtype, None if g is None else g.dtype, None if w is None else w.dtype)
        return y.to(x.dtype)

    @staticmethod
    def backward(ctx, dy):
        xx, gg, ww, rstd = ctx.saved_tensors
        xdt, gdt, wdt = ctx.meta
        dev = xx.device
        D = xx.shape[-1]
        rows = rstd.numel()
        dd = dy.to(xx.dtype).contiguous()
        dx = torch.empty_like(xx)
        dg = None if gg is None else torch.empty_like(gg)
        want_dw = ww is not None and ctx.needs_input_grad[2]
        dw = torch.empty(D, dtype=torch.float32, device=dev) if want_dw else None
        nws = int(_lib.load().tops_gla_rmsnorm_ws_bytes(rows, D)) if want_dw else 0
        ws = torch.empty(nws, dtype=torch.uint8, device=dev) if nws else None
        call("tops_gla_rmsnorm_gated_bwd", ptr(xx), ptr(gg), ptr(ww), ptr(rstd), ptr(dd), ptr(dx),
             ptr(dg), ptr(dw), ptr(ws), nws, rows, D, dtype_code(xx.dtype), stream_of(dev))
        return (dx.to(xdt), None if dg is None else dg.to(gdt),
                None if dw is None else dw.to(wdt), None)


class GateLogSigmoidFn(torch.autograd.Function):
    """y = max(log_sigmoid(x) / normalizer, clamp_min) (clamp when clamp_min is not None)."""

    @staticmethod
    def forward(ctx, x, normalizer, clamp_min):
        dev = check_device(x)
        dt = _io_dtype(x)
        xx = x.to(dt).contiguous()
        y = torch.empty_like(xx)
        has = clamp_min is not None
        call("tops_gla_gate_logsigmoid_fwd", ptr(xx), ptr(y), xx.numel(), float(normalizer),
             int(has), float(clamp_min if has else 0.0), dtype_code(dt), stream_of(dev))
        ctx.save_for_backward(xx)
        ctx.meta = (x.dtype, float(normalizer), clamp_min)
        return y.to(x.dtype)

    @staticmethod
    def backward(ctx, dy):
        (xx,) = ctx.saved_tensors
        xdt, normalizer, clamp_min = ctx.meta
        dd = dy.to(xx.dtype).contiguous()
        dx = torch.empty_like(xx)
        has = clamp_min is not None
        call("tops_gla_gate_logsigmoid_bwd", ptr(xx), ptr(dd), ptr(dx), xx.numel(), normalizer,
             int(has), float(clamp_min if has else 0.0), dtype_code(xx.dtype),
             stream_of(xx.device))
        return dx.to(xdt), None, None
