"""Standalone Qwen2 RMSNorm (input / final norm) with the optional fused fp16 output.

Mirrors the reference's solution/kernels/rmsnorm.py:104-188 (``_RMSNorm`` and
``rms_norm``): r = rsqrt(mean(x^2) + eps) and a = x r in fp32, q = cast(a,
x.dtype), y = weight q in promote(x, weight) or fp16 when out_dtype is
torch.float16; backward u = cast(g weight, x.dtype), dx = r (u - a mean(u a)),
dweight = sum over rows of g q (products rounded to fp16 when the exact output
dtype is fp16).  Kernels: ss_rmsnorm_fwd (the add-RMSNorm row kernel without
the residual add), and for the backward the add-RMSNorm backward with s = x
and no residual gradient (ss_add_rmsnorm_bwd, or ss_add_rmsnorm_bwd_dgamma
when the weight is trained).  Saves x, the weight and one fp32 rstd per row.
"""

import math
import numbers

import torch
from torch.autograd.function import once_differentiable

from .. import _lib


def _code(t):
    return _lib.dtype_code(t.dtype)


class _RMSNorm(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, eps, out_dtype):
        h = x.shape[-1]
        rows = math.prod(x.shape[:-1])
        exact = torch.promote_types(x.dtype, weight.dtype)
        out = torch.empty(x.shape, device=x.device, dtype=out_dtype or exact)
        rstd = torch.empty(rows, device=x.device, dtype=torch.float32)
        if rows:
            matrix = x if x.ndim == 2 else x.view(rows, h)
            _lib.call("ss_rmsnorm_fwd", matrix.data_ptr(), _code(x), matrix.stride(0),
                      weight.data_ptr(), _code(weight), weight.stride(0), out.data_ptr(),
                      _code(out), rstd.data_ptr(), rows, h, float(eps), _lib.stream(x.device))
        ctx.save_for_backward(x, weight, rstd)
        ctx.exact_dtype, ctx.rows = exact, rows
        ctx.set_materialize_grads(False)
        return out

    @staticmethod
    @once_differentiable
    def backward(ctx, grad):
        if grad is None:
            return None, None, None, None
        x, weight, rstd = ctx.saved_tensors
        h, rows = x.shape[-1], ctx.rows
        need_x, need_w = ctx.needs_input_grad[:2]
        dx = torch.empty(x.shape, device=x.device, dtype=x.dtype) if need_x else None
        dw = torch.empty(weight.shape, device=weight.device, dtype=weight.dtype) if need_w else None
        if not rows:
            if dw is not None:
                dw.zero_()
            return dx, dw, None, None
        s = x.reshape(rows, h).contiguous()
        g = grad.reshape(rows, h)
        stream = _lib.stream(x.device)
        half_products = int(ctx.exact_dtype == torch.float16)
        if need_w:
            waves = _lib.load().ss_add_rmsnorm_dgamma_waves(rows)
            partial = torch.empty((waves, h), device=x.device, dtype=torch.float32)
            _lib.call("ss_add_rmsnorm_bwd_dgamma", s.data_ptr(), _code(s), weight.data_ptr(),
                      _code(weight), weight.stride(0), rstd.data_ptr(), None, 0, 0, 0,
                      g.data_ptr(), _code(g), g.stride(0), g.stride(1), _lib.ptr(dx),
                      _code(dx) if dx is not None else 0, None, 0, half_products,
                      partial.data_ptr(), dw.data_ptr(), _code(dw), rows, h, stream)
        elif need_x:
            _lib.call("ss_add_rmsnorm_bwd", s.data_ptr(), _code(s), weight.data_ptr(),
                      _code(weight), weight.stride(0), rstd.data_ptr(), None, 0, 0, 0,
                      g.data_ptr(), _code(g), g.stride(0), g.stride(1), dx.data_ptr(), _code(dx),
                      None, 0, rows, h, stream)
        return dx, dw, None, None


def rms_norm(x, weight, eps, out_dtype=None):
    """Normalize the last dimension with Qwen2 cast semantics (reference rmsnorm.py:159-188).

    fp16/fp32 CUDA input, contiguous or a 2-D row-strided layout, and a 1-D
    fp16/fp32 weight.  out_dtype=None keeps the promoted dtype; torch.float16
    fuses the final cast.  Invalid inputs raise ValueError.
    """
    if (x.ndim < 1 or x.shape[-1] == 0 or weight.ndim != 1
            or weight.shape[0] != x.shape[-1]):
        raise ValueError("Expected x[...,H] and weight[H] with positive H")
    if not x.is_cuda or weight.device != x.device:
        raise ValueError("x and weight must be on the same CUDA device")
    if x.stride(-1) != 1:
        raise ValueError("The last input dimension must be contiguous")
    if not x.is_contiguous() and x.ndim != 2:
        raise ValueError("Noncontiguous leading dimensions require a 2-D input")
    if (x.dtype not in (torch.float16, torch.float32)
            or weight.dtype not in (torch.float16, torch.float32)):
        raise ValueError("RMSNorm supports only fp16/fp32 input and weight")
    if not isinstance(eps, numbers.Real) or not math.isfinite(eps) or eps < 0:
        raise ValueError("eps must be a finite nonnegative scalar")
    if out_dtype not in (None, torch.float16):
        raise ValueError("out_dtype must be None or torch.float16")
    with torch.cuda.device(x.device):
        return _RMSNorm.apply(x, weight, eps, out_dtype)
