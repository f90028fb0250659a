"""Residual addition and Qwen2 RMSNorm in one forward/backward row pass (A13-A15).

Mirrors the reference's solution/kernels/add_rmsnorm.py:84-161 (the
``_AddRMSNorm`` autograd node and ``add_rms_norm`` validation):
s = cast(residual + delta, promote), y = weight * cast(s * rstd, s.dtype) in
promote(s, weight) or fp16 when out_dtype=torch.float16; backward
ds = cast(rstd (u - a mean(u a))) + g_s with u = cast(g_y w); dgamma is the
two-stage non-atomic reduction of g_y * q (products rounded to fp16 when the
exact output dtype is fp16).  Kernels: ss_add_rmsnorm_fwd / _bwd, and
ss_add_rmsnorm_bwd_dgamma when the weight is trained (input gradients and the
per-wave column sums of dgamma in one pass over s and gy, then an in-order
sum of the wave partials).  Saves only s, the weight and one fp32 rstd per row.
"""

import math
import numbers

import torch
from torch.autograd.function import once_differentiable

from .. import _lib


def _code(t):
    return _lib.dtype_code(t.dtype)


class _AddRMSNorm(torch.autograd.Function):
    @staticmethod
    def forward(ctx, residual, delta, weight, eps, out_dtype):
        h = residual.shape[-1]
        rows = math.prod(residual.shape[:-1])
        sum_dtype = torch.promote_types(residual.dtype, delta.dtype)
        exact_dtype = torch.promote_types(sum_dtype, weight.dtype)
        new_residual = torch.empty(residual.shape, device=residual.device, dtype=sum_dtype)
        normed = torch.empty(residual.shape, device=residual.device,
                             dtype=out_dtype or exact_dtype)
        rstd = torch.empty(rows, device=residual.device, dtype=torch.float32)
        if rows:
            _lib.call("ss_add_rmsnorm_fwd", residual.data_ptr(), _code(residual), delta.data_ptr(),
                      _code(delta), weight.data_ptr(), _code(weight), weight.stride(0),
                      new_residual.data_ptr(), _code(new_residual), normed.data_ptr(),
                      _code(normed), rstd.data_ptr(), rows, h, float(eps),
                      _lib.stream(residual.device))
        ctx.save_for_backward(new_residual, weight, rstd)
        ctx.residual_dtype, ctx.delta_dtype = residual.dtype, delta.dtype
        ctx.exact_dtype, ctx.rows = exact_dtype, rows
        ctx.set_materialize_grads(False)
        return new_residual, normed

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_residual, grad_normed):
        s, weight, rstd = ctx.saved_tensors
        rows, h = ctx.rows, s.shape[-1]
        need_r, need_d, need_w = ctx.needs_input_grad[:3]
        dr = torch.empty(s.shape, device=s.device, dtype=ctx.residual_dtype) if need_r else None
        dd = torch.empty(s.shape, device=s.device, dtype=ctx.delta_dtype) if need_d else None
        dw = None
        stream = _lib.stream(s.device)
        if need_w and rows and grad_normed is not None:
            # dr / dd and the weight gradient in one pass over s and gy.
            gs = grad_residual.reshape(rows, h) if grad_residual is not None else None
            gy = grad_normed.reshape(rows, h)
            waves = _lib.load().ss_add_rmsnorm_dgamma_waves(rows)
            partial = torch.empty((waves, h), device=s.device, dtype=torch.float32)
            dw = torch.empty(weight.shape, device=weight.device, dtype=weight.dtype)
            _lib.call("ss_add_rmsnorm_bwd_dgamma", s.data_ptr(), _code(s), weight.data_ptr(),
                      _code(weight), weight.stride(0), rstd.data_ptr(), _lib.ptr(gs),
                      _code(gs) if gs is not None else 0,
                      gs.stride(0) if gs is not None else 0, gs.stride(1) if gs is not None else 0,
                      gy.data_ptr(), _code(gy), gy.stride(0), gy.stride(1),
                      _lib.ptr(dr), _code(dr) if dr is not None else 0, _lib.ptr(dd),
                      _code(dd) if dd is not None else 0,
                      int(ctx.exact_dtype == torch.float16), partial.data_ptr(), dw.data_ptr(),
                      _code(dw), rows, h, stream)
            return dr, dd, dw, None, None
        if rows and (need_r or need_d):
            gs = grad_residual.reshape(rows, h) if grad_residual is not None else None
            gy = grad_normed.reshape(rows, h) if grad_normed is not None else None
            _lib.call("ss_add_rmsnorm_bwd", s.data_ptr(), _code(s), weight.data_ptr(),
                      _code(weight), weight.stride(0), rstd.data_ptr(), _lib.ptr(gs),
                      _code(gs) if gs is not None else 0,
                      gs.stride(0) if gs is not None else 0, gs.stride(1) if gs is not None else 0,
                      _lib.ptr(gy), _code(gy) if gy is not None else 0,
                      gy.stride(0) if gy is not None else 0, gy.stride(1) if gy is not None else 0,
                      _lib.ptr(dr), _code(dr) if dr is not None else 0, _lib.ptr(dd),
                      _code(dd) if dd is not None else 0, rows, h, stream)
        if need_w:
            dw = torch.zeros(weight.shape, device=weight.device, dtype=weight.dtype)
            if rows and grad_normed is not None:
                gy = grad_normed.reshape(rows, h)
                groups = -(-rows // 32)
                partial = torch.empty((groups, h), device=s.device, dtype=torch.float32)
                _lib.call("ss_rmsnorm_dgamma", s.data_ptr(), _code(s), rstd.data_ptr(),
                          gy.data_ptr(), _code(gy), gy.stride(0), gy.stride(1),
                          int(ctx.exact_dtype == torch.float16), partial.data_ptr(),
                          dw.data_ptr(), _code(dw), rows, h, stream)
        return dr, dd, dw, None, None


def add_rms_norm(residual, delta, weight, eps, out_dtype=None):
    """Return residual+delta and its Qwen2 RMSNorm; inputs must be contiguous CUDA.

    residual/delta/weight support fp16/fp32; out_dtype is None (exact eager
    promotion) or torch.float16.  Invalid inputs raise ValueError before any
    launch (reference add_rmsnorm.py:139-161).
    """
    if residual.shape != delta.shape or residual.ndim < 1 or residual.shape[-1] == 0:
        raise ValueError("Expected matching residual/delta [...,H] with positive H")
    if weight.ndim != 1 or weight.shape[0] != residual.shape[-1]:
        raise ValueError("Expected weight[H]")
    if not residual.is_cuda or delta.device != residual.device or weight.device != residual.device:
        raise ValueError("All inputs must be on the same CUDA device")
    if not residual.is_contiguous() or not delta.is_contiguous():
        raise ValueError("residual and delta must be contiguous")
    if any(t.dtype not in (torch.float16, torch.float32) for t in (residual, delta, weight)):
        raise ValueError("Only fp16/fp32 inputs are supported")
    if out_dtype not in (None, torch.float16):
        raise ValueError("out_dtype must be None or torch.float16")
    if not isinstance(eps, numbers.Real) or not math.isfinite(eps) or eps < 0:
        raise ValueError("eps must be a finite nonnegative scalar")
    with torch.cuda.device(residual.device):
        return _AddRMSNorm.apply(residual, delta, weight, eps, out_dtype)
