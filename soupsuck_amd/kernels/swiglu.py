"""SwiGLU activation of the Qwen2 MLP: silu(gate) * up and both derivatives.

Mirrors the reference's solution/kernels/swiglu_fused.py:49-78
(``swiglu_fused_forward`` / ``swiglu_fused_backward`` over the 2-D
``swiglu_tile_engine``): the leading dimensions are flattened into rows, every
operand keeps its own strides and dtype (fp16 or fp32), the arithmetic is fp32
with p = 1/(1+exp(-g)), act = g p, a = act u, dg = (da u)(p + act(1-p)),
du = da act.  Kernels: ss_swiglu_fwd / ss_swiglu_bwd (HBM-bound, one pass).
``SwiGLU`` / ``swiglu`` are the autograd form of solution/swiglu.py:40-65.
"""

import math

import torch

from .. import _lib


def _matrix(t):
    cols = t.shape[-1] if t.ndim else 1
    return t.reshape(math.prod(t.shape[:-1]), cols)


def _out_matrix(t):
    try:
        return t.view(math.prod(t.shape[:-1]), t.shape[-1])
    except RuntimeError as exc:
        raise ValueError("swiglu output buffer must be viewable as [rows, cols]") from exc


def _args(m):
    return (m.data_ptr(), _lib.dtype_code(m.dtype), m.stride(0), m.stride(1))


def _check(*tensors):
    shape, device = tensors[0].shape, tensors[0].device
    for t in tensors:
        if t.shape != shape:
            raise ValueError(f"swiglu operands differ in shape: {tuple(t.shape)} vs {tuple(shape)}")
        if t.device != device or not t.is_cuda:
            raise ValueError("swiglu operands must be on one CUDA device")
        _lib.dtype_code(t.dtype)


def swiglu_fused_forward(gate, up, out=None):
    """Fill ``out`` (or a new gate-dtype tensor) with silu(gate) * up."""
    if out is None:
        out = torch.empty_like(gate)
    _check(gate, up, out)
    g, u, a = _matrix(gate), _matrix(up), _out_matrix(out)
    rows, cols = g.shape
    if rows and cols:
        _lib.call("ss_swiglu_fwd", *_args(g), *_args(u), *_args(a), rows, cols,
                  _lib.stream(gate.device))
    return out


def swiglu_fused_backward(gate, up, grad, gate_dtype=None, up_dtype=None):
    """Return (dgate, dup) in gate_dtype / up_dtype (default: the inputs' dtypes)."""
    dgate = torch.empty(gate.shape, device=gate.device, dtype=gate_dtype or gate.dtype)
    dup = torch.empty(up.shape, device=up.device, dtype=up_dtype or up.dtype)
    _check(gate, up, grad, dgate, dup)
    g, u, da = _matrix(gate), _matrix(up), _matrix(grad)
    dg, du = _out_matrix(dgate), _out_matrix(dup)
    rows, cols = g.shape
    if rows and cols:
        _lib.call("ss_swiglu_bwd", *_args(g), *_args(u), *_args(da), *_args(dg), *_args(du), rows,
                  cols, _lib.stream(gate.device))
    return dgate, dup


class SwiGLU(torch.autograd.Function):
    """silu(gate) * up with one kernel each way; saves gate and up."""

    @staticmethod
    def forward(ctx, gate, up):
        up = up.to(gate.dtype)
        out = swiglu_fused_forward(gate, up)
        ctx.save_for_backward(gate, up)
        ctx.up_dtype = up.dtype
        return out

    @staticmethod
    def backward(ctx, grad):
        gate, up = ctx.saved_tensors
        dgate, dup = swiglu_fused_backward(gate, up, grad.to(gate.dtype))
        return dgate, dup


def swiglu(gate, up):
    return SwiGLU.apply(gate, up)
