"""NF4 dequantize-fused GEMM: forward Y = X.W^T (+bias) and backward dX = dY.W.

Host side of ss_nf4_gemm_fwd / ss_nf4_gemm_dx.  Mirrors the reference's
solution/kernels/nf4_gemm.py:74-118 (``nf4_matmul`` and the ``_NF4Linear``
autograd node that saves only the packed weight and its state), but the
kernel is the MI355X MFMA engine in csrc/gemm.hip and it is the default path
for every shape, not an allow-listed experiment.

Path selection (all on the GPU):
  * K % 64 == 0 and a 16-byte aligned packed buffer: the fused kernel decodes
    W tiles in registers straight into LDS (small and mid T), or -- when
    ss_nf4_gemm_workspace_size() asks for it (large T) -- decodes W once into
    a caller workspace and runs the dense fp16 MFMA GEMM;
  * any other shape: ss_nf4_dequant_nested into a temporary + ss_gemm_f16.
The decoded weight is bit-exact in every path; GEMM outputs differ from a
float64 product only by fp32 accumulation order and the final fp16 rounding.
"""

import torch
from torch.autograd.function import once_differentiable

from .. import _lib
from ..contract import Rule, enforce
from .nf4 import _validate_state


def _fused_ok(packed, k):
    return k % 64 == 0 and packed.data_ptr() % 16 == 0


def _workspace(t, n, k, device):
    size = _lib.load().ss_nf4_gemm_workspace_size(t, n, k)
    if size == 0:
        return None, 0
    return torch.empty(size, dtype=torch.uint8, device=device), size


def _dense_weight(packed, state, n, k):
    w = torch.empty((n, k), device=packed.device, dtype=torch.float16)
    _lib.call("ss_nf4_dequant_nested", packed.data_ptr(), state.absmax.data_ptr(),
              state.state2.absmax.data_ptr(), state.state2.code.data_ptr(),
              state.offset.data_ptr(), w.data_ptr(), n * k, _lib.stream(packed.device))
    return w


def gemm_f16(a, b, *, a_trans=False, b_trans=False, out=None, out_dtype=torch.float16,
             alpha=1.0, accumulate=False, bias=None, split_k=False, alpha_dev=None):
    """C = alpha * op(A) . op(B) (+bias) (+C) on the MFMA engine (ss_gemm_f16).

    a: [M,K] (or [K,M] when a_trans), b: [K,N] (or [N,K] when b_trans); fp16,
    row-major with unit column stride.  Returns C [M,N] of out_dtype.
    split_k: give the dense NT kernel scratch to split a long reduction over
    workgroups when the output has few tiles (ss_gemm_f16_split).  alpha_dev: a
    one-element fp32 device tensor multiplying alpha (no host synchronisation).
    """
    if a.dtype != torch.float16 or b.dtype != torch.float16:
        raise ValueError("gemm_f16 expects fp16 operands")
    if a.stride(-1) != 1 or b.stride(-1) != 1 or a.ndim != 2 or b.ndim != 2:
        raise ValueError("gemm_f16 expects 2-D operands with unit column stride")
    m, k = (a.shape[1], a.shape[0]) if a_trans else a.shape
    kb, n = (b.shape[1], b.shape[0]) if b_trans else b.shape
    if k != kb:
        raise ValueError(f"gemm_f16: inner dimensions differ ({k} vs {kb})")
    if out is None:
        if accumulate:
            raise ValueError("accumulate requires out")
        out = torch.empty((m, n), device=a.device, dtype=out_dtype)
    if out.shape != (m, n) or out.stride(-1) != 1:
        raise ValueError("gemm_f16: bad output buffer")
    if alpha_dev is not None and (alpha_dev.dtype != torch.float32 or alpha_dev.numel() != 1
                                  or alpha_dev.device != a.device):
        raise ValueError("gemm_f16: alpha_dev must be one fp32 element on the operands' device")
    size = _lib.load().ss_gemm_f16_workspace_size(int(a_trans), int(b_trans), m, n, k) \
        if split_k else 0
    if size or alpha_dev is not None:
        ws = torch.empty(size, dtype=torch.uint8, device=a.device) if size else None
        _lib.call("ss_gemm_f16_split", int(a_trans), int(b_trans), m, n, k, float(alpha),
                  _lib.ptr(alpha_dev), a.data_ptr(), a.stride(0), b.data_ptr(), b.stride(0),
                  _lib.ptr(bias), 1.0 if accumulate else 0.0, out.data_ptr(),
                  _lib.dtype_code(out.dtype), out.stride(0), _lib.ptr(ws), size,
                  _lib.stream(a.device))
        return out
    _lib.call("ss_gemm_f16", int(a_trans), int(b_trans), m, n, k, float(alpha), a.data_ptr(),
              a.stride(0), b.data_ptr(), b.stride(0), _lib.ptr(bias), 1.0 if accumulate else 0.0,
              out.data_ptr(), _lib.dtype_code(out.dtype), out.stride(0), _lib.stream(a.device))
    return out


def nf4_forward_2d(x2d, packed, state, n, k, bias=None, out=None):
    """y[T,N] = x2d[T,K] . Wdec^T (+bias) into ``out`` (allocated if None)."""
    t = x2d.shape[0]
    if out is None:
        out = torch.empty((t, n), device=x2d.device, dtype=torch.float16)
    if t == 0:
        return out
    stream = _lib.stream(x2d.device)
    if _fused_ok(packed, k):
        ws, size = _workspace(t, n, k, x2d.device)
        _lib.call("ss_nf4_gemm_fwd", x2d.data_ptr(), x2d.stride(0), t, packed.data_ptr(),
                  state.absmax.data_ptr(), state.state2.absmax.data_ptr(),
                  state.state2.code.data_ptr(), state.offset.data_ptr(), n, k, _lib.ptr(bias),
                  out.data_ptr(), out.stride(0), _lib.ptr(ws), size, stream)
    else:
        gemm_f16(x2d, _dense_weight(packed, state, n, k), b_trans=True, out=out, bias=bias)
    return out


def nf4_dx_2d(dy2d, packed, state, n, k, out=None, accumulate=False):
    """dx[T,K] = dy2d[T,N] . Wdec (+ out when accumulate)."""
    t = dy2d.shape[0]
    if out is None:
        out = torch.empty((t, k), device=dy2d.device, dtype=torch.float16)
    if t == 0:
        return out
    stream = _lib.stream(dy2d.device)
    if _fused_ok(packed, k):
        ws, size = _workspace(t, n, k, dy2d.device)
        _lib.call("ss_nf4_gemm_dx", dy2d.data_ptr(), dy2d.stride(0), t, packed.data_ptr(),
                  state.absmax.data_ptr(), state.state2.absmax.data_ptr(),
                  state.state2.code.data_ptr(), state.offset.data_ptr(), n, k, out.data_ptr(),
                  out.stride(0), int(accumulate), _lib.ptr(ws), size, stream)
    else:
        gemm_f16(dy2d, _dense_weight(packed, state, n, k), out=out, accumulate=accumulate)
    return out


def _activation_ok(a):
    x = a.x
    return (isinstance(x, torch.Tensor) and x.device == a.packed.device and x.ndim >= 2
            and x.shape[-1] == a.width_in)


def _bias_ok(a):
    b = a.bias
    if b is None:
        return True
    return (not a.transpose and isinstance(b, torch.Tensor) and b.device == a.x.device
            and b.dtype == torch.float16 and tuple(b.shape) == (a.width_out,)
            and b.is_contiguous() and not b.requires_grad)


# nf4_matmul's operands once the NF4 state itself is accepted (NESTED_STATE_RULES).
MATMUL_RULES = (
    Rule("nf4_matmul: the activation must be a tensor of two or more dimensions on the "
         "weight's CUDA device whose last extent is the product's reduction length",
         _activation_ok),
    Rule("nf4_matmul: the activation must be fp16 and contiguous",
         lambda a: a.x.dtype == torch.float16 and a.x.is_contiguous()),
    Rule("nf4_matmul: a bias belongs to the forward product only, as a frozen contiguous "
         "fp16 vector of the output width", _bias_ok),
)


def nf4_matmul(x, packed, state, *, transpose=False, bias=None):
    """X[..., K] . W^T (+bias) or, with transpose, dY[..., N] . W (reference nf4_gemm.py:74-96)."""
    n, k = _validate_state(packed, state, torch.float16)
    width = k if transpose else n
    enforce(MATMUL_RULES, x=x, packed=packed, bias=bias, transpose=transpose,
            width_in=n if transpose else k, width_out=width)
    m = x.numel() // x.shape[-1]
    x2d = x.reshape(m, x.shape[-1])
    with torch.cuda.device(x.device):
        if transpose:
            out = nf4_dx_2d(x2d, packed, state, n, k)
        else:
            out = nf4_forward_2d(x2d, packed, state, n, k, bias=bias)
    return out.reshape(*x.shape[:-1], width)


class NF4Linear(torch.autograd.Function):
    """Frozen NF4 linear: saves the packed weight and its state only (reference nf4_gemm.py:99-118)."""

    @staticmethod
    def forward(ctx, x, packed, state, bias):
        ctx.save_for_backward(packed)
        ctx.state = state
        return nf4_matmul(x, packed, state, bias=bias)

    @staticmethod
    @once_differentiable
    def backward(ctx, grad):
        (packed,) = ctx.saved_tensors
        dx = nf4_matmul(grad.contiguous(), packed, ctx.state, transpose=True)
        return dx, None, None, None
