"""One autograd node for both Qwen2 row norms: with and without the residual add.

The add-RMSNorm (solution/kernels/add_rmsnorm.py:1-24) and the standalone
RMSNorm (solution/kernels/rmsnorm.py:1-14) are the same row computation; the
plain norm is the add-RMSNorm with no delta, where s = x.  Semantics, in the
reference's order of casts:

  forward   s = cast(r + d, promote(r, d))              (plain norm: s = x)
            rstd = rsqrt(mean(fp32(s)^2) + eps)         (fp32, saved per row)
            y = w * cast(s * rstd, s.dtype)  in promote(s, w), or fp16 when asked
  backward  a = s rstd, u = cast(g_y w, s.dtype)
            ds = rstd (u - a mean(u a)) (+ g_s), cast to each input's dtype
            dw = sum over rows of g_y * cast(a, s.dtype)  (products rounded to
                 fp16 when promote(s, w) is fp16)

Launches: ss_add_rmsnorm_fwd / ss_rmsnorm_fwd; the backward is one pass of
ss_add_rmsnorm_bwd_dgamma when the weight is trained (input gradients and the
column partial sums together, then an in-order sum of the partials), else
ss_add_rmsnorm_bwd.  Saved: s, the weight and the fp32 rstd.
"""

import math

import torch
from torch.autograd.function import once_differentiable

from .. import _lib


def _dt(t):
    return 0 if t is None else _lib.dtype_code(t.dtype)


def _strides(t):
    return (0, 0) if t is None else (t.stride(0), t.stride(1))


def _as_rows(t, rows, h):
    return None if t is None else t.reshape(rows, h)


class _Layout:
    """Dtypes and sizes of one norm call (computed once, kept for the backward)."""

    def __init__(self, x, delta, weight, out_dtype):
        self.h = x.shape[-1]
        self.rows = math.prod(x.shape[:-1])
        self.x_dtype = x.dtype
        self.delta_dtype = None if delta is None else delta.dtype
        self.s_dtype = x.dtype if delta is None else torch.promote_types(x.dtype, delta.dtype)
        self.exact_dtype = torch.promote_types(self.s_dtype, weight.dtype)
        self.y_dtype = out_dtype or self.exact_dtype

    @property
    def half_products(self):
        return int(self.exact_dtype == torch.float16)


def _forward_launch(lay, x, delta, weight, eps):
    """Return (s, y, rstd); s is x itself for the plain norm."""
    dev = x.device
    y = torch.empty(x.shape, device=dev, dtype=lay.y_dtype)
    rstd = torch.empty(lay.rows, device=dev, dtype=torch.float32)
    if delta is None:
        s = x
        if lay.rows:
            rows2d = x if x.ndim == 2 else x.view(lay.rows, lay.h)
            _lib.call("ss_rmsnorm_fwd", rows2d.data_ptr(), _dt(x), rows2d.stride(0),
                      weight.data_ptr(), _dt(weight), weight.stride(0), y.data_ptr(), _dt(y),
                      rstd.data_ptr(), lay.rows, lay.h, float(eps), _lib.stream(dev))
        return s, y, rstd
    s = torch.empty(x.shape, device=dev, dtype=lay.s_dtype)
    if lay.rows:
        _lib.call("ss_add_rmsnorm_fwd", x.data_ptr(), _dt(x), delta.data_ptr(), _dt(delta),
                  weight.data_ptr(), _dt(weight), weight.stride(0), s.data_ptr(), _dt(s),
                  y.data_ptr(), _dt(y), rstd.data_ptr(), lay.rows, lay.h, float(eps),
                  _lib.stream(dev))
    return s, y, rstd


def _backward_launch(lay, s, weight, rstd, g_s, g_y, want):
    """Gradients (d_x, d_delta, d_weight) for the flags in ``want``."""
    want_x, want_d, want_w = want
    dev = s.device
    d_x = torch.empty(s.shape, device=dev, dtype=lay.x_dtype) if want_x else None
    d_d = torch.empty(s.shape, device=dev, dtype=lay.delta_dtype) if want_d else None
    rows, h = lay.rows, lay.h
    s2 = s.reshape(rows, h).contiguous() if rows else s
    gs2, gy2 = _as_rows(g_s, rows, h), _as_rows(g_y, rows, h)
    stream = _lib.stream(dev)
    state = (s2.data_ptr(), _dt(s2), weight.data_ptr(), _dt(weight), weight.stride(0),
             rstd.data_ptr(), _lib.ptr(gs2), _dt(gs2), *_strides(gs2))
    if want_w and rows and gy2 is not None:
        d_w = torch.empty(weight.shape, device=weight.device, dtype=weight.dtype)
        partial = torch.empty((_lib.load().ss_add_rmsnorm_dgamma_waves(rows), h), device=dev,
                              dtype=torch.float32)
        _lib.call("ss_add_rmsnorm_bwd_dgamma", *state, gy2.data_ptr(), _dt(gy2), *_strides(gy2),
                  _lib.ptr(d_x), _dt(d_x), _lib.ptr(d_d), _dt(d_d), lay.half_products,
                  partial.data_ptr(), d_w.data_ptr(), _dt(d_w), rows, h, stream)
        return d_x, d_d, d_w
    if rows and (want_x or want_d):
        _lib.call("ss_add_rmsnorm_bwd", *state, _lib.ptr(gy2), _dt(gy2), *_strides(gy2),
                  _lib.ptr(d_x), _dt(d_x), _lib.ptr(d_d), _dt(d_d), rows, h, stream)
    # No output gradient reaches the weight (or there are no rows): zero.
    d_w = torch.zeros(weight.shape, device=weight.device, dtype=weight.dtype) if want_w else None
    return d_x, d_d, d_w


class RowNorm(torch.autograd.Function):
    """(s, y) = add-RMSNorm(x, delta, w) when delta is given, else y = RMSNorm(x, w)."""

    @staticmethod
    def forward(ctx, x, delta, weight, eps, out_dtype):
        lay = _Layout(x, delta, weight, out_dtype)
        s, y, rstd = _forward_launch(lay, x, delta, weight, eps)
        ctx.lay = lay
        ctx.save_for_backward(s, weight, rstd)
        ctx.set_materialize_grads(False)
        if delta is None:
            return y
        return s, y

    @staticmethod
    @once_differentiable
    def backward(ctx, *grads):
        lay = ctx.lay
        g_s, g_y = (None, grads[0]) if lay.delta_dtype is None else grads
        if g_s is None and g_y is None:
            return None, None, None, None, None
        s, weight, rstd = ctx.saved_tensors
        want = ctx.needs_input_grad[:3]
        d_x, d_d, d_w = _backward_launch(lay, s, weight, rstd, g_s, g_y, want)
        return d_x, d_d, d_w, None, None


def row_norm(x, delta, weight, eps, out_dtype):
    """Run the node on x's device (arguments already checked by the caller)."""
    with torch.cuda.device(x.device):
        return RowNorm.apply(x, delta, weight, eps, out_dtype)
