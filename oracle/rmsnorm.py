"""Fused residual add + Qwen2 RMSNorm oracle (A13-A14) -- test infrastructure only.

Reference semantics (solution/kernels/add_rmsnorm.py:1-11,37-81;
solution/kernels/rmsnorm.py:1-14,73-102):
  forward   s = cast(r + d, promote(r, d))                      (exact)
            rstd = rsqrt(mean(fp32(s)^2) + eps)
            q = cast(fp32(s) * rstd, s.dtype)
            y = w * q in promote(s.dtype, w.dtype), optionally cast to fp16
  backward  a = fp32(s) * rstd;  u = cast(gy * w, s.dtype)
            ds = cast(rstd * (u - a * mean(u * a)), s.dtype) + gs, then cast
            to each input's dtype (dr, dd)
  dgamma    sum over rows of gy * q (each product rounded to fp16 when the
            exact output dtype is fp16), fp32 reduction.
Statistics are computed in float64 here (the ideal the fp32 reductions
approximate); every dtype cast follows the reference order.  Tolerances are
the reference's: fp32 1e-5, fp16 2e-3 (solution/tests/test_add_rmsnorm.py:10-11).

Pins: the eager composition of solution/tests/test_add_rmsnorm.py:19-28 is a
different formula for the same quantity (torch autograd of the forward) --
the CPU tests compare this module's backward against torch.autograd on CPU
in float64; plus the invariants rms(y/w) == 1 and ds orthogonal to a when
gs = 0 and the fp16 roundings are removed.
"""

import numpy as np

F32 = np.float32


def _promote(a, b):
    return np.promote_types(a, b)


def add_rmsnorm_forward(r, d, w, eps, out_half=False):
    r, d, w = np.asarray(r), np.asarray(d), np.asarray(w)
    sdt = _promote(r.dtype, d.dtype)
    acc = np.float64 if sdt == np.float64 else F32   # fp16/fp32 inputs add in fp32
    s = (r.astype(acc) + d.astype(acc)).astype(acc).astype(sdt)
    sf = s.astype(np.float64)
    rstd = 1.0 / np.sqrt((sf * sf).mean(axis=-1, keepdims=True) + eps)
    q = (sf * rstd).astype(sdt)
    exact = _promote(sdt, w.dtype)
    y = (w.astype(np.float64) * q.astype(np.float64)).astype(exact)
    if out_half:
        y = y.astype(np.float16)
    return s, y, rstd[..., 0]


def add_rmsnorm_backward(gs, gy, s, w, rstd, r_dtype, d_dtype, y_exact_dtype):
    """Return (dr, dd, dgamma) following add_rmsnorm.py:54-81 and rmsnorm.py:73-102."""
    s = np.asarray(s)
    sdt = s.dtype
    sf = s.astype(np.float64)
    rs = np.asarray(rstd, np.float64)[..., None]
    a = sf * rs
    h = s.shape[-1]
    if gy is not None:
        gyf = np.asarray(gy).astype(np.float64)
        u = (gyf * np.asarray(w, np.float64)).astype(sdt).astype(np.float64)
        proj = (u * a).sum(axis=-1, keepdims=True) / h
        ds = (rs * (u - a * proj)).astype(sdt).astype(np.float64)
    else:
        ds = np.zeros_like(sf)
    if gs is not None:
        ds = ds + np.asarray(gs).astype(np.float64)
    ds = ds.astype(sdt)
    dgamma = None
    if gy is not None:
        q = a.astype(sdt).astype(np.float64)
        prod = gyf * q
        if y_exact_dtype == np.float16:
            prod = prod.astype(np.float16).astype(np.float64)
        dgamma = prod.reshape(-1, h).sum(axis=0)
    return ds.astype(r_dtype), ds.astype(d_dtype), dgamma
