"""``add_rms_norm``: residual add + Qwen2 RMSNorm (A13-A15), the reference's entry point.

Same name, arguments and results as solution/kernels/add_rmsnorm.py:139-161:
returns (s, y) with s = residual + delta in promote(residual, delta) and y the
normed s, in promote(s, weight) or fp16 when out_dtype=torch.float16.  The
row computation and its autograd node are shared with the plain norm
(kernels/rownorm.py); this module holds the argument contract.
"""

import torch

from ..contract import Rule, enforce, finite_real, float_dtypes, is_tensor, on_one_cuda_device
from .rownorm import row_norm

ADD_RMS_NORM_RULES = (
    Rule("add_rms_norm: residual and delta must be tensors of one shape [..., H] with H > 0",
         lambda a: is_tensor(a.residual, a.delta, a.weight) and a.residual.ndim >= 1
         and a.residual.shape == a.delta.shape and a.residual.shape[-1] > 0),
    Rule("add_rms_norm: weight must be one-dimensional of length H",
         lambda a: a.weight.ndim == 1 and a.weight.shape[0] == a.residual.shape[-1]),
    Rule("add_rms_norm: residual, delta and weight must be CUDA tensors on one device",
         lambda a: on_one_cuda_device(a.residual, a.delta, a.weight)),
    Rule("add_rms_norm: residual and delta must be contiguous",
         lambda a: a.residual.is_contiguous() and a.delta.is_contiguous()),
    Rule("add_rms_norm: residual, delta and weight must be fp16 or fp32",
         lambda a: float_dtypes(a.residual, a.delta, a.weight)),
    Rule("add_rms_norm: out_dtype must be None or torch.float16",
         lambda a: a.out_dtype is None or a.out_dtype == torch.float16),
    Rule("add_rms_norm: eps must be a finite real number >= 0",
         lambda a: finite_real(a.eps, minimum=0)),
)


def add_rms_norm(residual, delta, weight, eps, out_dtype=None):
    """Return (residual + delta, its Qwen2 RMSNorm); ValueError before launch if unsupported."""
    enforce(ADD_RMS_NORM_RULES, residual=residual, delta=delta, weight=weight, eps=eps,
            out_dtype=out_dtype)
    return row_norm(residual, delta, weight, eps, out_dtype)
