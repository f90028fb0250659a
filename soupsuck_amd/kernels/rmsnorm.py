"""``rms_norm``: the standalone Qwen2 RMSNorm (input / final norm), the reference's entry point.

Same name, arguments and result as solution/kernels/rmsnorm.py:159-188:
y = weight * cast(x * rstd, x.dtype) in promote(x, weight), or fp16 when
out_dtype=torch.float16.  x is contiguous with any leading shape, or a 2-D
row-strided view (unit last stride).  The computation is the add-RMSNorm
node without a delta (kernels/rownorm.py); this module holds the contract.
"""

import torch

from ..contract import Rule, enforce, finite_real, float_dtypes, is_tensor, on_one_cuda_device
from .rownorm import row_norm

RMS_NORM_RULES = (
    Rule("rms_norm: expected x [..., H] with H > 0 and weight [H]",
         lambda a: is_tensor(a.x, a.weight) and a.x.ndim >= 1 and a.x.shape[-1] > 0
         and a.weight.ndim == 1 and a.weight.shape[0] == a.x.shape[-1]),
    Rule("rms_norm: x and weight must be CUDA tensors on one device",
         lambda a: on_one_cuda_device(a.x, a.weight)),
    Rule("rms_norm: the last dimension of x must be contiguous",
         lambda a: a.x.stride(-1) == 1),
    Rule("rms_norm: a row-strided (non-contiguous) x must be 2-D",
         lambda a: a.x.is_contiguous() or a.x.ndim == 2),
    Rule("rms_norm: x and weight must be fp16 or fp32",
         lambda a: float_dtypes(a.x, a.weight)),
    Rule("rms_norm: eps must be a finite real number >= 0",
         lambda a: finite_real(a.eps, minimum=0)),
    Rule("rms_norm: out_dtype must be None or torch.float16",
         lambda a: a.out_dtype is None or a.out_dtype == torch.float16),
)


def rms_norm(x, weight, eps, out_dtype=None):
    """Normalize the last dimension with Qwen2's casts; ValueError before launch if unsupported."""
    enforce(RMS_NORM_RULES, x=x, weight=weight, eps=eps, out_dtype=out_dtype)
    return row_norm(x, None, weight, eps, out_dtype)
