"""``lora_epilogue``: add the scaled LoRA branch to the base result with eager rounding (A11).

Interface of solution/kernels/lora_epilogue.py:80-90 and the semantics of
its kernels (:1-43): out = result + round_adapter(lora_out * scaling), the
rounded product cast to the result dtype first when ``cast_to_result``
(PEFT's ``result + lora.to(result.dtype)``), out dtype = result.dtype when
cast_to_result else promote(result, lora_out).  Gradients: the result's is
the upstream gradient in the result dtype, the adapter's is
round_adapter(round_adapter(g) * scaling).  Kernels: ss_lora_epilogue_fwd /
ss_lora_epilogue_bwd (one pass each, fp32 arithmetic).
"""

import torch
from torch.autograd.function import once_differentiable

from .. import _lib
from ..contract import FLOAT_DTYPES, Rule, enforce, finite_real, is_tensor


def _out_dtype(result, lora_out, cast_to_result):
    return result.dtype if cast_to_result else torch.promote_types(result.dtype, lora_out.dtype)


def _scale_add(result, lora_out, scaling, cast_to_result):
    out = torch.empty(result.shape, device=result.device,
                      dtype=_out_dtype(result, lora_out, cast_to_result))
    count = result.numel()
    if count:
        _lib.call("ss_lora_epilogue_fwd", result.data_ptr(), _lib.dtype_code(result.dtype),
                  lora_out.data_ptr(), _lib.dtype_code(lora_out.dtype), out.data_ptr(),
                  _lib.dtype_code(out.dtype), count, float(scaling), int(cast_to_result),
                  _lib.stream(result.device))
    return out


def _scale_grad(grad, scaling, adapter_dtype):
    grad = grad.contiguous()
    d_adapter = torch.empty(grad.shape, device=grad.device, dtype=adapter_dtype)
    if grad.numel():
        _lib.call("ss_lora_epilogue_bwd", grad.data_ptr(), _lib.dtype_code(grad.dtype),
                  d_adapter.data_ptr(), _lib.dtype_code(adapter_dtype), grad.numel(),
                  float(scaling), _lib.stream(grad.device))
    return d_adapter


class LoRAEpilogue(torch.autograd.Function):
    @staticmethod
    def forward(ctx, result, lora_out, scaling, cast_to_result):
        ctx.dtypes = (result.dtype, lora_out.dtype)
        ctx.scaling = scaling
        ctx.set_materialize_grads(False)
        return _scale_add(result, lora_out, scaling, cast_to_result)

    @staticmethod
    @once_differentiable
    def backward(ctx, grad):
        want_result, want_adapter = ctx.needs_input_grad[:2]
        if grad is None:
            return None, None, None, None
        result_dtype, adapter_dtype = ctx.dtypes
        d_result = grad.to(result_dtype) if want_result else None
        d_adapter = _scale_grad(grad, ctx.scaling, adapter_dtype) if want_adapter else None
        return d_result, d_adapter, None, None


LORA_EPILOGUE_RULES = (
    Rule("lora_epilogue: result and lora_out must be CUDA tensors of one shape on one device",
         lambda a: is_tensor(a.result, a.lora_out) and a.result.is_cuda
         and a.lora_out.device == a.result.device and a.result.shape == a.lora_out.shape),
    Rule("lora_epilogue: result and lora_out must be fp16 or fp32",
         lambda a: a.result.dtype in FLOAT_DTYPES and a.lora_out.dtype in FLOAT_DTYPES),
    Rule("lora_epilogue: scaling must be a finite real number",
         lambda a: finite_real(a.scaling)),
    Rule("lora_epilogue: cast_to_result must be a bool",
         lambda a: isinstance(a.cast_to_result, bool)),
)


def lora_epilogue(result, lora_out, scaling, *, cast_to_result=False):
    """result + rounded(scaling * lora_out); ValueError before launch if unsupported."""
    enforce(LORA_EPILOGUE_RULES, result=result, lora_out=lora_out, scaling=scaling,
            cast_to_result=cast_to_result)
    with torch.cuda.device(result.device):
        return LoRAEpilogue.apply(result.contiguous(), lora_out.contiguous(), float(scaling),
                                  cast_to_result)
