"""Route for PEFT's ``tuners.lora.bnb.Linear4bit.forward`` into the fused QLoRA projection.

The reference keeps PEFT's forward structure (base layer, then LoRA A/B with
PEFT's dropout, then a rounded scale/add epilogue; solution/lora.py:135-163).
On MI355X the whole projection is one node (soupsuck_amd.lora.qlora_projection):
the NF4 base GEMM with the LoRA product added in its epilogue, and the
backward dX = g.W + dZ.A in one accumulator.  That node computes the LoRA
branch in fp16, so a layer is routed only where PEFT itself computes it in
fp16: an fp16 activation with CUDA fp16 autocast on or fp16 A/B weights.

Eligibility (everything else runs PEFT's original forward):
  * routing enabled; x a contiguous CUDA fp16 tensor; no extra positional
    arguments; no keyword arguments other than ``adapter_names=None`` and
    ``alora_offsets=None`` (mixed-adapter batches and aLoRA stay on PEFT);
  * adapters enabled and unmerged, exactly one active adapter, no DoRA, no
    LoRA variant, no LoRA bias (solution/lora.py:66-101 excludes the same);
  * lora_A / lora_B plain bias-free ``torch.nn.Linear`` on x's device, the
    dropout ``torch.nn.Identity`` or a non-inplace ``torch.nn.Dropout``, a
    finite real scaling;
  * the base layer a frozen nested-NF4 ``Linear4bit`` (fp16 or unset compute
    dtype) with a frozen bias or none, and no hooks or per-instance forward
    on any of the modules involved.
Dropout with p > 0 in training runs fused too (soupsuck_amd.lora: a Philox
mask recomputed by the kernels from a per-call seed; the keep probability and
the fp32 scaling are the reference's, solution/lora.py:1-40, the bits are not
those of torch's CUDA RNG).
"""

import math
import numbers

import torch

from .utils import enabled
from .utils import hookless as _hookless

_ALLOWED_KWARGS = ("adapter_names", "alora_offsets")


def _plain_linear(m, device):
    return (type(m) is torch.nn.Linear and m.bias is None and m.weight.is_cuda
            and m.weight.device == device and m.weight.dtype in (torch.float16, torch.float32))


def _nf4_base(base):
    """(packed, state, bias16 or None) of a frozen nested-NF4 Linear4bit base, else None."""
    from .kernels.nf4 import _validate_state

    weight = getattr(base, "weight", None)
    state = getattr(weight, "quant_state", None)
    if state is None or weight.requires_grad:
        return None
    if getattr(base, "compute_dtype", None) not in (None, torch.float16):
        return None
    packed = weight.data if isinstance(weight, torch.nn.Parameter) else weight
    try:
        n, _ = _validate_state(packed, state, torch.float16)
    except ValueError:
        return None
    bias = getattr(base, "bias", None)
    if bias is not None:
        if bias.requires_grad or bias.shape != (n,) or bias.dtype not in (torch.float16,
                                                                          torch.float32):
            return None
        bias = bias.detach().to(torch.float16).contiguous()
    return packed, state, bias


def routed_call(layer, x, args, kwargs, as_fp16=False):
    """The arguments of qlora_projection for an eligible call, else None.

    as_fp16: judge the call as if x were the contiguous fp16 tensor it is about
    to become (an owner deciding to produce x in fp16 asks this first)."""
    if not enabled() or args or any(k not in _ALLOWED_KWARGS or kwargs[k] is not None
                                    for k in kwargs):
        return None
    if not (isinstance(x, torch.Tensor) and x.is_cuda and x.ndim >= 1
            and (as_fp16 or (x.dtype == torch.float16 and x.is_contiguous()))):
        return None
    if layer.disable_adapters or layer.merged or len(layer.active_adapters) != 1:
        return None
    name = layer.active_adapters[0]
    if name not in layer.lora_A or name not in layer.lora_B:
        return None
    if getattr(layer, "use_dora", {}).get(name, False) or name in getattr(layer, "lora_variant",
                                                                          {}):
        return None
    if getattr(layer, "lora_bias", {}).get(name, False):
        return None
    a, b, drop = layer.lora_A[name], layer.lora_B[name], layer.lora_dropout[name]
    scaling = layer.scaling[name]
    if not (_plain_linear(a, x.device) and _plain_linear(b, x.device)):
        return None
    if type(drop) not in (torch.nn.Identity, torch.nn.Dropout) or getattr(drop, "inplace", False):
        return None
    if isinstance(scaling, bool) or not isinstance(scaling, numbers.Real) \
            or not math.isfinite(scaling):
        return None
    fp16_lora = (torch.is_autocast_enabled("cuda")
                 and torch.get_autocast_dtype("cuda") == torch.float16) or \
        (a.weight.dtype == b.weight.dtype == torch.float16)
    if not fp16_lora:
        return None
    base = layer.base_layer
    if not _hookless(base, a, b, drop):
        return None
    nf4 = _nf4_base(base)
    if nf4 is None or packed_k(nf4) != x.shape[-1] or nf4[0].device != x.device:
        return None
    packed, state, bias = nf4
    p = float(drop.p) if isinstance(drop, torch.nn.Dropout) else 0.0
    return dict(x=x, lora_a=a.weight, lora_b=b.weight, packed=packed, state=state, bias=bias,
                scaling=float(scaling), dropout_p=p, training=bool(drop.training))


def fp16_ingress_ready(layer, x):
    """True when the routed PEFT forward would take ``layer``'s input x as fp16
    (reference solution/lora.py:104-127): an exact, hook-free PEFT Linear4bit whose
    class carries this route, over an fp16-compute NF4 base, eligible for an fp16 x."""
    import sys

    from .norm_scope import _nf4_linear
    from .patch import PEFT_ROUTE

    cls = getattr(sys.modules.get(PEFT_ROUTE.module), PEFT_ROUTE.owner, None)
    if (not isinstance(cls, type) or type(layer) is not cls
            or not hasattr(cls.forward, PEFT_ROUTE.marker) or not _hookless(layer)):
        return False
    base = getattr(layer, "base_layer", None)
    if (base is None or not _nf4_linear(base) or base.compute_dtype != torch.float16
            or not base.compute_type_is_set or not _hookless(base)):
        return False
    return routed_call(layer, x, (), {}, as_fp16=True) is not None


def packed_k(nf4):
    return nf4[1].shape[1]


def build_linear4bit_forward(original, module):
    cls = getattr(module, "Linear4bit", None)
    if not isinstance(cls, type):
        return None

    def forward(self, x, *args, **kwargs):
        call = routed_call(self, x, args, kwargs) if type(self) is cls else None
        if call is None:
            return original(self, x, *args, **kwargs)
        check = getattr(self, "_check_forward_args", None)
        if check is not None:
            check(x, *args, **kwargs)
        from .lora import qlora_projection

        return qlora_projection(**call)

    return forward
