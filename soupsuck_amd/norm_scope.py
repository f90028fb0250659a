"""fp16 output of explicitly owned Qwen2 RMSNorms (reference solution/patch.py:35-125,
solution/decoder.py:62-85).

Under Qwen2's dtype promotion an RMSNorm with an fp32 weight returns fp32.
Where every consumer of the output would cast it to fp16 anyway -- projections
under CUDA fp16 autocast, or frozen NF4 Linear4bit layers computing in fp16 --
the norm kernel can write fp16(exact fp32 output) directly: the values the
consumers see are the same, the activation takes half the memory and the
consumers' cast kernels disappear.

Which norm does this is decided per call by its owner and scoped with a
ContextVar holding that one module (never "all norms of a class"):
  * a decoder layer's input norm, when q/k/v are all fp16 consumers
    (``input_norm_half_ready``; the attention runs under fp16 autocast);
  * a decoder layer's post-attention norm (the fused residual add + norm),
    when gate/up/down are fp16 consumers (``post_norm_half_ready``);
  * the model's final norm, when the causal-LM head is an fp16 consumer
    (``final_norm_half_ready``).
SOUP_FUSED_NORM_FP16=0 keeps the exact promotion everywhere (fp32 output).
"""

import os
from contextlib import contextmanager
from contextvars import ContextVar

import torch

from .utils import enabled, hookless

QWEN = "transformers.models.qwen2.modeling_qwen2"
_OWNER = ContextVar("soupsuck_half_norm_owner", default=None)


@contextmanager
def half_norm_scope(norm):
    """Within the block, ``norm`` (or nobody, for None) owns an fp16 output."""
    token = _OWNER.set(norm)
    try:
        yield
    finally:
        _OWNER.reset(token)


def _hookless(m):
    return hookless(m)


def half_norm_enabled(norm):
    return (isinstance(norm, torch.nn.Module) and enabled()
            and os.environ.get("SOUP_FUSED_NORM_FP16") != "0" and _hookless(norm))


def owns_half_output(norm):
    """True when ``norm`` is the scoped owner of an fp16 output right now."""
    return _OWNER.get() is norm and half_norm_enabled(norm)


def _fp16_autocast():
    return torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.float16


def _float_cuda(t):
    return isinstance(t, torch.Tensor) and t.is_cuda and t.dtype in (torch.float16, torch.float32)


def _nf4_linear(module):
    """A bitsandbytes-style Linear4bit (real bitsandbytes or bnb_compat)."""
    from . import bnb_compat

    cls = type(module)
    return (cls is bnb_compat.Linear4bit
            or (cls.__name__ == "Linear4bit" and cls.__module__ == "bitsandbytes.nn.modules"))


def plain_half_consumer(module, x):
    """``module`` consumes ``x`` as fp16 without any other effect of its dtype."""
    if not isinstance(module, torch.nn.Module) or not _hookless(module):
        return False
    weight = getattr(module, "weight", None)
    if type(module) is torch.nn.Linear:
        return _fp16_autocast() and _float_cuda(weight) and weight.device == x.device
    return (_nf4_linear(module) and module.compute_dtype == torch.float16
            and module.compute_type_is_set
            and getattr(weight, "quant_state", None) is not None and weight.device == x.device
            and not any(p.requires_grad for p in module.parameters()))


def _exact(obj, name):
    cls = type(obj)
    return cls.__module__ == QWEN and cls.__name__ == name and _hookless(obj)


def _hidden_states_requested(config, kwargs):
    return bool(kwargs.get("output_hidden_states") or getattr(config, "output_hidden_states",
                                                              False))


def input_norm_half_ready(layer, x, kwargs):
    """Qwen2Attention feeds the input norm's output to q_proj, k_proj and v_proj only."""
    from .peft_route import fp16_ingress_ready

    attention = getattr(layer, "self_attn", None)
    if (not _fp16_autocast() or not half_norm_enabled(getattr(layer, "input_layernorm", None))
            or not _float_cuda(x) or not _exact(attention, "Qwen2Attention")
            or _hidden_states_requested(attention.config, kwargs)):
        return False
    return all(plain_half_consumer(p, x) or fp16_ingress_ready(p, x)
               for p in (attention.q_proj, attention.k_proj, attention.v_proj))


def post_norm_half_ready(layer, x):
    """The post-attention norm's output feeds gate_proj and up_proj only."""
    mlp = getattr(layer, "mlp", None)
    if (not half_norm_enabled(getattr(layer, "post_attention_layernorm", None))
            or not _float_cuda(x) or not _exact(mlp, "Qwen2MLP")):
        return False
    if torch.is_autocast_enabled("cuda") and not _fp16_autocast():
        return False
    projections = (mlp.gate_proj, mlp.up_proj, mlp.down_proj)
    return len({type(p) for p in projections}) == 1 and all(
        plain_half_consumer(p, x) for p in projections)


def final_norm_half_ready(model, kwargs):
    """The final norm's output feeds only the causal-LM head (a plain fp16 Linear)."""
    inner = getattr(model, "model", None)
    norm = getattr(inner, "norm", None)
    if (not _fp16_autocast() or type(getattr(model, "lm_head", None)) is not torch.nn.Linear
            or not half_norm_enabled(norm) or not _float_cuda(getattr(norm, "weight", None))):
        return False
    if not _hookless(inner) or _hidden_states_requested(model.config, kwargs):
        return False
    return plain_half_consumer(model.lm_head, norm.weight)
