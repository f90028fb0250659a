"""Lossless fp16 storage of a frozen, tied Qwen2 embedding / lm_head table.

Behaviour of the reference (solution/embedding.py:51-141): after PEFT setup,
the tied fp32 table of an exact ``Qwen2ForCausalLM`` is replaced -- in place,
on the same ``Parameter`` -- by fp16 storage, but only when every element
survives the fp32 -> fp16 -> fp32 round trip exactly (the representation
changes, no value does).  The embedding's output is upcast back to fp32; the
head under CUDA autocast multiplies the same values in fp16 as before, and
outside autocast runs on a temporary fp32 copy.  At V = 151936, H = 1536 this
frees 445 MiB of training storage.

Here the conversion and its check are one HIP pass (ss_f32_to_f16_exact: read
fp32, write the fp16 candidate, raise a flag on any inexact element) and one
flag read, instead of the reference's 32 MiB chunks compared by torch; the
candidate is the eventual storage, so nothing fp32-sized is allocated.

Acceptance (anything else declines, reporting the reason once per process):
routing enabled; an exact Qwen2ForCausalLM under any PEFT / DDP wrapping; a
plain ``Embedding`` and a plain bias-free ``Linear`` head sharing one
Parameter, frozen, fp32, CUDA, contiguous and 2-D, no max_norm and no
per-instance forward; a PEFT LoRA configuration targeting only q_proj /
v_proj, with no modules_to_save, trainable tokens or bias; PEFT's own
``save_embedding_layers="auto"`` policy saving LoRA tensors only (a resized
vocabulary would make PEFT save the table); and an exact round trip.

``route_soup_setup`` installs the call after Soup's
``SFTTrainerWrapper._setup_transformers`` (solution/embedding.py:146-169).
"""

import importlib
import sys
from types import MethodType

import torch

from . import _lib
from .utils import enabled

ACTIVE = "_soupsuck_lossless_embedding"
_REPORTED = set()


def _decline(reason):
    if reason not in _REPORTED:
        _REPORTED.add(reason)
        print(f"[soupsuck_amd] lossless embedding skipped: {reason}", file=sys.stderr, flush=True)
    return False


def unwrap(model, cls):
    """The ``cls`` instance under PEFT (get_base_model) / DDP (module) wrappers, or None."""
    seen = set()
    while model is not None and id(model) not in seen:
        seen.add(id(model))
        if type(model) is cls:
            return model
        inner = model.get_base_model() if hasattr(model, "get_base_model") else \
            getattr(model, "module", None)
        if inner is model:
            return None
        model = inner
    return None


def exact_half(weight):
    """fp16 copy of a CUDA fp32 tensor when every element round-trips exactly, else None."""
    if not (weight.is_cuda and weight.dtype == torch.float32 and weight.is_contiguous()):
        raise ValueError("exact_half: a contiguous CUDA fp32 tensor is required")
    out = torch.empty_like(weight, dtype=torch.float16)
    flag = torch.zeros(1, dtype=torch.int32, device=weight.device)
    with torch.cuda.device(weight.device):
        _lib.call("ss_f32_to_f16_exact", weight.data_ptr(), out.data_ptr(), weight.numel(),
                  flag.data_ptr(), _lib.stream(weight.device))
    return None if int(flag.item()) else out


def _adapter_reason(model):
    configs = getattr(model, "peft_config", None)
    if not isinstance(configs, dict) or not configs:
        return "no PEFT adapter configuration on the model"
    for config in configs.values():
        targets = getattr(config, "target_modules", None)
        kind = getattr(config, "peft_type", None)
        if (getattr(kind, "value", kind) != "LORA"
                or not isinstance(targets, (tuple, list, set)) or not targets
                or not set(targets) <= {"q_proj", "v_proj"}
                or getattr(config, "modules_to_save", None)
                or getattr(config, "trainable_token_indices", None)
                or getattr(config, "bias", "none") != "none"):
            return "needs q_proj / v_proj-only LoRA without saved modules, tokens or bias"
    try:
        from peft import get_peft_model_state_dict
    except ImportError:
        return "peft is not importable, so its embedding save policy cannot be checked"
    for name in configs:
        saved = get_peft_model_state_dict(model, adapter_name=name, save_embedding_layers="auto")
        if not saved or any("lora_" not in key for key in saved):
            return "PEFT's auto save policy would store non-LoRA tensors (e.g. a resized vocabulary)"
    return None


def compress_tied_embedding(model):
    """Install lossless fp16 storage of the tied table; True when it is (or already was) in place."""
    if not enabled() or not isinstance(model, torch.nn.Module):
        return False
    try:
        qwen = importlib.import_module("transformers.models.qwen2.modeling_qwen2")
    except ImportError:
        return False
    cls = getattr(qwen, "Qwen2ForCausalLM", None)
    if not isinstance(cls, type) or cls.__module__ != qwen.__name__:
        return False
    raw = unwrap(model, cls)
    if raw is None:
        return _decline("not an exact Qwen2ForCausalLM")
    embedding, head = raw.get_input_embeddings(), raw.get_output_embeddings()
    if type(embedding) is not torch.nn.Embedding or type(head) is not torch.nn.Linear:
        return _decline("the input / output embeddings are wrapped or not plain modules")
    weight = embedding.weight
    if head.weight is not weight:
        return _decline("lm_head and embed_tokens do not share one Parameter")
    if getattr(raw, ACTIVE, False):
        return weight.dtype == torch.float16 and not weight.requires_grad
    if (weight.requires_grad or weight.dtype != torch.float32 or not weight.is_cuda
            or not weight.is_contiguous() or weight.ndim != 2):
        return _decline("the tied table must be frozen, fp32, CUDA, contiguous and 2-D")
    if (embedding.max_norm is not None or head.bias is not None
            or "forward" in embedding.__dict__ or "forward" in head.__dict__):
        return _decline("max_norm embedding, biased head or per-instance forward")
    reason = _adapter_reason(model)
    if reason is not None:
        return _decline(reason)
    candidate = exact_half(weight.detach())
    if candidate is None:
        return _decline("an element of the table has no exact fp16 representation")
    embed_forward, head_forward = type(embedding).forward, type(head).forward

    def embedding_forward(self, ids):
        return embed_forward(self, ids).to(torch.float32)

    def linear_forward(self, x):
        if torch.is_autocast_enabled("cuda"):
            return head_forward(self, x)
        return torch.nn.functional.linear(x, self.weight.float(), self.bias)

    with torch.no_grad():
        weight.data = candidate
    embedding.forward = MethodType(embedding_forward, embedding)
    head.forward = MethodType(linear_forward, head)
    setattr(raw, ACTIVE, True)
    return True


def build_soup_setup(original, module):
    """Route body for soup_cli.trainer.sft.SFTTrainerWrapper._setup_transformers."""
    if not isinstance(getattr(module, "SFTTrainerWrapper", None), type):
        return None

    def _setup_transformers(self, *args, **kwargs):
        result = original(self, *args, **kwargs)
        if isinstance(getattr(self, "model", None), torch.nn.Module):
            compress_tied_embedding(self.model)
        return result

    return _setup_transformers
