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

Acceptance is data: routing enabled and an exact Qwen2ForCausalLM under any
PEFT / DDP wrapping, then the ordered TABLE_RULES on its embedding and head,
then _LORA_CONFIG on every adapter configuration (LoRA on q_proj / v_proj
only, nothing else saved or trained), then PEFT's own
``save_embedding_layers="auto"`` policy storing LoRA tensors only (a resized
vocabulary would make PEFT save the table), then an exact round trip.  The
first rule that fails is the decline reason, reported once per process.

``route_soup_setup`` installs the call after Soup's
``SFTTrainerWrapper._setup_transformers`` (solution/embedding.py:146-169).
"""

import importlib
import sys
from types import MethodType, SimpleNamespace

import torch

from . import _lib
from .contract import Rule
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


_QV = frozenset({"q_proj", "v_proj"})

# What every PEFT adapter configuration must hold: (attribute, value when absent, test).
_LORA_CONFIG = (
    ("peft_type", None, lambda v: getattr(v, "value", v) == "LORA"),
    ("target_modules", None,
     lambda v: isinstance(v, (tuple, list, set)) and len(v) > 0 and set(v) <= _QV),
    ("modules_to_save", None, lambda v: not v),
    ("trainable_token_indices", None, lambda v: not v),
    ("bias", "none", lambda v: v == "none"),
)


def _saves_only_lora(model, names):
    """True when PEFT's save_embedding_layers="auto" policy stores LoRA tensors only for
    every adapter (it adds the table when the vocabulary was resized)."""
    from peft import get_peft_model_state_dict

    for name in names:
        state = get_peft_model_state_dict(model, adapter_name=name, save_embedding_layers="auto")
        if not state or not all("lora_" in key for key in state):
            return False
    return True


def _adapter_reason(model):
    """Why the adapter setup rules the fp16 table out, or None when it allows it."""
    configs = getattr(model, "peft_config", None)
    if not isinstance(configs, dict) or not configs:
        return "no PEFT adapter configuration on the model"
    if not all(test(getattr(config, attr, absent)) for config in configs.values()
               for attr, absent, test in _LORA_CONFIG):
        return ("the LoRA adapters must be q_proj / v_proj-only, with no saved modules, "
                "trainable tokens or bias")
    try:
        lora_only = _saves_only_lora(model, list(configs))
    except ImportError:
        return "peft is not importable, so its embedding save policy cannot be checked"
    if not lora_only:
        return "PEFT's auto save policy would store non-LoRA tensors (e.g. a resized vocabulary)"
    return None


def _plain_pair(c):
    return type(c.embedding) is torch.nn.Embedding and type(c.head) is torch.nn.Linear


def _storable(c):
    w = c.embedding.weight
    return (not w.requires_grad and w.dtype == torch.float32 and w.is_cuda
            and w.is_contiguous() and w.ndim == 2)


def _default_forwards(c):
    return (c.embedding.max_norm is None and c.head.bias is None
            and "forward" not in c.embedding.__dict__ and "forward" not in c.head.__dict__)


# Checked in order on the unwrapped model; the first failure is the decline reason.
TABLE_RULES = (
    Rule("the input / output embeddings are not a plain Embedding and a plain Linear",
         _plain_pair),
    Rule("the input embedding and the output head are not tied to one shared Parameter",
         lambda c: c.head.weight is c.embedding.weight),
    Rule("the tied table must be a frozen, contiguous 2-D fp32 tensor on CUDA", _storable),
    Rule("the embedding has max_norm, the head has a bias, or either has its own forward",
         _default_forwards),
)


def _fp32_lookup(self, ids):
    """Embedding forward over the fp16 table: the rows come back in fp32, as before."""
    return torch.nn.Embedding.forward(self, ids).to(torch.float32)


def _head_product(self, hidden):
    """Head forward over the fp16 table: autocast multiplies in fp16 exactly as it did
    with the fp32 table; without autocast the product runs on an fp32 copy."""
    if torch.is_autocast_enabled("cuda"):
        return torch.nn.Linear.forward(self, hidden)
    return torch.nn.functional.linear(hidden, self.weight.to(torch.float32))


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
        return _decline("not an exact Qwen2ForCausalLM under the PEFT / DDP wrappers")
    pair = SimpleNamespace(embedding=raw.get_input_embeddings(),
                           head=raw.get_output_embeddings())
    if getattr(raw, ACTIVE, False):
        table = pair.embedding.weight
        return table.dtype == torch.float16 and not table.requires_grad
    for rule in TABLE_RULES:
        if not rule.holds(pair):
            return _decline(rule.text)
    reason = _adapter_reason(model)
    if reason is not None:
        return _decline(reason)
    table = pair.embedding.weight
    storage = exact_half(table.detach())
    if storage is None:
        return _decline("an element of the table has no exact fp16 representation")
    with torch.no_grad():
        table.data = storage          # same Parameter: ties, names and references survive
    pair.embedding.forward = MethodType(_fp32_lookup, pair.embedding)
    pair.head.forward = MethodType(_head_product, pair.head)
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
