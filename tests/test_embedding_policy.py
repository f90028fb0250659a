"""CPU tests of the lossless tied-embedding policy (soupsuck_amd.embedding): the
acceptance rules of solution/embedding.py:66-141 that decide before any GPU work,
and the Soup setup route (solution/embedding.py:146-169).  PEFT and Soup are not
installed, so their pieces are stand-ins (ModuleType objects / plain classes).
"""

import sys
from types import ModuleType, SimpleNamespace

import pytest
import torch

from soupsuck_amd import embedding, patch


def _tiny_lm(tie=True):
    from transformers import Qwen2Config
    from transformers.models.qwen2 import modeling_qwen2 as qwen

    cfg = Qwen2Config(hidden_size=64, intermediate_size=128, num_attention_heads=2,
                      num_key_value_heads=1, num_hidden_layers=1, vocab_size=100,
                      tie_word_embeddings=tie)
    torch.manual_seed(0)
    model = qwen.Qwen2ForCausalLM(cfg)
    model.model.embed_tokens.weight.requires_grad_(False)
    return model


class _Peft(torch.nn.Module):
    """What compress_tied_embedding reads of a PeftModel: get_base_model and peft_config."""

    def __init__(self, base, configs):
        super().__init__()
        self.base = base
        self.peft_config = configs

    def get_base_model(self):
        return self.base


def _lora(targets=("q_proj", "v_proj"), **kw):
    targets = targets if isinstance(targets, str) else list(targets)
    cfg = dict(peft_type="LORA", target_modules=targets, modules_to_save=None,
               trainable_token_indices=None, bias="none")
    cfg.update(kw)
    return SimpleNamespace(**cfg)


def test_unwrap_finds_the_model_under_wrappers():
    model = _tiny_lm()
    cls = type(model)
    ddp = SimpleNamespace(module=_Peft(model, {}))
    assert embedding.unwrap(ddp, cls) is model
    assert embedding.unwrap(SimpleNamespace(module=None), cls) is None
    loop = SimpleNamespace()
    loop.module = loop
    assert embedding.unwrap(loop, cls) is None


@pytest.mark.parametrize("configs, reason", [
    ({}, "no PEFT adapter"),
    ({"a": _lora(targets=("q_proj", "o_proj"))}, "q_proj / v_proj-only"),
    ({"a": _lora(modules_to_save=["lm_head"])}, "q_proj / v_proj-only"),
    ({"a": _lora(bias="all")}, "q_proj / v_proj-only"),
    ({"a": _lora(peft_type="IA3")}, "q_proj / v_proj-only"),
    ({"a": _lora(targets="q_proj")}, "q_proj / v_proj-only"),
])
def test_adapter_rules_decline(configs, reason):
    assert reason in embedding._adapter_reason(_Peft(_tiny_lm(), configs))


def test_adapter_rules_use_peft_auto_save_policy(monkeypatch):
    peft = ModuleType("peft")
    saved = {"a": {"base_model.model.layers.0.self_attn.q_proj.lora_A.weight": 0}}
    peft.get_peft_model_state_dict = lambda model, adapter_name, save_embedding_layers: (
        saved[adapter_name] if save_embedding_layers == "auto" else None)
    monkeypatch.setitem(sys.modules, "peft", peft)
    wrapped = _Peft(_tiny_lm(), {"a": _lora()})
    assert embedding._adapter_reason(wrapped) is None
    saved["a"]["base_model.model.embed_tokens.weight"] = 0   # resized vocabulary: table saved
    assert "auto save policy" in embedding._adapter_reason(wrapped)


def test_cpu_and_untied_tables_are_declined(monkeypatch):
    messages = []
    monkeypatch.setattr(embedding, "_decline", lambda reason: messages.append(reason) or False)
    assert embedding.compress_tied_embedding(_tiny_lm()) is False
    assert "CUDA" in messages[-1]
    assert embedding.compress_tied_embedding(_tiny_lm(tie=False)) is False
    assert "tied to one shared Parameter" in messages[-1]
    assert embedding.compress_tied_embedding(torch.nn.Linear(2, 2)) is False
    assert "exact Qwen2ForCausalLM" in messages[-1]
    monkeypatch.setenv("SOUP_FUSED_DISABLE", "1")
    n = len(messages)
    assert embedding.compress_tied_embedding(_tiny_lm()) is False and len(messages) == n


def test_soup_setup_route_runs_the_original_then_the_policy(monkeypatch):
    module = ModuleType("soup_cli.trainer.sft")

    class SFTTrainerWrapper:
        def _setup_transformers(self, *args, **kwargs):
            self.model = _tiny_lm()
            return ("set up", args, kwargs)

    SFTTrainerWrapper.__module__ = module.__name__
    module.SFTTrainerWrapper = SFTTrainerWrapper
    seen = []
    monkeypatch.setattr(embedding, "compress_tied_embedding", lambda m: seen.append(m))
    assert patch.install_route(patch.SOUP_SETUP_ROUTE, module)
    assert patch.install_route(patch.SOUP_SETUP_ROUTE, module)           # idempotent
    wrapper = SFTTrainerWrapper()
    assert wrapper._setup_transformers(1, k=2) == ("set up", (1,), {"k": 2})
    assert seen == [wrapper.model]
    original = getattr(SFTTrainerWrapper._setup_transformers, patch.MARKER)
    assert original.__name__ == "_setup_transformers"
