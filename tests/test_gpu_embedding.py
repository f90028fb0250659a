"""GPU tests of the lossless fp16 table storage (ss_f32_to_f16_exact, embedding.py).

Parity bar (solution/embedding.py:51-64): the fp16 candidate is bit-identical to
torch's round-to-nearest-even ``.half()`` of the table, and the table is accepted
exactly when ``torch.equal(candidate.float(), table)`` -- checked here against
torch on the same inputs, with single inexact elements planted at the first,
middle and last element, in the scalar tail and on an unaligned view (which
takes the scalar path), plus NaN (never exact), +-inf and -0.0 (exact).  The
installed model (solution/embedding.py:116-141): same Parameter object, fp16
storage, fp32 embedding output equal to before, head logits under fp16 autocast
and outside it equal to the fp32 model's.
"""

import sys
from types import ModuleType, SimpleNamespace

import pytest
import torch

from soupsuck_amd import embedding

pytestmark = pytest.mark.gpu


def _lossless(n, device, seed=0):
    gen = torch.Generator(device="cpu").manual_seed(seed)
    return (torch.randn(n, generator=gen) * 0.02).half().float().to(device)


@pytest.mark.parametrize("n", [1, 7, 8, 1000, 1 << 20, 3 * 65536 + 5])
def test_exact_table_converts_bit_identically(device, n):
    table = _lossless(n, device)
    out = embedding.exact_half(table)
    assert out is not None and out.dtype == torch.float16
    assert torch.equal(out.view(torch.int16), table.half().view(torch.int16))


@pytest.mark.parametrize("where", ["first", "middle", "last", "tail"])
def test_one_inexact_element_is_found(device, where):
    n = 8 * 4099 + 3                        # a vector body and a 3-element scalar tail
    table = _lossless(n, device, seed=1)
    i = {"first": 0, "middle": n // 2, "last": n - 4, "tail": n - 1}[where]
    table[i] = 1.0 + 2.0 ** -20              # needs 21 mantissa bits
    assert embedding.exact_half(table) is None
    assert not torch.equal(table.half().float(), table)   # torch agrees


def test_special_values(device):
    base = _lossless(64, device, seed=2)
    for value, ok in ((float("inf"), True), (float("-inf"), True), (-0.0, True),
                      (float("nan"), False), (70000.0, False), (1e-8, False)):
        table = base.clone()
        table[17] = value
        got = embedding.exact_half(table)
        assert (got is not None) == ok, value
        assert torch.equal(table.half().float(), table) == ok, value
        if ok:
            assert torch.equal(got.view(torch.int16), table.half().view(torch.int16))


def test_unaligned_view_takes_the_scalar_path(device):
    table = _lossless(4097, device, seed=3)
    view = table[1:]                         # 4-byte aligned, not 16
    out = embedding.exact_half(view)
    assert out is not None
    assert torch.equal(out.view(torch.int16), view.half().view(torch.int16))
    view[100] = 1.0 + 2.0 ** -20
    assert embedding.exact_half(view) is None


def _peft_stack(device, monkeypatch):
    from transformers import Qwen2Config
    from transformers.models.qwen2 import modeling_qwen2 as qwen

    cfg = Qwen2Config(hidden_size=128, intermediate_size=256, num_attention_heads=2,
                      num_key_value_heads=1, num_hidden_layers=1, vocab_size=1000,
                      tie_word_embeddings=True)
    torch.manual_seed(4)
    model = qwen.Qwen2ForCausalLM(cfg).to(device)
    with torch.no_grad():    # a table that fp16 holds exactly (e.g. loaded from fp16)
        model.model.embed_tokens.weight.copy_(model.model.embed_tokens.weight.half().float())
    model.requires_grad_(False)
    peft = ModuleType("peft")
    peft.get_peft_model_state_dict = lambda m, adapter_name, save_embedding_layers: {
        "base_model.model.model.layers.0.self_attn.q_proj.lora_A.weight": None}
    monkeypatch.setitem(sys.modules, "peft", peft)

    class Wrapper(torch.nn.Module):
        def __init__(self, base):
            super().__init__()
            self.base = base
            self.peft_config = {"default": SimpleNamespace(
                peft_type="LORA", target_modules={"q_proj", "v_proj"}, modules_to_save=None,
                trainable_token_indices=None, bias="none")}

        def get_base_model(self):
            return self.base

    return model, Wrapper(model)


def test_tied_table_is_stored_in_fp16(device, monkeypatch):
    model, wrapped = _peft_stack(device, monkeypatch)
    weight = model.model.embed_tokens.weight
    reference = weight.detach().clone()
    ids = torch.randint(0, 1000, (2, 9), device=device)
    hidden = torch.randn(2, 9, 128, device=device)
    emb_before = model.model.embed_tokens(ids)
    logits_fp32 = torch.nn.functional.linear(hidden, reference)
    with torch.autocast("cuda", dtype=torch.float16):
        logits_amp = model.lm_head(hidden)
    assert embedding.compress_tied_embedding(wrapped) is True
    assert model.model.embed_tokens.weight is weight and model.lm_head.weight is weight
    assert weight.dtype == torch.float16 and not weight.requires_grad
    assert torch.equal(weight.float(), reference)
    out = model.model.embed_tokens(ids)
    assert out.dtype == torch.float32 and torch.equal(out, emb_before)
    assert torch.equal(model.lm_head(hidden), logits_fp32)
    with torch.autocast("cuda", dtype=torch.float16):
        assert torch.equal(model.lm_head(hidden), logits_amp)
    assert embedding.compress_tied_embedding(wrapped) is True        # already in place


def test_inexact_table_is_left_alone(device, monkeypatch):
    model, wrapped = _peft_stack(device, monkeypatch)
    weight = model.model.embed_tokens.weight
    with torch.no_grad():
        weight[5, 3] = 1.0 + 2.0 ** -20
    before = weight.detach().clone()
    assert embedding.compress_tied_embedding(wrapped) is False
    assert weight.dtype == torch.float32 and torch.equal(weight, before)
    assert "forward" not in model.model.embed_tokens.__dict__
