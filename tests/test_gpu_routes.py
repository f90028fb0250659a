"""GPU tests of the routes: each routed call must reach the HIP entry points and agree
with the original (eager) code it replaces.

  * PEFT ``Linear4bit.forward`` (reference solution/lora.py:135-163): a PEFT-shaped
    layer over bnb_compat's Linear4bit reaches ss_qlora_forward / ss_qlora_backward;
    output within the EXP-002 gate of the original forward, gradients (x, A, B)
    within relative L2 1e-2;
  * ``Qwen2ForCausalLM.forward`` (solution/patch.py:167-229): loss of the fused
    head vs the eager head within 1e-3 relative, with padding labels and with a
    ``num_items_in_batch`` denominator; the final-norm weight gradient within
    relative L2 1e-2; no logits materialised;
  * ``Qwen2DecoderLayer.forward`` (solution/decoder.py:54-89): the fused residual
    add + norm vs the original layer within fp16 tolerance;
  * ``bitsandbytes.matmul_4bit`` (fake bitsandbytes 0.50.2 module): routed output
    bit-identical to nf4_matmul;
  * ``Qwen2Model`` / ``Qwen2Attention`` (solution/unpad.py:359-450): a right-padded
    fp16 batch runs packed (gather, packed causal attention, fused head on the real
    rows) and matches the original padded forward (SDPA with the mask).
PEFT and bitsandbytes are not installed, so their modules are stand-ins
(ModuleType objects holding a class / function of the same name and signature).
"""

import sys
from types import ModuleType

import pytest
import torch

from soupsuck_amd import _lib, patch
from soupsuck_amd.bnb_compat import Linear4bit, quantize_4bit
from soupsuck_amd.kernels.nf4_gemm import nf4_matmul

pytestmark = pytest.mark.gpu


class _Recorder:
    def __init__(self, names):
        self.names, self.calls = names, []

    def __enter__(self):
        for n in self.names:
            _lib.hooks[n] = (lambda name, args: self.calls.append(name), lambda name, args: None)
        return self

    def __exit__(self, *exc):
        for n in self.names:
            _lib.hooks.pop(n, None)


def _rel(a, b):
    a, b = a.double(), b.double()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def _fake_peft_module():
    module = ModuleType("peft.tuners.lora.bnb")

    class Linear4bit(torch.nn.Module):
        """The attributes and eager forward of PEFT's bnb LoRA layer (peft 0.20.0)."""

        def __init__(self, base, r, alpha):
            super().__init__()
            self.base_layer = base
            k, n = base.in_features, base.out_features
            self.lora_A = torch.nn.ModuleDict({"default": torch.nn.Linear(k, r, bias=False)})
            self.lora_B = torch.nn.ModuleDict({"default": torch.nn.Linear(r, n, bias=False)})
            self.lora_dropout = torch.nn.ModuleDict({"default": torch.nn.Identity()})
            self.scaling = {"default": alpha / r}
            self.active_adapters = ["default"]
            self.disable_adapters = self.merged = False
            self.use_dora, self.lora_variant, self.lora_bias = {}, {}, {}

        def forward(self, x, *args, **kwargs):
            result = self.base_layer(x)
            a, b = self.lora_A["default"], self.lora_B["default"]
            lora = b(a(self.lora_dropout["default"](x.to(a.weight.dtype))))
            return result + (lora * self.scaling["default"]).to(result.dtype)

    module.Linear4bit = Linear4bit
    return module


def test_peft_linear4bit_reaches_the_fused_projection(device):
    module = _fake_peft_module()
    assert patch.install_route(patch.PEFT_ROUTE, module)
    torch.manual_seed(0)
    k, n, t = 1536, 256, 300
    base = Linear4bit(k, n, bias=True, compute_dtype=torch.float16)
    with torch.no_grad():
        base.weight.data.normal_(0, 0.02)
        base.bias.normal_(0, 0.02)
    base = base.to(device)
    layer = module.Linear4bit(base, 16, 32).to(device).half()
    with torch.no_grad():
        layer.lora_B["default"].weight.normal_(0, 0.01)
    x = torch.randn(2, t // 2, k, device=device, dtype=torch.float16, requires_grad=True)
    g = torch.randn(2, t // 2, n, device=device, dtype=torch.float16)
    with _Recorder(["ss_qlora_forward", "ss_qlora_backward"]) as rec:
        out = layer(x)
        out.backward(g)
    assert rec.calls == ["ss_qlora_forward", "ss_qlora_backward"]
    routed = (x.grad.clone(), layer.lora_A["default"].weight.grad.clone(),
              layer.lora_B["default"].weight.grad.clone())
    x.grad = None
    layer.zero_grad()
    original = getattr(module.Linear4bit.forward, "_solution_lora_4bit_original")
    eager = original(layer, x)
    eager.backward(g)
    torch.testing.assert_close(out, eager, rtol=2e-3, atol=2e-3)
    eager_grads = (x.grad, layer.lora_A["default"].weight.grad,
                   layer.lora_B["default"].weight.grad)
    for name, got, ref in zip(("dX", "dA", "dB"), routed, eager_grads):
        assert _rel(got, ref) < 1e-2, name


def _tiny_causal_lm(device, dtype):
    from transformers import Qwen2Config
    from transformers.models.qwen2 import modeling_qwen2 as qwen

    cfg = Qwen2Config(hidden_size=128, intermediate_size=256, num_attention_heads=4,
                      num_key_value_heads=2, num_hidden_layers=2, vocab_size=1000,
                      tie_word_embeddings=True)
    torch.manual_seed(1)
    return qwen, qwen.Qwen2ForCausalLM(cfg).to(device=device, dtype=dtype)


@pytest.mark.parametrize("num_items", [None, 37])
def test_causal_lm_head_route_matches_eager(device, num_items):
    qwen, model = _tiny_causal_lm(device, torch.float32)
    model.model.embed_tokens.weight.requires_grad_(False)   # frozen tied head (QLoRA)
    assert patch.install_route(patch.HEAD_ROUTE, qwen)
    ids = torch.randint(0, 1000, (3, 40), device=device)
    labels = ids.clone()
    labels[0, 30:] = -100
    labels[2, 10:] = -100
    kwargs = {} if num_items is None else {"num_items_in_batch": num_items}
    with _Recorder(["ss_ce_stats", "ss_ce_derivative"]) as rec:
        out = model(input_ids=ids, labels=labels, **kwargs)
        out.loss.backward()
    assert out.logits is None and "ss_ce_stats" in rec.calls and "ss_ce_derivative" in rec.calls
    routed_grad = model.model.norm.weight.grad.clone()
    model.zero_grad()
    original = getattr(qwen.Qwen2ForCausalLM.forward, patch.MARKER)
    ref = original(model, input_ids=ids, labels=labels, **kwargs)
    ref.loss.backward()
    assert abs(out.loss.item() - ref.loss.item()) <= 1e-3 * abs(ref.loss.item())
    assert _rel(routed_grad, model.model.norm.weight.grad) < 1e-2
    step = model._soupsuck_head_step
    assert step.token_loss.shape == labels.shape
    assert int(step.labelled) == int((labels[:, 1:] != -100).sum())


def test_decoder_route_matches_original_layer(device):
    from transformers import Qwen2Config
    from transformers.models.qwen2 import modeling_qwen2 as qwen

    assert patch.install_route(patch.DECODER_ROUTE, qwen)
    cfg = Qwen2Config(hidden_size=256, intermediate_size=512, num_attention_heads=4,
                      num_key_value_heads=2, num_hidden_layers=1, vocab_size=64)
    torch.manual_seed(2)
    layer = qwen.Qwen2DecoderLayer(cfg, 0).to(device=device, dtype=torch.float16)
    h = torch.randn(2, 33, 256, device=device, dtype=torch.float16)
    emb = qwen.Qwen2RotaryEmbedding(cfg).to(device)(h, torch.arange(33, device=device)[None])
    with _Recorder(["ss_add_rmsnorm_fwd"]) as rec:
        got = layer(h, position_embeddings=emb)
    assert rec.calls == ["ss_add_rmsnorm_fwd"]
    original = getattr(qwen.Qwen2DecoderLayer.forward, patch.MARKER)
    torch.testing.assert_close(got, original(layer, h, position_embeddings=emb),
                               rtol=2e-3, atol=2e-3)


def test_bnb_matmul_route_runs_the_nf4_gemm(device, monkeypatch):
    fake = ModuleType("bitsandbytes")
    fake.__version__ = "0.50.2"

    def matmul_4bit(A, B, quant_state, out=None, bias=None):
        raise AssertionError("the original must not run for a supported call")

    fake.matmul_4bit = matmul_4bit
    monkeypatch.setitem(sys.modules, "bitsandbytes", fake)
    assert patch.install_route(patch.BNB_ROUTES[3], fake)
    w = (torch.randn(640, 1536, device=device) * 0.02).half()
    packed, state = quantize_4bit(w)
    x = torch.randn(2, 70, 1536, device=device, dtype=torch.float16)
    bias = (torch.randn(640, device=device) * 0.1).half()
    got = fake.matmul_4bit(x, packed.t(), state, bias=bias)
    assert torch.equal(got, nf4_matmul(x, packed, state, bias=bias))


def test_unpadded_model_matches_padded_eager(device, monkeypatch):
    """Qwen2ForCausalLM on a right-padded fp16 batch: the packed path (Qwen2Model and
    Qwen2Attention routes, packed causal attention kernels, fused head on the real
    rows) against the original padded forward (SOUP_FUSED_DISABLE=1, SDPA with the
    padding mask): loss within 5e-3 relative, gradients within relative L2 5e-2."""
    from transformers import Qwen2Config
    from transformers.models.qwen2 import modeling_qwen2 as qwen

    for route in (patch.MODEL_ROUTE, patch.ATTENTION_ROUTE, patch.HEAD_ROUTE):
        assert patch.install_route(route, qwen)
    cfg = Qwen2Config(hidden_size=256, intermediate_size=512, num_attention_heads=2,
                      num_key_value_heads=1, num_hidden_layers=2, vocab_size=1000,
                      use_cache=False, attn_implementation="sdpa")
    torch.manual_seed(5)
    model = qwen.Qwen2ForCausalLM(cfg).to(device=device, dtype=torch.float16).train()
    lengths = [37, 12, 50]
    b, s = len(lengths), max(lengths)
    ids = torch.randint(0, 1000, (b, s), device=device)
    mask = torch.zeros((b, s), device=device, dtype=torch.long)
    for r, n in enumerate(lengths):
        mask[r, :n] = 1
    labels = ids.masked_fill(mask == 0, -100)

    def run():
        model.zero_grad()
        out = model(input_ids=ids, attention_mask=mask, labels=labels)
        out.loss.backward()
        grads = [p.grad.detach().float().clone() for p in (
            model.model.layers[0].self_attn.q_proj.weight,
            model.model.layers[1].self_attn.v_proj.weight,
            model.model.layers[1].mlp.down_proj.weight)]
        return out.loss.detach().float(), grads

    with _Recorder(["ss_attn_varlen_fwd", "ss_attn_varlen_bwd", "ss_unpad_gather",
                    "ss_ce_stats"]) as rec:
        loss, grads = run()
    assert rec.calls.count("ss_attn_varlen_fwd") == 2 and "ss_attn_varlen_bwd" in rec.calls
    assert "ss_unpad_gather" in rec.calls and "ss_ce_stats" in rec.calls
    monkeypatch.setenv("SOUP_FUSED_DISABLE", "1")
    ref_loss, ref_grads = run()
    assert abs(loss.item() - ref_loss.item()) <= 5e-3 * abs(ref_loss.item())
    for got, ref in zip(grads, ref_grads):
        assert _rel(got, ref) < 5e-2


class _FixedMask(torch.nn.Module):
    """A LoRA dropout replaced by a given keep mask: fp(fp32(x) / (1 - p)) where kept."""

    def __init__(self, keep, p):
        super().__init__()
        self.keep, self.inv = keep, 1.0 / (1.0 - p)

    def forward(self, x):
        return torch.where(self.keep, (x.float() * self.inv).to(x.dtype), torch.zeros_like(x))


def test_unpadded_model_packs_under_lora_dropout(device, monkeypatch):
    """The task's LoRA dropout (p = 0.05 on q / v, fp32 adapters, fp16 autocast, training) keeps
    the packed path on (reference solution/unpad.py:207-273): the right-padded batch is
    gathered, attention runs on the packed rows and the q / v projections take the fused
    Philox dropout.  Against the original padded forward with the same keep masks
    (ss_dropout_mask of each call's seed, scattered to the padded layout): loss within
    5e-3 relative, gradients within relative L2 5e-2 (the bars of the dropout-free test)."""
    from transformers import Qwen2Config
    from transformers.models.qwen2 import modeling_qwen2 as qwen

    from soupsuck_amd import unpad_route

    peft = _fake_peft_module()
    for route in (patch.MODEL_ROUTE, patch.ATTENTION_ROUTE, patch.HEAD_ROUTE):
        assert patch.install_route(route, qwen)
    assert patch.install_route(patch.PEFT_ROUTE, peft)
    cfg = Qwen2Config(hidden_size=256, intermediate_size=512, num_attention_heads=2,
                      num_key_value_heads=1, num_hidden_layers=2, vocab_size=1000,
                      use_cache=False, attn_implementation="sdpa")
    torch.manual_seed(6)
    model = qwen.Qwen2ForCausalLM(cfg).to(device=device, dtype=torch.float16)
    p = 0.05
    adapters = []
    for layer in model.model.layers:
        for name in ("q_proj", "v_proj"):
            old = getattr(layer.self_attn, name)
            base = Linear4bit(old.in_features, old.out_features, bias=True,
                              compute_dtype=torch.float16)
            with torch.no_grad():
                base.weight.data.normal_(0, 0.02)
                base.bias.normal_(0, 0.02)
            wrapped = peft.Linear4bit(base.to(device), 16, 32).to(device)
            with torch.no_grad():
                wrapped.lora_B["default"].weight.normal_(0, 0.01)
            wrapped.lora_dropout["default"] = torch.nn.Dropout(p)
            setattr(layer.self_attn, name, wrapped)
            adapters.append(wrapped)
    model.train()
    lengths = [37, 12, 50]
    b, s = len(lengths), max(lengths)
    ids = torch.randint(0, 1000, (b, s), device=device)
    mask = torch.zeros((b, s), device=device, dtype=torch.long)
    for r, n in enumerate(lengths):
        mask[r, :n] = 1
    labels = ids.masked_fill(mask == 0, -100)

    def run():
        model.zero_grad()
        with torch.autocast("cuda", dtype=torch.float16):
            out = model(input_ids=ids, attention_mask=mask, labels=labels)
        out.loss.backward()
        grads = [t.grad.detach().float().clone() for t in (
            adapters[0].lora_A["default"].weight, adapters[0].lora_B["default"].weight,
            adapters[3].lora_A["default"].weight, adapters[3].lora_B["default"].weight,
            model.model.layers[1].mlp.down_proj.weight,
            model.model.layers[0].input_layernorm.weight)]
        return out.loss.detach().float(), grads

    seeds = []
    _lib.hooks["ss_qlora_forward_dropout"] = (
        lambda name, args: seeds.append((args[14], args[2], args[9])), lambda name, args: None)
    try:
        with _Recorder(["ss_unpad_gather", "ss_attn_varlen_fwd", "ss_attn_varlen_bwd",
                        "ss_qlora_backward_dropout", "ss_ce_stats"]) as rec:
            torch.manual_seed(11)
            loss, grads = run()
    finally:
        _lib.hooks.pop("ss_qlora_forward_dropout", None)
    assert unpad_route.last_refusal() is None
    assert "ss_unpad_gather" in rec.calls and rec.calls.count("ss_attn_varlen_fwd") == 2
    assert "ss_attn_varlen_bwd" in rec.calls and "ss_ce_stats" in rec.calls
    assert rec.calls.count("ss_qlora_backward_dropout") == 4
    tokens = sum(lengths)
    assert len(seeds) == 4 and all(t == tokens for _, t, _ in seeds)
    # the same masks on the padded layout, in call order (layer 0 q, v; layer 1 q, v)
    batch_index = torch.cat([torch.arange(r * s, r * s + n, device=device)
                             for r, n in enumerate(lengths)])
    for layer_drop, (seed, t, k) in zip(adapters, seeds):
        keep = torch.empty(t * k, dtype=torch.uint8, device=device)
        _lib.call("ss_dropout_mask", seed, p, t, k, keep.data_ptr(), _lib.stream(device))
        padded = torch.zeros((b * s, k), dtype=torch.bool, device=device)
        padded.index_copy_(0, batch_index, keep.reshape(t, k).bool())
        layer_drop.lora_dropout["default"] = _FixedMask(padded.reshape(b, s, k), p)
    monkeypatch.setenv("SOUP_FUSED_DISABLE", "1")
    ref_loss, ref_grads = run()
    assert abs(loss.item() - ref_loss.item()) <= 5e-3 * abs(ref_loss.item())
    for i, (got, ref) in enumerate(zip(grads, ref_grads)):
        assert _rel(got, ref) < 5e-2, i


def test_packed_lora_dropout_fallback_keeps_the_padded_masks(device):
    """A LoRA dropout packing accepted, reached through PEFT's own forward (its routed call
    declined), draws torch's masks on the padded layout: the same generator state gives
    the padded run's mask at every real token, and zeros nowhere else are produced."""
    from soupsuck_amd import unpad
    from soupsuck_amd.unpad_route import _PACKED, _bind_dropout

    lengths, s, k = (5, 9, 3), 9, 64
    batch = unpad.make_batch(lengths, s, device)
    drop = torch.nn.Dropout(0.3).train()
    x_padded = torch.randn((len(lengths), s, k), device=device)
    torch.manual_seed(21)
    want = drop(x_padded)
    _bind_dropout(drop)
    batch.dropout_ids = frozenset({id(drop)})
    packed = unpad.pack(x_padded, batch)
    token = _PACKED.set(batch)
    try:
        torch.manual_seed(21)
        got = drop(packed)
    finally:
        _PACKED.reset(token)
    assert torch.equal(got, unpad.pack(want, batch))
    torch.manual_seed(21)
    assert torch.equal(drop(x_padded), want)        # outside a packed batch: the module itself
