"""CPU tests of the patch surface (soupsuck_amd.patch): apply() idempotency, import order,
route fallbacks, the bitsandbytes provenance scope, and the head's label shift.

Models the reference's solution/tests/test_integration.py:175-207,546-558: fake
packages stand in for bitsandbytes and PEFT (neither is installed here), written
as real files under a temporary sys.path entry so that the meta-path finder sees
them imported after apply().  No GPU: every routed call here falls back (CPU
tensors) and the tests check which function ran.
"""

import importlib
import sys
import textwrap

import pytest
import torch

import soupsuck_amd
from soupsuck_amd import patch

FAKE_BNB = {
    "bitsandbytes/__init__.py": """
        from . import functional            # submodules load before __version__ exists
        from .backends.cuda import ops
        calls = []
        def matmul_4bit(A, B, quant_state, out=None, bias=None):
            calls.append("matmul_4bit")
            return "original matmul"
        __version__ = "0.50.2"
    """,
    "bitsandbytes/functional.py": """
        def dequantize_4bit(A, quant_state=None, absmax=None, out=None, blocksize=None,
                            quant_type="fp4"):
            from .backends.cuda import ops
            return ops._dequantize_4bit_impl(A, absmax, blocksize, quant_type, None, out)
    """,
    "bitsandbytes/backends/__init__.py": "",
    "bitsandbytes/backends/cuda/__init__.py": "",
    "bitsandbytes/backends/cuda/ops.py": """
        seen = []
        def _dequantize_4bit_impl(A, absmax, blocksize, quant_type, dtype, out):
            from soupsuck_amd import bnb_routes
            seen.append(("impl", bnb_routes._NESTED_ABSMAX.get()))
            return "original impl"
        def _dequant_linear_fallback(A, B, shapeB, absmax, blocksize, quant_type, bias=None,
                                     absmax_8bit=None, absmax_code=None, absmax_offset=None):
            import sys
            mod = sys.modules[__name__]
            return mod._dequantize_4bit_impl(A, absmax, blocksize, quant_type, None, None)
    """,
}

FAKE_PEFT = {
    "peft/__init__.py": "",
    "peft/tuners/__init__.py": "",
    "peft/tuners/lora/__init__.py": "",
    "peft/tuners/lora/bnb.py": """
        import torch
        class Linear4bit(torch.nn.Module):
            def forward(self, x, *args, **kwargs):
                return ("original peft", x)
    """,
}


def _write(root, files):
    for rel, text in files.items():
        path = root / rel
        path.parent.mkdir(parents=True, exist_ok=True)
        path.write_text(textwrap.dedent(text))


@pytest.fixture
def clean_world(tmp_path, monkeypatch):
    """Fake packages on sys.path; every global change undone afterwards."""
    _write(tmp_path, {**FAKE_BNB, **FAKE_PEFT})
    monkeypatch.syspath_prepend(str(tmp_path))
    monkeypatch.setenv("SOUP_BNB_COMPAT", "0")
    fakes = ("bitsandbytes", "peft")
    saved_modules = {k: v for k, v in sys.modules.items()
                     if k.split(".")[0] in fakes}
    for k in saved_modules:
        del sys.modules[k]
    saved_meta = list(sys.meta_path)
    qwen = importlib.import_module(patch.QWEN)
    saved_qwen = {(r.owner, r.attr): getattr(patch._holder(r, qwen), r.attr)
                  for r in patch.ROUTES if r.module == patch.QWEN}
    importlib.invalidate_caches()
    yield tmp_path
    for k in [k for k in sys.modules if k.split(".")[0] in fakes]:
        del sys.modules[k]
    sys.modules.update(saved_modules)
    sys.meta_path[:] = saved_meta
    for (owner, attr), fn in saved_qwen.items():
        holder = qwen if owner is None else getattr(qwen, owner)
        setattr(holder, attr, fn)


def _installed(module, owner, attr, marker=patch.MARKER):
    holder = module if owner is None else getattr(module, owner)
    return hasattr(getattr(holder, attr), marker)


def test_apply_is_idempotent(clean_world):
    soupsuck_amd.apply()
    qwen = sys.modules[patch.QWEN]
    installed = {r.attr + str(r.owner): getattr(patch._holder(r, qwen), r.attr)
                 for r in patch.ROUTES if r.module == patch.QWEN}
    assert all(hasattr(fn, patch.MARKER) for fn in installed.values())
    soupsuck_amd.apply()
    again = {r.attr + str(r.owner): getattr(patch._holder(r, qwen), r.attr)
             for r in patch.ROUTES if r.module == patch.QWEN}
    assert again == installed
    assert sum(getattr(f, "_solution_patch_finder", False) for f in sys.meta_path) == 1
    # the marker holds the unpatched original
    for fn in installed.values():
        assert not hasattr(getattr(fn, patch.MARKER), patch.MARKER)


def test_routes_installed_when_imported_after_apply(clean_world):
    soupsuck_amd.apply()
    import bitsandbytes
    from bitsandbytes import functional
    from bitsandbytes.backends.cuda import ops
    from peft.tuners.lora import bnb as peft_bnb

    assert _installed(functional, None, "dequantize_4bit")
    assert _installed(ops, None, "_dequantize_4bit_impl")
    assert _installed(ops, None, "_dequant_linear_fallback")
    assert _installed(bitsandbytes, None, "matmul_4bit")
    assert _installed(peft_bnb, "Linear4bit", "forward", "_solution_lora_4bit_original")


def test_routes_installed_when_imported_before_apply(clean_world):
    import bitsandbytes
    from bitsandbytes import functional
    from peft.tuners.lora import bnb as peft_bnb

    assert not _installed(functional, None, "dequantize_4bit")
    soupsuck_amd.apply()
    assert _installed(functional, None, "dequantize_4bit")
    assert _installed(bitsandbytes, None, "matmul_4bit")
    assert _installed(peft_bnb, "Linear4bit", "forward", "_solution_lora_4bit_original")
    first = functional.dequantize_4bit
    soupsuck_amd.apply()
    assert functional.dequantize_4bit is first


def test_bnb_routes_need_the_pinned_version(clean_world):
    import bitsandbytes
    from bitsandbytes import functional

    bitsandbytes.__version__ = "0.49.0"
    soupsuck_amd.apply()
    assert not _installed(functional, None, "dequantize_4bit")
    assert not _installed(bitsandbytes, None, "matmul_4bit")


def test_unsupported_calls_reach_the_originals_with_provenance(clean_world):
    soupsuck_amd.apply()
    import bitsandbytes
    from bitsandbytes import functional
    from bitsandbytes.backends.cuda import ops

    cpu = torch.zeros(4, dtype=torch.uint8)
    assert functional.dequantize_4bit(cpu, quant_state=None) == "original impl"
    assert ops.seen[-1] == ("impl", False)
    ops._dequant_linear_fallback(cpu, cpu, (2, 4), None, 64, "nf4", absmax_8bit=cpu)
    assert ops.seen[-1] == ("impl", True)      # nested statistics: the flat decode may route
    ops._dequant_linear_fallback(cpu, cpu, (2, 4), None, 64, "nf4")
    assert ops.seen[-1] == ("impl", False)
    assert bitsandbytes.matmul_4bit(cpu, cpu, None) == "original matmul"


def test_disable_switch_and_foreign_calls_use_the_originals(clean_world, monkeypatch):
    soupsuck_amd.apply()
    from peft.tuners.lora import bnb as peft_bnb

    layer = peft_bnb.Linear4bit()
    x = torch.zeros(2, 3)
    assert layer(x)[0] == "original peft"                 # CPU input: not routed
    monkeypatch.setenv("SOUP_FUSED_DISABLE", "1")
    assert layer(x)[0] == "original peft"


def test_peft_route_rejects_ineligible_calls():
    from types import SimpleNamespace

    from soupsuck_amd.peft_route import routed_call

    layer = SimpleNamespace(disable_adapters=False, merged=False, active_adapters=["a"])
    x = torch.zeros(2, 8, dtype=torch.float16)
    assert routed_call(layer, x, (), {}) is None                      # not on a GPU
    assert routed_call(layer, x, (1,), {}) is None                    # extra positional
    assert routed_call(layer, x, (), {"adapter_names": ["a"]}) is None  # mixed batch


def test_decoder_route_falls_back_on_cpu(clean_world):
    qwen = sys.modules[patch.QWEN]
    from transformers import Qwen2Config

    soupsuck_amd.apply()
    cfg = Qwen2Config(hidden_size=32, intermediate_size=64, num_attention_heads=4,
                      num_key_value_heads=2, num_hidden_layers=1, vocab_size=64)
    layer = qwen.Qwen2DecoderLayer(cfg, 0)
    h = torch.randn(1, 5, 32)
    pos = torch.arange(5)[None]
    rope = qwen.Qwen2RotaryEmbedding(cfg)
    emb = rope(h, pos)
    original = getattr(qwen.Qwen2DecoderLayer.forward, patch.MARKER)
    torch.testing.assert_close(layer(h, position_embeddings=emb),
                               original(layer, h, position_embeddings=emb))


def test_shift_happens_before_packed_selection():
    from soupsuck_amd.head import select_targets, shift_targets

    labels = torch.tensor([[1, 2, 3, -100], [4, 5, 6, 7]])
    assert shift_targets(labels).tolist() == [[2, 3, -100, -100], [5, 6, 7, -100]]
    # row 0 has 3 real tokens, row 1 has 4 (S = 4): its last real token must
    # predict the (ignored) padding, not row 1's first label
    indices = torch.tensor([0, 1, 2, 4, 5, 6, 7])
    assert select_targets(labels, indices).tolist() == [2, 3, -100, 5, 6, 7, -100]


def test_register_as_bitsandbytes_only_when_absent(monkeypatch):
    from soupsuck_amd import bnb_compat

    for k in [k for k in sys.modules if k.split(".")[0] == "bitsandbytes"]:
        monkeypatch.delitem(sys.modules, k)
    assert bnb_compat.register_as_bitsandbytes()
    import bitsandbytes as bnb

    assert bnb.nn.Linear4bit is bnb_compat.Linear4bit
    assert bnb.functional.quantize_4bit is bnb_compat.quantize_4bit
    assert bnb.__version__.startswith("0.50.2+")
    assert not bnb_compat.register_as_bitsandbytes()          # already loaded
    for k in [k for k in sys.modules if k.split(".")[0] == "bitsandbytes"]:
        monkeypatch.delitem(sys.modules, k)
