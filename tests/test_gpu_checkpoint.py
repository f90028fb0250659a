"""GPU round trip of a quantized Linear4bit through a checkpoint (bnb_compat).

A Linear4bit quantized on the GPU saves its packed codes plus the QuantState
record (bitsandbytes 0.50.2 layout, see tests/test_quant_state_format.py) in its
state dict; the dict goes through safetensors (every entry is a tensor that owns
its storage) and loads into a fresh, never-quantized Linear4bit.  Bar: identical
packed codes and statistics, a bit-identical decoded weight (ss_nf4_dequant_nested)
and a bit-identical forward output.  Also Params4bit.from_prequantized, the
bitsandbytes entry point transformers uses for pre-quantized checkpoints.
"""

import pytest
import torch

from soupsuck_amd.bnb_compat import Linear4bit, Params4bit, dequantize_4bit

pytestmark = pytest.mark.gpu


def _layer(device, k=1536, n=640, bias=True, seed=0):
    torch.manual_seed(seed)
    layer = Linear4bit(k, n, bias=bias, compute_dtype=torch.float16)
    with torch.no_grad():
        layer.weight.data.normal_(0, 0.02)
        if bias:
            layer.bias.normal_(0, 0.02)
    return layer.to(device)


@pytest.mark.parametrize("bias", [True, False])
def test_state_dict_round_trip_through_safetensors(device, tmp_path, bias):
    from safetensors.torch import load_file, save_file

    src = _layer(device, bias=bias)
    sd = src.state_dict()
    assert {"weight", "weight.absmax", "weight.quant_map", "weight.nested_absmax",
            "weight.nested_quant_map", "weight.quant_state.bitsandbytes__nf4"} <= set(sd)
    path = tmp_path / "layer.safetensors"
    save_file({k: v.contiguous() for k, v in sd.items()}, str(path))
    loaded = load_file(str(path))                        # CPU tensors
    dst = Linear4bit(1536, 640, bias=bias, compute_dtype=torch.float16)
    result = dst.load_state_dict(loaded, strict=True)
    assert not result.missing_keys and not result.unexpected_keys
    dst = dst.to(device)
    a, b = src.weight.quant_state, dst.weight.quant_state
    assert torch.equal(src.weight.data, dst.weight.data)
    assert dst.weight.device == src.weight.device and dst.weight.dtype == torch.uint8
    assert torch.equal(a.absmax, b.absmax) and torch.equal(a.state2.absmax, b.state2.absmax)
    assert torch.equal(a.state2.code, b.state2.code) and a.offset.item() == b.offset.item()
    assert tuple(b.shape) == (640, 1536)
    assert torch.equal(dequantize_4bit(src.weight.data, a), dequantize_4bit(dst.weight.data, b))
    x = torch.randn(3, 50, 1536, device=device, dtype=torch.float16)
    assert torch.equal(src(x), dst(x))


def test_from_prequantized(device):
    src = _layer(device, n=256)
    stats = {k: v.cpu() for k, v in src.weight.quant_state.as_dict(packed=True).items()}
    w = Params4bit.from_prequantized(src.weight.data.cpu(), stats, device=device)
    assert w.quant_state.quant_type == "nf4" and w.blocksize == 64 and w.compress_statistics
    assert torch.equal(dequantize_4bit(w.data, w.quant_state),
                       dequantize_4bit(src.weight.data, src.weight.quant_state))
