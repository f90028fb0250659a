"""CPU tests of the serialized QuantState (bnb_compat.QuantState.as_dict / from_dict).

The format is bitsandbytes 0.50.2's checkpoint layout (not installed here, so
it is pinned by a spelled-out golden record instead of an import): the tensors
absmax / quant_map / nested_absmax / nested_quant_map, and the key
``quant_state.bitsandbytes__nf4`` holding the UTF-8 bytes of
``json.dumps`` of the remaining fields in the order quant_type, blocksize,
dtype, shape, nested_blocksize, nested_dtype, nested_offset.  A Linear4bit
state dict carries these under ``<prefix>weight.``.
"""

import json

import pytest
import torch

from soupsuck_amd.bnb_compat import (QuantState, pack_dict_to_tensor, unpack_tensor_to_dict)

GOLDEN_JSON = ('{"quant_type": "nf4", "blocksize": 64, "dtype": "float16", "shape": [4, 64], '
               '"nested_blocksize": 256, "nested_dtype": "float32", "nested_offset": 0.03125}')


def _state():
    gen = torch.Generator().manual_seed(0)
    state2 = QuantState(torch.rand(1, generator=gen), code=torch.linspace(-1, 1, 256),
                        blocksize=256, dtype=torch.float32)
    return QuantState(torch.randint(0, 256, (4,), dtype=torch.uint8, generator=gen),
                      shape=(4, 64), code=torch.linspace(-1, 1, 16), blocksize=64,
                      quant_type="nf4", dtype=torch.float16,
                      offset=torch.tensor([0.03125]), state2=state2)


def test_packed_record_matches_the_golden_layout():
    st = _state()
    d = st.as_dict(packed=True)
    assert list(d) == ["absmax", "quant_map", "nested_absmax", "nested_quant_map",
                       "quant_state.bitsandbytes__nf4"]
    blob = d["quant_state.bitsandbytes__nf4"]
    assert blob.dtype == torch.uint8 and bytes(blob.tolist()).decode() == GOLDEN_JSON
    assert torch.equal(d["absmax"], st.absmax) and d["absmax"].dtype == torch.uint8
    assert torch.equal(d["nested_quant_map"], st.state2.code)
    assert d["nested_quant_map"].data_ptr() != st.state2.code.data_ptr()   # not shared
    assert all(isinstance(v, torch.Tensor) for v in d.values())


def test_unpacked_record_keeps_plain_fields():
    d = _state().as_dict()
    assert d["quant_type"] == "nf4" and d["blocksize"] == 64 and d["dtype"] == "float16"
    assert d["shape"] == (4, 64) and d["nested_offset"] == 0.03125
    assert json.dumps({k: v for k, v in d.items() if not isinstance(v, torch.Tensor)}) \
        == GOLDEN_JSON


@pytest.mark.parametrize("packed, prefix", [(True, ""), (False, ""),
                                             (True, "model.layers.0.mlp.gate_proj.weight.")])
def test_round_trip(packed, prefix):
    # Key prefixes (state-dict names) are stripped; an unpacked record is read
    # by its bare "quant_type" key, as bitsandbytes does.
    st = _state()
    d = {prefix + k: v for k, v in st.as_dict(packed=packed).items()}
    back = QuantState.from_dict(d, device="cpu")
    assert back.quant_type == "nf4" and back.blocksize == 64 and back.dtype == torch.float16
    assert back.shape == torch.Size((4, 64)) and back.nested
    assert torch.equal(back.absmax, st.absmax) and torch.equal(back.code, st.code)
    assert torch.equal(back.state2.absmax, st.state2.absmax)
    assert torch.equal(back.state2.code, st.state2.code)
    assert back.state2.blocksize == 256 and back.state2.dtype == torch.float32
    assert not back.state2.nested
    assert back.offset.item() == 0.03125 and back.offset.dtype == torch.float32


def test_pack_unpack_inverse():
    items = {"quant_type": "nf4", "shape": [3, 5], "nested_offset": -1.5e-3}
    assert unpack_tensor_to_dict(pack_dict_to_tensor(items)) == items


def test_malformed_records_raise():
    d = _state().as_dict(packed=True)
    with pytest.raises(ValueError, match="neither"):
        QuantState.from_dict({"absmax": d["absmax"]}, device="cpu")
    two = dict(d)
    two["other.quant_state.bitsandbytes__nf4"] = d["quant_state.bitsandbytes__nf4"]
    with pytest.raises(ValueError, match="exactly one"):
        QuantState.from_dict(two, device="cpu")
    bad = dict(d)
    bad["quant_state.bitsandbytes__int8"] = bad.pop("quant_state.bitsandbytes__nf4")
    with pytest.raises(ValueError, match="exactly one"):
        QuantState.from_dict(bad, device="cpu")
    extra = dict(d)
    extra["weight.something_else"] = torch.zeros(1)
    with pytest.raises(ValueError, match="unknown"):
        QuantState.from_dict(extra, device="cpu")
