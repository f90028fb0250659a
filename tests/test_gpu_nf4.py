"""GPU parity of the NF4 decoder and encoder (ss_nf4_dequant_* / ss_nf4_quantize).

Bar: bit-exact (int16 views, so +0/-0 differ) against oracle/nf4.py and the
committed golden fixtures.  Cases follow the reference's tests:
solution/tests/test_nf4.py (real quantized states at Qwen shapes and tiny
shapes, transposed packed view, zero weight sign bits, out= aliasing,
unsupported states) and solution/tests/test_nf4_fast.py (synthetic states
with every byte value and tails, signed flat scales, unaligned out/packed).
"""

import copy
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import nf4 as onf4
from soupsuck_amd import _lib
from soupsuck_amd.bnb_compat import dynamic_map_signed, quantize_4bit
from soupsuck_amd.kernels import nf4 as knf4
from tests.gpu_util import bits, device_state, random_weight

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"

SYNTHETIC_SHAPES = [(1, 1), (1, 2), (1, 3), (1, 5), (1, 6), (1, 7), (1, 8), (1, 9), (3, 21), (1, 64),
                    (1, 65), (7, 13), (1, 4095), (1, 4096), (1, 4097), (1, 16383), (1, 16384),
                    (1, 16385), (1536, 1536), (8960, 1536), (1536, 8960), (256, 1536)]


@pytest.mark.parametrize("name", ["nf4_synthetic.npz", "nf4_quantized.npz"])
def test_golden_fixtures_bit_exact(device, name):
    data = np.load(GOLDEN / name, allow_pickle=False)
    for key in sorted(k for k in data.files if k.endswith("_out")):
        stem = key[:-4]
        state = onf4.NF4State(tuple(data[stem + "_shape"]), data[stem + "_packed"],
                              data[stem + "_qabs"], data[stem + "_absmax2"],
                              data[stem + "_code2"], data[stem + "_offset"])
        packed, qs = device_state(state, device)
        out = knf4.dequantize_nf4(packed, qs)
        np.testing.assert_array_equal(bits(out), data[key].view(np.int16), err_msg=stem)


@pytest.mark.parametrize("shape", SYNTHETIC_SHAPES)
@pytest.mark.parametrize("offset", [0.0, 0.0625])
def test_synthetic_state_bit_exact(device, shape, offset):
    state = onf4.synthetic_state(shape, offset)
    packed, qs = device_state(state, device)
    expected = state.decode().view(np.int16)
    # reference view rule (solution/kernels/nf4.py:203): a packed tensor whose
    # first dimension is 1 returns the transposed view of the canonical output
    out = knf4.dequantize_nf4(packed, qs)
    np.testing.assert_array_equal(bits(out), expected.T if packed.shape[0] == 1 else expected)
    out_t = knf4.dequantize_nf4(packed.t(), qs)
    assert out_t.shape == (shape[1], shape[0])
    np.testing.assert_array_equal(bits(out_t.t()), expected)


@pytest.mark.parametrize("shape", [(1536, 1536), (8960, 1536), (1536, 8960), (256, 1536), (7, 13),
                                   (3, 65), (17, 127), (1, 1), (1, 3)])
def test_real_quantized_weights_bit_exact(device, shape):
    state = onf4.quantize_nested(random_weight(*shape, seed=2026))
    packed, qs = device_state(state, device)
    np.testing.assert_array_equal(bits(knf4.dequantize_nf4(packed, qs)),
                                  state.decode().view(np.int16))


def test_zero_weight_sign_bits(device):
    packed, qs = quantize_4bit(torch.zeros((17, 127), device=device, dtype=torch.float16))
    out = knf4.dequantize_nf4(packed, qs)
    ref = onf4.quantize_nested(np.zeros((17, 127), np.float16))
    np.testing.assert_array_equal(bits(out), ref.decode().view(np.int16))
    assert np.all(bits(out) == np.int16(-32768))   # every element is -0.0


def test_out_is_written_in_place_without_allocation(device):
    state = onf4.synthetic_state((256, 64), 0.0625)
    packed, qs = device_state(state, device)
    out = torch.empty((256, 64), device=device, dtype=torch.float16)
    knf4.dequantize_nf4(packed, qs)   # warm up
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    result = knf4.dequantize_nf4(packed, qs, out=out)
    torch.cuda.synchronize()
    assert result.data_ptr() == out.data_ptr()
    assert torch.cuda.max_memory_allocated() == before
    np.testing.assert_array_equal(bits(out), state.decode().view(np.int16))


@pytest.mark.parametrize("n", [1, 2, 3, 5, 6, 7, 8, 9, 63, 64, 65, 4095, 4096, 4097, 16385])
def test_flat_signed_scales_and_unaligned_out(device, n):
    state = onf4.synthetic_state((1, n), 0.0)
    packed, _ = device_state(state, device)
    blocks = -(-n // 64)
    scales = torch.linspace(-2, 2, blocks, device=device, dtype=torch.float32)
    guarded = torch.full((n + 2,), 123.0, device=device, dtype=torch.float16)
    out = guarded[1:n + 1].view(1, n)   # contiguous, not 16-byte aligned
    assert knf4._dequantize_flat_into(packed, scales, out).data_ptr() == out.data_ptr()
    expected = onf4.decode_flat(state.packed, scales.cpu().numpy(), n)
    np.testing.assert_array_equal(bits(out).reshape(-1), expected.view(np.int16))
    assert guarded[0].item() == 123.0 and guarded[-1].item() == 123.0


def test_unaligned_packed_view(device):
    state = onf4.synthetic_state((17, 127), 0.0625)
    packed, qs = device_state(state, device)
    storage = torch.empty(packed.numel() + 1, dtype=torch.uint8, device=device)
    source = storage[1:].view(packed.shape)
    source.copy_(packed)
    assert source.data_ptr() % 4 != 0
    np.testing.assert_array_equal(bits(knf4.dequantize_nf4(source, qs)),
                                  state.decode().view(np.int16))


def test_unsupported_states_raise_before_launch(device):
    state = onf4.synthetic_state((17, 128), 0.0)
    packed, qs = device_state(state, device)
    with pytest.raises(ValueError, match="fp16"):
        knf4.dequantize_nf4(packed, qs, torch.float32)
    for field, value in (("quant_type", "fp4"), ("blocksize", 128), ("nested", False)):
        changed = copy.copy(qs)
        setattr(changed, field, value)
        with pytest.raises(ValueError):
            knf4.dequantize_nf4(packed, changed)
    changed = copy.copy(qs)
    changed.state2 = copy.copy(qs.state2)
    changed.state2.blocksize = 64
    with pytest.raises(ValueError, match="state2"):
        knf4.dequantize_nf4(packed, changed)


@pytest.mark.parametrize("shape", [(7, 13), (17, 127), (256, 1536), (8960, 1536), (1, 65)])
def test_gpu_encoder_matches_restated_encoder(device, shape):
    w = random_weight(*shape, seed=7)
    n = w.size
    blocks = -(-n // 64)
    wt = torch.from_numpy(w).to(device)
    packed = torch.empty(-(-n // 2), dtype=torch.uint8, device=device)
    qabs = torch.empty(blocks, dtype=torch.uint8, device=device)
    absmax2 = torch.empty(-(-blocks // 256), dtype=torch.float32, device=device)
    offset = torch.empty(1, dtype=torch.float32, device=device)
    absmax = torch.empty(blocks, dtype=torch.float32, device=device)
    code2 = dynamic_map_signed().to(device)
    np.testing.assert_array_equal(code2.cpu().numpy(), onf4.dynamic_map_signed())
    _lib.call("ss_nf4_quantize", wt.data_ptr(), _lib.F16, n, packed.data_ptr(), qabs.data_ptr(),
              absmax2.data_ptr(), code2.data_ptr(), offset.data_ptr(), absmax.data_ptr(),
              _lib.stream(device))
    ref_packed, ref_absmax = onf4.quantize_nf4(w)
    np.testing.assert_array_equal(packed.cpu().numpy(), ref_packed)
    np.testing.assert_array_equal(absmax.cpu().numpy(), ref_absmax)
    # the mean's summation order is not part of the format: compare given the same offset
    assert abs(offset.item() - float(ref_absmax.mean(dtype=np.float64))) <= 1e-6 * ref_absmax.max()
    ref_q, ref_a2, _, _ = onf4.double_quant(ref_absmax, offset=offset.cpu().numpy())
    np.testing.assert_array_equal(absmax2.cpu().numpy(), ref_a2)
    np.testing.assert_array_equal(qabs.cpu().numpy(), ref_q)


@pytest.mark.parametrize("shape", [(64, 64), (256, 1536), (1536, 8960), (8960, 1536), (37, 128),
                                   (100, 192)])
def test_transposed_decode_bit_exact(device, shape):
    state = onf4.quantize_nested(random_weight(*shape, seed=11))
    packed, qs = device_state(state, device)
    rows, cols = shape
    out = torch.empty((cols, rows), device=device, dtype=torch.float16)
    _lib.call("ss_nf4_dequant_nested_t", packed.data_ptr(), qs.absmax.data_ptr(),
              qs.state2.absmax.data_ptr(), qs.state2.code.data_ptr(), qs.offset.data_ptr(),
              out.data_ptr(), rows, cols, _lib.stream(device))
    np.testing.assert_array_equal(bits(out), state.decode().T.view(np.int16))
