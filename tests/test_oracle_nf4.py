"""CPU pins of the NF4 oracle (oracle/nf4.py) -- no GPU, no reference import.

What each test pins:
  * numpy's float32 -> float16 cast against an integer restatement of IEEE
    round-to-nearest-even (normal, halfway, subnormal, overflow cases);
  * the NF4 table's decimal literals are exactly fp32 values;
  * the vectorised decoder against a scalar per-element decoder written from
    the reference docstring (solution/kernels/nf4.py:7-10) with struct-based
    fp32 rounding and the bit-level fp16 rounding above: a swapped nibble,
    a wrong block/group index or a fused multiply-add fails it;
  * hand-computed known answers on the reference's synthetic state
    (solution/tests/test_nf4_fast.py:85-99);
  * nested decode == flat decode of the reconstructed fp32 absmax (the two
    reference entry points, nf4.py:41-59 vs :181-187);
  * signed zeros of an all-zero weight (solution/tests/test_nf4.py:78-85);
  * encoder invariants: nearest-code choice and bounded round-trip error;
  * committed golden fixtures (tests/golden/nf4_*.npz) reproduce.
"""

import struct
from pathlib import Path

import numpy as np
import pytest

from oracle import nf4

GOLDEN = Path(__file__).resolve().parent / "golden"


def f32(x):
    return struct.unpack("<f", struct.pack("<f", x))[0]


def f32_to_f16_bits(x):
    """IEEE binary32 -> binary16 bits, round to nearest even (integer arithmetic)."""
    b = struct.unpack("<I", struct.pack("<f", x))[0]
    sign = (b >> 16) & 0x8000
    exp = (b >> 23) & 0xFF
    mant = b & 0x7FFFFF
    if exp == 0xFF:
        return sign | 0x7C00 | (0x200 if mant else 0)
    if exp == 0 and mant == 0:
        return sign
    # Significand as an integer with 23 fractional bits; value = sig * 2**(e - 23).
    if exp == 0:
        sig, e = mant, -126
    else:
        sig, e = mant | 0x800000, exp - 127
    # Target: half value = q * 2**(he - 10) with q an integer, he >= -14.
    he = max(e, -14)
    shift = 23 - 10 + (he - e)           # bits to drop from sig
    q, rem = sig >> shift, sig & ((1 << shift) - 1)
    half = 1 << (shift - 1)
    if rem > half or (rem == half and (q & 1)):
        q += 1
    if q >= 2048:                        # carried into the next binade
        q >>= 1
        he += 1
    if he > 15:
        return sign | 0x7C00
    if q < 1024:                         # subnormal (he == -14)
        return sign | q
    return sign | ((he + 15) << 10) | (q - 1024)


def np_half_bits(x):
    return int(np.array([x], np.float32).astype(np.float16).view(np.uint16)[0])


def test_fp16_rounding_matches_integer_rne():
    rng = np.random.default_rng(0)
    values = []
    # random bit patterns over the whole fp16-relevant exponent range
    for exp in range(100, 150):
        for m in rng.integers(0, 1 << 23, 40):
            values.append(struct.unpack("<f", struct.pack("<I", (exp << 23) | int(m)))[0])
    # exact halfway cases between adjacent halves (ties to even), normal and subnormal
    for hb in list(range(0, 1024, 7)) + list(range(0x0400, 0x7BFF, 97)):
        lo = np.array([hb], np.uint16).view(np.float16).astype(np.float64)[0]
        hi = np.array([hb + 1], np.uint16).view(np.float16).astype(np.float64)[0]
        mid = (lo + hi) / 2
        values += [mid, -mid, np.nextafter(np.float32(mid), np.float32(0)).item()]
    values += [65504.0, 65519.99, 65520.0, 1e-8, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 0.0, -0.0]
    for v in values:
        v = f32(v)
        assert np_half_bits(v) == f32_to_f16_bits(v), v


def test_nf4_table_literals_are_exact_fp32():
    literals = [-1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
                -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
                0.07958029955625534, 0.16093020141124725, 0.24611230194568634,
                0.33791524171829224, 0.44070982933044434, 0.5626170039176941,
                0.7229568362236023, 1.0]
    for lit, v in zip(literals, nf4.NF4_VALUES):
        assert f32(lit) == lit == float(v)
    assert np.all(np.diff(nf4.NF4_VALUES) > 0)


def scalar_decode(state):
    """Per-element decode from the docstring formula, independent of numpy casts."""
    out = []
    packed = [int(b) for b in state.packed]
    for i in range(state.n):
        byte = packed[i // 2]
        nib = (byte >> 4) if i % 2 == 0 else (byte & 15)
        b = i // 64
        code = float(state.code2[int(state.qabs[b])])
        product = f32(code * float(state.absmax2[b // 256]))
        scale = f32(product + float(state.offset[0]))
        value = f32(float(nf4.NF4_VALUES[nib]) * scale)
        out.append(f32_to_f16_bits(value))
    return np.array(out, np.uint16)


@pytest.mark.parametrize("shape", [(1, 1), (1, 2), (1, 3), (7, 13), (3, 65), (17, 127), (1, 300)])
@pytest.mark.parametrize("offset", [0.0, 0.0625])
def test_vectorised_decode_equals_scalar_formula(shape, offset):
    state = nf4.synthetic_state(shape, offset)
    got = state.decode().reshape(-1).view(np.uint16)
    np.testing.assert_array_equal(got, scalar_decode(state))


def test_scalar_formula_on_multi_group_state():
    # crosses two second-level groups (block 256 -> index 256 uses absmax2[1])
    rng = np.random.default_rng(3)
    n = 64 * 300
    state = nf4.NF4State((1, n), rng.integers(0, 256, n // 2).astype(np.uint8),
                         rng.integers(0, 256, 300).astype(np.uint8),
                         np.array([0.7, 1.9], np.float32),
                         np.sort(rng.uniform(-1, 1, 256)).astype(np.float32),
                         np.array([0.01], np.float32))
    got = state.decode().reshape(-1).view(np.uint16)
    np.testing.assert_array_equal(got, scalar_decode(state))


def test_known_answers_on_reference_synthetic_state():
    state = nf4.synthetic_state((1, 4), 0.0)
    out = state.decode().reshape(-1).astype(np.float64)
    # byte0 = 0x00, byte1 = 0x01; qabs[0] = 0 -> code2[0] = -1; absmax2[0] = 1.125
    scale = -1.125
    assert out[0] == out[1] == -1.0 * scale
    assert out[2] == -1.0 * scale
    assert out[3] == np.float16(np.float32(-0.6961928009986877) * np.float32(scale))
    # code 7 is 0.0: 0 * (negative scale) is -0.0 (sign bit set)
    s = nf4.NF4State((1, 2), np.array([0x77], np.uint8), np.array([0], np.uint8),
                     np.array([1.0], np.float32), np.linspace(-1, 1, 256).astype(np.float32),
                     np.array([0.0], np.float32))
    bits = s.decode().reshape(-1).view(np.uint16)
    assert list(bits) == [0x8000, 0x8000]
    # code 15 is 1.0: the output is exactly the scale
    s.packed = np.array([0xFF], np.uint8)
    s.qabs = np.array([255], np.uint8)
    assert list(s.decode().reshape(-1).astype(np.float32)) == [1.0, 1.0]


@pytest.mark.parametrize("shape", [(7, 13), (1, 4097), (256, 64), (3, 70000)])
def test_nested_equals_flat_of_reconstructed_absmax(shape):
    state = nf4.synthetic_state(shape, 0.0625)
    n = state.n
    absmax = nf4.blockwise_absmax(state.qabs, state.absmax2, state.code2, state.offset,
                                  -(-n // 64))
    flat = nf4.decode_flat(state.packed, absmax, n)
    np.testing.assert_array_equal(flat.view(np.uint16), state.decode().reshape(-1).view(np.uint16))


def test_zero_weight_decodes_to_signed_zeros():
    state = nf4.quantize_nested(np.zeros((17, 127), np.float16))
    out = state.decode().reshape(-1)
    assert np.all(out == 0)
    nib = nf4.unpack_nibbles(state.packed, state.n)
    bits = out.view(np.uint16)
    # every code in a zero block is 0 (NaN compares false) -> NF4 -1.0 times a +0 scale
    assert np.all(nib == 0)
    scale = nf4.blockwise_absmax(state.qabs, state.absmax2, state.code2, state.offset,
                                 -(-state.n // 64))
    expected_sign = np.where(np.signbit(scale)[np.arange(state.n) // 64], 0, 0x8000)
    np.testing.assert_array_equal(bits, expected_sign.astype(np.uint16))


def test_encoder_picks_nearest_code_and_bounds_error():
    rng = np.random.default_rng(0)
    w = (rng.standard_normal((64, 256)) * 0.02).astype(np.float16)
    packed, absmax = nf4.quantize_nf4(w)
    x = w.reshape(-1).astype(np.float32)
    codes = nf4.unpack_nibbles(packed, x.size)
    normed = x * (np.float32(1) / absmax[np.arange(x.size) // 64])
    dist = np.abs(normed[:, None] - nf4.NF4_VALUES[None, :])
    chosen = dist[np.arange(x.size), codes]
    assert np.all(chosen <= dist.min(axis=1) + 1e-7)
    state = nf4.quantize_nested(w)
    err = np.abs(state.decode().astype(np.float64).reshape(-1) - x)
    gap = np.max(np.diff(nf4.NF4_VALUES)) / 2
    bound = gap * absmax[np.arange(x.size) // 64] * 1.05 + 2e-3 * np.abs(x) + 1e-4
    assert np.all(err <= bound)


def test_double_quant_reconstructs_absmax():
    rng = np.random.default_rng(1)
    absmax = rng.uniform(0.02, 0.09, 5000).astype(np.float32)
    qabs, absmax2, code2, offset = nf4.double_quant(absmax)
    rec = nf4.blockwise_absmax(qabs, absmax2, code2, offset, absmax.size)
    assert np.max(np.abs(rec - absmax)) <= 0.02 * np.max(np.abs(absmax - offset[0])) + 1e-6
    slow = nf4._quantize_8bit_code(
        ((absmax - offset[0]) / np.repeat(absmax2, 256)[:absmax.size]).astype(np.float32)[:300],
        code2)
    np.testing.assert_array_equal(slow, qabs[:300])


def test_dynamic_map_shape():
    code = nf4.dynamic_map_signed()
    assert code.shape == (256,) and code.dtype == np.float32
    assert np.all(np.diff(code) >= 0)
    assert code[-1] == 1.0 and 0.0 in code and code[0] < -0.99
    assert np.sum(code > 0) == 128 and np.sum(code < 0) == 127


@pytest.mark.parametrize("name", ["nf4_synthetic.npz", "nf4_quantized.npz"])
def test_golden_fixtures_reproduce(name):
    data = np.load(GOLDEN / name, allow_pickle=False)
    for key in sorted(k for k in data.files if k.endswith("_out")):
        stem = key[:-4]
        state = nf4.NF4State(tuple(data[stem + "_shape"]), data[stem + "_packed"],
                             data[stem + "_qabs"], data[stem + "_absmax2"], data[stem + "_code2"],
                             data[stem + "_offset"])
        np.testing.assert_array_equal(state.decode().view(np.uint16), data[key].view(np.uint16))
