"""NF4 format, encoder and exact decoders (numpy) -- test infrastructure only.

Reference anchors (all relative to the reference tree):
  * format table and nibble order: solution/kernels/nf4.py:6-7,32-37,44-47
    (byte j holds element 2j in the HIGH nibble, element 2j+1 in the low one)
  * nested decode formula (A2):   solution/kernels/nf4.py:7-10,48-58
        scale = fp32(fp32(code2[qabs[b]] * absmax2[b // 256]) + offset)
        out[i] = fp16_rne(fp32(NF4[nibble(i)] * scale)),  b = i // 64
    with floating-point contraction disabled (nf4.py:126, enable_fp_fusion=False)
  * flat decode (A3):             solution/kernels/nf4.py:56-57,181-187
        out[i] = fp16_rne(fp32(NF4[nibble(i)] * absmax_f32[i // 64]))
  * synthetic nested state:       solution/tests/test_nf4_fast.py:85-99

The encoder follows bitsandbytes 0.50.2 (third-party, pinned by the
reference at solution/nf4_patch.py:53; not present in /root/reference and not
installed here): ``functional.quantize_4bit(A, blocksize=64,
compress_statistics=True, quant_type="nf4")``.  Its published algorithm is
restated below: per-64-block absmax, multiply by the fp32 reciprocal, pick the
NF4 code by midpoint thresholds, pack two codes per byte; then subtract the
mean absmax and 8-bit quantize the remainder blockwise (block 256) with the
signed dynamic map.  Bit parity of the ENCODER against bitsandbytes is
therefore unpinned; decode parity is unaffected because the decoder is
defined on whatever state it is given.

Pins (tests/test_oracle_nf4.py):
  * fp16 conversion: numpy's float32->float16 cast is checked against an
    integer bit-level round-to-nearest-even restatement on every halfway case
    and the subnormal range;
  * decode_nested == decode_flat(blockwise_absmax(...)) for every state
    (the two reference paths must agree, nf4.py:181-187 vs :41-59);
  * decoding the reference's synthetic state (arange bytes, linspace code2)
    against a per-element scalar loop written from the docstring formula and
    against committed golden vectors;
  * all-zero weights decode to signed zeros (test_nf4.py:78-85 semantics);
  * encoder: round trip error <= half the widest NF4 gap * absmax + the 8-bit
    absmax quantization error; every chosen code is a nearest code.
"""

import numpy as np

# Sixteen NF4 code points (format data; solution/kernels/nf4.py:32-37).
NF4_VALUES = np.array([
    -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
    -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
    0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
    0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0,
], dtype=np.float32)

BLOCK = 64        # NF4 block size (solution/kernels/nf4.py:147)
BLOCK2 = 256      # second-level block size (solution/kernels/nf4.py:160)


def f32(x):
    return np.asarray(x, dtype=np.float32)


def unpack_nibbles(packed, n):
    """Element i's 4-bit code: high nibble for even i, low for odd i (nf4.py:44-47)."""
    packed = np.asarray(packed, dtype=np.uint8).reshape(-1)
    idx = np.arange(n, dtype=np.int64)
    byte = packed[idx // 2].astype(np.int32)
    return np.where((idx & 1) == 0, byte >> 4, byte & 15).astype(np.int64)


def pack_nibbles(codes):
    codes = np.asarray(codes, dtype=np.uint8).reshape(-1)
    if codes.size % 2:
        codes = np.concatenate([codes, np.zeros(1, np.uint8)])
    return ((codes[0::2] << 4) | codes[1::2]).astype(np.uint8)


def blockwise_absmax(qabs, absmax2, code2, offset, nblocks):
    """fp32 scale per 64-block: fp32(fp32(code2[q] * absmax2[b//256]) + offset).

    Equals bitsandbytes ``dequantize_blockwise(qabs, state2) + offset``, the
    fp32 absmax the flat path receives (solution/tests/test_nf4.py:110).
    """
    b = np.arange(nblocks, dtype=np.int64)
    code_value = f32(code2)[np.asarray(qabs, dtype=np.int64)[b]]
    product = (code_value * f32(absmax2)[b // BLOCK2]).astype(np.float32)
    return (product + np.float32(np.asarray(offset, dtype=np.float32).reshape(-1)[0])).astype(np.float32)


def decode_flat(packed, absmax_f32, n):
    """A3: fp16(NF4[nibble] * absmax_f32[i // 64]) (solution/kernels/nf4.py:56-58)."""
    nib = unpack_nibbles(packed, n)
    scale = f32(absmax_f32)[np.arange(n, dtype=np.int64) // BLOCK]
    return (NF4_VALUES[nib] * scale).astype(np.float32).astype(np.float16)


def decode_nested(packed, qabs, absmax2, code2, offset, n):
    """A2: nested decode, no FMA, one RNE rounding to fp16 (nf4.py:7-10,41-59)."""
    nblocks = -(-n // BLOCK)
    return decode_flat(packed, blockwise_absmax(qabs, absmax2, code2, offset, nblocks), n)


# ---------------------------------------------------------------- encoder ---

def dynamic_map_signed():
    """bitsandbytes ``create_dynamic_map(signed=True, max_exponent_bits=7, total_bits=8)``.

    For exponent i in 0..6: 2**i midpoints of linspace(0.1, 1, 2**i + 1),
    scaled by 10**(i-6), with both signs; plus 0 and 1.0; sorted (256 values).
    The published recipe builds the float32 boundaries with torch.linspace on
    the CPU, so this restatement does too (its rounding is part of the table).
    """
    import torch

    data = []
    for i in range(7):
        items = 2 ** i + 1
        bounds = torch.linspace(0.1, 1.0, items, dtype=torch.float32)
        means = (bounds[:-1] + bounds[1:]) / 2.0
        scaled = (10.0 ** (i - 6)) * means
        data += scaled.tolist()
        data += (-scaled).tolist()
    data += [0.0, 1.0]
    assert len(data) == 256
    return np.array(sorted(data), dtype=np.float32)


def nf4_thresholds():
    """Midpoints between consecutive NF4 codes, as fp32 comparison constants."""
    v = NF4_VALUES.astype(np.float64)
    return ((v[:-1] + v[1:]) / 2.0).astype(np.float32)


def quantize_nf4(w):
    """Return (packed uint8[ceil(n/2)], absmax fp32[ceil(n/64)]) for fp16/fp32 w.

    Code = number of midpoint thresholds strictly below x*(1/absmax); a NaN
    (zero block: 0 * inf) compares false everywhere and gets code 0, as the
    threshold decision tree of the published kernel does.
    """
    x = np.asarray(w).reshape(-1).astype(np.float32)
    n = x.size
    nblocks = -(-n // BLOCK)
    padded = np.zeros(nblocks * BLOCK, np.float32)
    padded[:n] = x
    valid = np.arange(nblocks * BLOCK) < n
    mag = np.where(valid, np.abs(padded), 0).reshape(nblocks, BLOCK)
    absmax = mag.max(axis=1).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        inv = (np.float32(1.0) / absmax).astype(np.float32)
        normed = (padded.reshape(nblocks, BLOCK) * inv[:, None]).astype(np.float32).reshape(-1)[:n]
        t = nf4_thresholds()
        codes = (normed[:, None] > t[None, :]).sum(axis=1)
    return pack_nibbles(codes), absmax


def _quantize_8bit_code(x, code):
    """Published 8-bit dynamic quantizer: bisection from pivot 127, then midpoint."""
    out = np.empty(x.size, np.uint8)
    for j, v in enumerate(np.asarray(x, np.float32)):
        pivot, upper_pivot, lower_pivot = 127, 255, 0
        lower, upper = np.float32(-1.0), np.float32(1.0)
        val = code[pivot]
        step = 64
        while step > 0:
            if v > val:
                lower_pivot, lower = pivot, val
                pivot += step
            else:
                upper_pivot, upper = pivot, val
                pivot -= step
            val = code[pivot]
            step >>= 1
        if upper_pivot == 255:
            upper = code[upper_pivot]
        if lower_pivot == 0:
            lower = code[lower_pivot]
        if v > val:
            mid = np.float32((upper + val) * np.float32(0.5))
            out[j] = upper_pivot if v > mid else pivot
        else:
            mid = np.float32((lower + val) * np.float32(0.5))
            out[j] = lower_pivot if v < mid else pivot
    return out


def double_quant(absmax, offset=None):
    """Compress fp32 absmax: offset=mean; 8-bit blockwise (256) of absmax-offset.

    Returns (qabs uint8[nblocks], absmax2 fp32[ceil(nblocks/256)], code2 fp32[256], offset fp32[1]).
    ``offset`` may be given to reuse another implementation's mean (the mean's
    summation order is not part of the format).
    """
    absmax = f32(absmax)
    if offset is None:
        offset = np.float32(absmax.mean(dtype=np.float32))
    offset = np.float32(np.asarray(offset, np.float32).reshape(-1)[0])
    centered = (absmax - offset).astype(np.float32)
    nb = centered.size
    groups = -(-nb // BLOCK2)
    padded = np.zeros(groups * BLOCK2, np.float32)
    padded[:nb] = centered
    absmax2 = np.abs(padded).reshape(groups, BLOCK2).max(axis=1).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        inv = (np.float32(1.0) / absmax2).astype(np.float32)
        normed = (padded.reshape(groups, BLOCK2) * inv[:, None]).astype(np.float32).reshape(-1)[:nb]
    code2 = dynamic_map_signed()
    qabs = _quantize_8bit_code_fast(normed, code2)
    return qabs, absmax2, code2, np.array([offset], np.float32)


def _quantize_8bit_code_fast(x, code):
    """Vectorised form of ``_quantize_8bit_code`` (same decisions, elementwise)."""
    x = np.asarray(x, np.float32)
    pivot = np.full(x.size, 127, np.int64)
    upper_pivot = np.full(x.size, 255, np.int64)
    lower_pivot = np.zeros(x.size, np.int64)
    lower = np.full(x.size, -1.0, np.float32)
    upper = np.full(x.size, 1.0, np.float32)
    val = code[pivot]
    step = 64
    while step > 0:
        gt = x > val
        lower_pivot = np.where(gt, pivot, lower_pivot)
        lower = np.where(gt, val, lower)
        upper_pivot = np.where(gt, upper_pivot, pivot)
        upper = np.where(gt, upper, val)
        pivot = np.where(gt, pivot + step, pivot - step)
        val = code[pivot]
        step >>= 1
    upper = np.where(upper_pivot == 255, code[255], upper).astype(np.float32)
    lower = np.where(lower_pivot == 0, code[0], lower).astype(np.float32)
    gt = x > val
    mid_hi = ((upper + val) * np.float32(0.5)).astype(np.float32)
    mid_lo = ((lower + val) * np.float32(0.5)).astype(np.float32)
    res = np.where(gt, np.where(x > mid_hi, upper_pivot, pivot),
                   np.where(x < mid_lo, lower_pivot, pivot))
    return res.astype(np.uint8)


class NF4State:
    """Plain container mirroring bitsandbytes QuantState fields (solution/kernels/nf4.py:140-168)."""

    def __init__(self, shape, packed, qabs, absmax2, code2, offset):
        self.shape = tuple(shape)
        self.packed, self.qabs, self.absmax2 = packed, qabs, absmax2
        self.code2, self.offset = code2, offset

    @property
    def n(self):
        return int(np.prod(self.shape))

    def decode(self):
        return decode_nested(self.packed, self.qabs, self.absmax2, self.code2,
                             self.offset, self.n).reshape(self.shape)

    def decode_exact(self):
        """float64 NF4[nibble] * scale with no rounding (the product of two fp32
        values is exact in float64): the weight the fp16 decode rounds."""
        return decode_exact(self.packed, self.qabs, self.absmax2, self.code2, self.offset,
                            self.n).reshape(self.shape)


def decode_exact(packed, qabs, absmax2, code2, offset, n):
    """Unrounded nested decode: float64(NF4[nibble(i)]) * float64(scale[i // 64]).

    decode_nested is this value rounded to fp32 and then to fp16.  Used as the
    exact-weight reference when a GEMM's error is compared with the error of the
    reference's own decode-then-dense path.
    """
    nblocks = -(-n // BLOCK)
    scale = blockwise_absmax(qabs, absmax2, code2, offset, nblocks).astype(np.float64)
    nib = unpack_nibbles(packed, n)
    return NF4_VALUES.astype(np.float64)[nib] * scale[np.arange(n, dtype=np.int64) // BLOCK]


def quantize_nested(w):
    """quantize_4bit(..., compress_statistics=True, quant_type='nf4') restated."""
    w = np.asarray(w)
    packed, absmax = quantize_nf4(w)
    qabs, absmax2, code2, offset = double_quant(absmax)
    return NF4State(w.shape, packed, qabs, absmax2, code2, offset)


def synthetic_state(shape, offset):
    """The reference's synthetic nested state (solution/tests/test_nf4_fast.py:85-99).

    packed = arange % 256 over ceil(n/2) bytes, qabs = arange % 256 over
    ceil(n/64) blocks, code2 = linspace(-1, 1, 256), absmax2 = 1.125 + 0.375*j.
    """
    n = int(np.prod(shape))
    blocks = -(-n // BLOCK)
    packed = (np.arange(-(-n // 2), dtype=np.int64) % 256).astype(np.uint8)
    qabs = (np.arange(blocks, dtype=np.int64) % 256).astype(np.uint8)
    code2 = np.linspace(-1, 1, 256).astype(np.float32)
    absmax2 = (np.float32(1.125) + np.float32(0.375) *
               np.arange(-(-blocks // BLOCK2), dtype=np.float32)).astype(np.float32)
    return NF4State(shape, packed, qabs, absmax2, code2, np.array([offset], np.float32))
