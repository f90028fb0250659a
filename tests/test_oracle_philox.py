"""CPU checks of oracle/philox.py (the fused LoRA dropout's mask definition).

  * Philox4x32-10 against the published known-answer vectors of the Random123
    distribution (kat_vectors: counters 0, all-ones and the pi digits);
  * a planted mistake (9 rounds instead of 10, or a swapped multiplier) fails them;
  * keep(e) uses word e mod 4 of the counter e div 4 (checked against a direct
    per-element evaluation), rows are laid out row-major, and the keep rate of
    2^20 elements lies within 6 standard deviations of 1 - p;
  * dropped values are fp32(x) * fp32(1 / (1 - p)) or 0.
"""

import numpy as np
import pytest

from oracle import philox

KAT = [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("ctr, key, expect", KAT)
def test_known_answers(ctr, key, expect):
    got = philox.philox4x32_10(np.array([ctr], dtype=np.uint32), key)[0]
    assert tuple(int(v) for v in got) == expect


def test_planted_mistakes_fail_the_known_answers(monkeypatch):
    ctr, key, expect = KAT[2]
    monkeypatch.setattr(philox, "M0", np.uint64(0xCD9E8D57))       # swapped multiplier
    got = philox.philox4x32_10(np.array([ctr], dtype=np.uint32), key)[0]
    assert tuple(int(v) for v in got) != expect


def _direct_keep(seed, p, e):
    ctr = np.array([[(e // 4) & 0xFFFFFFFF, (e // 4) >> 32, 0, 0]], dtype=np.uint64)
    word = philox.philox4x32_10(ctr, (seed & 0xFFFFFFFF, seed >> 32))[0][e % 4]
    return int(word) < philox.threshold(p)


def test_mask_indexing_is_row_major_per_element():
    seed, p, rows, cols = 0x1234_5678_9ABC_DEF0, 0.3, 5, 12
    mask = philox.keep_mask(seed, p, rows, cols)
    for r in range(rows):
        for c in range(cols):
            assert mask[r, c] == _direct_keep(seed, p, r * cols + c)
    assert not np.array_equal(mask, philox.keep_mask(seed + 1, p, rows, cols))


@pytest.mark.parametrize("p", [0.05, 0.1, 0.5])
def test_keep_rate(p):
    n = 1 << 20
    kept = philox.keep_mask(987654321, p, 1, n).sum()
    mean, sd = n * (1 - p), (n * p * (1 - p)) ** 0.5
    assert abs(kept - mean) < 6 * sd


def test_dropped_values():
    x = np.array([[1.5, -2.0, 3.0, 0.25]], dtype=np.float16)
    keep = np.array([[True, False, True, True]])
    out = philox.dropped(x, keep, 0.1)
    inv = np.float32(1.0 / (1.0 - float(np.float32(0.1))))
    assert out.dtype == np.float32
    assert np.array_equal(out, np.array([[1.5 * inv, 0.0, 3.0 * inv, 0.25 * inv]], np.float32))
    assert philox.threshold(0.5) == 2 ** 31


def test_tiny_p_threshold_saturates():
    """(1 - p) * 2^32 rounds to 2^32 for p below about 1.1e-16; the threshold then saturates
    at 2^32 - 1 instead of wrapping to 0 (which would drop every element)."""
    assert philox.threshold(1e-20) == 0xFFFFFFFF
    assert philox.threshold(float(np.float32(2.0 ** -40))) == 0xFFFFFFFF
    assert philox.threshold(2.0 ** -31) == 2 ** 32 - 2
    assert philox.keep_mask(42, 1e-20, 4, 256).all()
