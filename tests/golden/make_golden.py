"""Write the committed NF4 golden fixtures (small .npz files, data only).

nf4_synthetic.npz: the reference's synthetic nested states
(solution/tests/test_nf4_fast.py:85-99: packed = arange % 256, qabs = arange % 256,
code2 = linspace(-1, 1, 256), absmax2 = 1.125 + 0.375 j, offset 0 / 0.0625) at
tail-heavy shapes from that test's list, and their decoded fp16 output.
nf4_quantized.npz: seeded N(0, 0.02) fp16 weights quantized by the oracle's
restated encoder, and their decoded output.

The expected outputs come from oracle/nf4.py, whose decoder is pinned by the
independent checks in tests/test_oracle_nf4.py; the fixtures freeze those
vectors so that GPU tests and later oracle edits are checked against the same
bits.  Run from the repository root:  python tests/golden/make_golden.py
"""

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import nf4  # noqa: E402

HERE = Path(__file__).resolve().parent


def put(store, stem, state):
    store[stem + "_shape"] = np.array(state.shape, np.int64)
    store[stem + "_packed"] = state.packed
    store[stem + "_qabs"] = state.qabs
    store[stem + "_absmax2"] = state.absmax2
    store[stem + "_code2"] = state.code2
    store[stem + "_offset"] = state.offset
    store[stem + "_out"] = state.decode()


def main():
    store = {}
    for shape in [(1, 1), (1, 3), (1, 9), (3, 21), (1, 65), (7, 13), (17, 127), (1, 4097),
                  (1, 16385), (256, 64)]:
        for offset in (0.0, 0.0625):
            tag = f"s{shape[0]}x{shape[1]}_o{int(offset * 10000)}"
            put(store, tag, nf4.synthetic_state(shape, offset))
    np.savez_compressed(HERE / "nf4_synthetic.npz", **store)

    store = {}
    rng = np.random.default_rng(2026)
    for shape in [(7, 13), (17, 127), (64, 128), (32, 1536)]:
        w = (rng.standard_normal(shape) * 0.02).astype(np.float16)
        tag = f"q{shape[0]}x{shape[1]}"
        put(store, tag, nf4.quantize_nested(w))
        store[tag + "_weight"] = w
    np.savez_compressed(HERE / "nf4_quantized.npz", **store)


if __name__ == "__main__":
    main()
