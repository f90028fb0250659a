"""Right-padding removal oracle (A16) -- test infrastructure only.

Reference semantics (solution/unpad.py:51-72,149-161,184-199):
  * right_padding_lengths(rows): a binary, nonempty, right-padded mask gives
    per-row lengths; anything else gives None;
  * indices[t] = row * S + position for position < length[row], row-major;
  * pack:    [B*S, H] -> [T, H] by index_select(indices);
  * scatter: zeros[B*S, H] then index_copy(indices, packed).
Both copies are bit-exact.

Pins: the reference's own table (solution/tests/test_unpad.py:23-37) and its
indices example lengths (1, 3), S = 3 -> [0, 3, 4, 5] (test_unpad.py:183-184);
scatter(pack(x)) == x * mask and pack(scatter(p)) == p.
"""

import numpy as np


def right_padding_lengths(rows):
    if not rows or not rows[0]:
        return None
    width = len(rows[0])
    lengths = []
    for row in rows:
        if len(row) != width:
            return None
        count, padding = 0, False
        for value in row:
            if value not in (0, 1):
                return None
            if value == 0:
                padding = True
            elif padding:
                return None
            else:
                count += 1
        if not count:
            return None
        lengths.append(count)
    return tuple(lengths)


def indices_from_lengths(lengths, sequence):
    return np.concatenate([row * sequence + np.arange(n, dtype=np.int64)
                           for row, n in enumerate(lengths)]) if lengths else np.zeros(0, np.int64)


def pack(x, indices):
    x = np.asarray(x)
    return x.reshape(-1, x.shape[-1])[np.asarray(indices)]


def scatter(packed, indices, batch, sequence):
    packed = np.asarray(packed)
    out = np.zeros((batch * sequence, packed.shape[-1]), dtype=packed.dtype)
    out[np.asarray(indices)] = packed
    return out.reshape(batch, sequence, packed.shape[-1])
