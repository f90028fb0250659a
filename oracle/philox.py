"""CPU restatement of the LoRA dropout mask (test infrastructure: only tests/, smoke()
and bench.py's cpu_baseline may import this; the product path never does).

The reference's LoRA dropout is PEFT's ``nn.Dropout`` on an fp32 copy of X
(solution/lora.py:1-40,151-163): each element kept with probability 1 - p and
scaled by 1 / (1 - p).  Its bits come from torch's RNG, which a fused kernel
cannot reproduce; the fused path instead draws them from a counter-based
generator, Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random
numbers: as easy as 1, 2, 3", SC'11), so that the forward and the backward
regenerate the same mask from a seed.  Definition (also in the kernels'
header soupsuck_amd/csrc/philox.h):

    element e = row * cols + col of X [rows, cols]
    key = (seed mod 2^32, seed div 2^32); counter = (e div 4 mod 2^32, e div 4 div 2^32, 0, 0)
    keep(e) = word (e mod 4) of Philox4x32-10(counter, key) < floor((1 - p) 2^32)
    dropped = fp32(x) * fp32(1 / (1 - p)) where kept, else 0

Pinned by tests/test_oracle_philox.py: the published Philox4x32-10 known-answer
vectors (Random123 kat_vectors), the keep rate against the binomial bound, and
bit-exact agreement with the GPU mask (ss_dropout_mask).
"""

import numpy as np

M0, M1 = np.uint64(0xD2511F53), np.uint64(0xCD9E8D57)
W0, W1 = 0x9E3779B9, 0xBB67AE85
MASK32 = np.uint64(0xFFFFFFFF)


def philox4x32_10(ctr, key):
    """Philox4x32-10 of counters ``ctr`` [n, 4] uint32 under key (k0, k1) -> [n, 4] uint32."""
    c = [np.asarray(ctr, dtype=np.uint64)[:, i].copy() for i in range(4)]
    k0, k1 = int(key[0]) & 0xFFFFFFFF, int(key[1]) & 0xFFFFFFFF
    for r in range(10):
        if r:
            k0 = (k0 + W0) & 0xFFFFFFFF
            k1 = (k1 + W1) & 0xFFFFFFFF
        p0 = M0 * c[0]
        p1 = M1 * c[2]
        c = [((p1 >> np.uint64(32)) ^ c[1] ^ np.uint64(k0)) & MASK32, p1 & MASK32,
             ((p0 >> np.uint64(32)) ^ c[3] ^ np.uint64(k1)) & MASK32, p0 & MASK32]
    return np.stack(c, axis=1).astype(np.uint32)


def threshold(p):
    """floor((1 - p) * 2^32) for p in (0, 1), as the host computes it (double), saturated at
    2^32 - 1 (a p below 2^-32 rounds 1 - p to 1)."""
    return min(int(np.floor((1.0 - float(np.float32(p))) * 4294967296.0)), 0xFFFFFFFF)


def inverse_keep(p):
    """fp32(1 / (1 - p)) with p the fp32 argument the C ABI receives."""
    return np.float32(1.0 / (1.0 - float(np.float32(p))))


def keep_mask(seed, p, rows, cols):
    """bool [rows, cols]: the elements the fused dropout keeps."""
    n = rows * cols
    groups = (n + 3) // 4
    g = np.arange(groups, dtype=np.uint64)
    ctr = np.zeros((groups, 4), dtype=np.uint64)
    ctr[:, 0] = g & MASK32
    ctr[:, 1] = g >> np.uint64(32)
    words = philox4x32_10(ctr, (seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF))
    return (words.reshape(-1)[:n] < threshold(p)).reshape(rows, cols)


def dropped(x, keep, p):
    """fp32 dropped activations: fp32(x) * fp32(1 / (1 - p)) where kept, else 0."""
    x = np.asarray(x, dtype=np.float32)
    return np.where(keep, x * inverse_keep(p), np.float32(0.0)).astype(np.float32)
