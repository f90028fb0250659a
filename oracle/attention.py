"""Causal attention over packed rows -- test infrastructure only.

Reference semantics (solution/unpad.py:359-410): the packed token axis holds
rows of lengths L_r back to back; a query at position t of row r attends to
the keys of row r at positions <= t, with softmax(scale . q . k) and GQA (kv
head = q head // (Hq / Hk)); nothing crosses a row boundary.

Restated in float64 numpy: q [T, Hq, D], k / v [T, Hk, D] (any float dtype),
lengths a sequence of row lengths summing to T.  Returns o [T, Hq, D] and the
natural-log log-sum-exp [Hq, T]; the backward returns dq, dk, dv for an
upstream do [T, Hq, D] by the closed forms dV = P^T dO, dP = dO V^T,
dS = P (dP - rowsum(dO o O)), dQ = scale dS K, dK = scale dS^T Q (summed over
the q heads of a kv head).

Pins (tests/test_oracle_attention.py): torch's scaled_dot_product_attention
(is_causal=True, float64, CPU) per row with the KV heads repeated, and its
autograd for the gradients (a library routine); a row of length 1 returns its
value row; equal scores give the running mean of the value rows; a planted
mistake (no causal mask) fails the torch comparison.
"""

import numpy as np


def _rows(lengths):
    start = 0
    for n in lengths:
        yield start, int(n)
        start += int(n)


def forward(q, k, v, lengths, scale):
    q, k, v = (np.asarray(x, np.float64) for x in (q, k, v))
    t, hq, d = q.shape
    hk = k.shape[1]
    group = hq // hk
    o = np.zeros((t, hq, d))
    lse = np.zeros((hq, t))
    for start, n in _rows(lengths):
        mask = np.tril(np.ones((n, n), bool))
        for h in range(hq):
            qs = q[start:start + n, h]
            ks = k[start:start + n, h // group]
            vs = v[start:start + n, h // group]
            s = np.where(mask, qs @ ks.T * scale, -np.inf)
            m = s.max(axis=1, keepdims=True)
            e = np.exp(s - m)
            l = e.sum(axis=1, keepdims=True)
            o[start:start + n, h] = (e / l) @ vs
            lse[h, start:start + n] = (m + np.log(l))[:, 0]
    return o, lse


def backward(q, k, v, do, lengths, scale):
    q, k, v, do = (np.asarray(x, np.float64) for x in (q, k, v, do))
    t, hq, d = q.shape
    hk = k.shape[1]
    group = hq // hk
    dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    for start, n in _rows(lengths):
        mask = np.tril(np.ones((n, n), bool))
        for h in range(hq):
            kvh = h // group
            rows = slice(start, start + n)
            qs, ks, vs, dos = q[rows, h], k[rows, kvh], v[rows, kvh], do[rows, h]
            s = np.where(mask, qs @ ks.T * scale, -np.inf)
            p = np.exp(s - s.max(axis=1, keepdims=True))
            p /= p.sum(axis=1, keepdims=True)
            o = p @ vs
            dv[rows, kvh] += p.T @ dos
            dp = dos @ vs.T
            ds = p * (dp - (dos * o).sum(axis=1, keepdims=True))
            dq[rows, h] = scale * ds @ ks
            dk[rows, kvh] += scale * ds.T @ qs
    return dq, dk, dv
