"""CPU pins of oracle/attention.py (packed causal attention, forward and backward).

torch's scaled_dot_product_attention (float64, CPU, is_causal=True) applied
row by row with the KV heads repeated -- a library routine, and its autograd
for the gradients -- must agree to rounding; closed forms: a row of length 1
returns its value row, and zero queries (equal scores) give the running mean
of the value rows; a planted mistake (no causal mask) must fail the comparison.
"""

import numpy as np
import pytest
import torch

from oracle import attention as oattn


def _inputs(lengths, hq, hk, d=16, seed=0):
    rng = np.random.default_rng(seed)
    t = sum(lengths)
    q = rng.standard_normal((t, hq, d))
    k = rng.standard_normal((t, hk, d))
    v = rng.standard_normal((t, hk, d))
    return q, k, v


def _torch_rows(q, k, v, lengths, scale, do=None):
    hq, hk = q.shape[1], k.shape[1]
    tq = torch.tensor(q, requires_grad=True)
    tk = torch.tensor(k, requires_grad=True)
    tv = torch.tensor(v, requires_grad=True)
    outs, start = [], 0
    for n in lengths:
        rows = slice(start, start + n)
        qq = tq[rows].transpose(0, 1)[None]
        kk = tk[rows].transpose(0, 1).repeat_interleave(hq // hk, 0)[None]
        vv = tv[rows].transpose(0, 1).repeat_interleave(hq // hk, 0)[None]
        o = torch.nn.functional.scaled_dot_product_attention(qq, kk, vv, is_causal=True,
                                                             scale=scale)
        outs.append(o[0].transpose(0, 1))
        start += n
    out = torch.cat(outs, 0)
    if do is not None:
        out.backward(torch.tensor(do))
        return out.detach().numpy(), tq.grad.numpy(), tk.grad.numpy(), tv.grad.numpy()
    return out.detach().numpy()


@pytest.mark.parametrize("lengths,hq,hk", [((5, 1, 9), 4, 2), ((12,), 6, 1), ((3, 7, 2, 8), 2, 2)])
def test_forward_and_backward_match_torch(lengths, hq, hk):
    q, k, v = _inputs(lengths, hq, hk)
    scale = 1 / np.sqrt(q.shape[-1])
    do = np.random.default_rng(1).standard_normal(q.shape)
    o, lse = oattn.forward(q, k, v, lengths, scale)
    ro, rdq, rdk, rdv = _torch_rows(q, k, v, lengths, scale, do)
    np.testing.assert_allclose(o, ro, rtol=1e-10, atol=1e-12)
    dq, dk, dv = oattn.backward(q, k, v, do, lengths, scale)
    np.testing.assert_allclose(dq, rdq, rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(dk, rdk, rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(dv, rdv, rtol=1e-9, atol=1e-11)
    # lse: the log of the softmax denominator of the scaled scores
    start = 0
    for n in lengths:
        for h in range(hq):
            s = q[start:start + n, h] @ k[start:start + n, h // (hq // hk)].T * scale
            s = np.where(np.tril(np.ones((n, n), bool)), s, -np.inf)
            np.testing.assert_allclose(lse[h, start:start + n],
                                       np.log(np.exp(s).sum(axis=1)), rtol=1e-12)
        start += n


def test_closed_forms():
    lengths = (1, 6)
    q, k, v = _inputs(lengths, 2, 1)
    o, _ = oattn.forward(q, k, v, lengths, 0.3)
    np.testing.assert_allclose(o[0, :, :], np.repeat(v[0, :1, :], 2, 0))
    o, _ = oattn.forward(np.zeros_like(q), k, v, lengths, 0.3)
    row = v[1:, 0, :]
    running = np.cumsum(row, 0) / np.arange(1, 7)[:, None]
    np.testing.assert_allclose(o[1:, 0, :], running, rtol=1e-12)


def test_missing_causal_mask_fails_the_pin():
    lengths = (6, 5)
    q, k, v = _inputs(lengths, 2, 2, seed=3)
    ro = _torch_rows(q, k, v, lengths, 0.25)
    # planted: full (non-causal) attention within each row
    bad = np.zeros_like(q)
    start = 0
    for n in lengths:
        for h in range(2):
            s = q[start:start + n, h] @ k[start:start + n, h].T * 0.25
            p = np.exp(s - s.max(1, keepdims=True))
            bad[start:start + n, h] = (p / p.sum(1, keepdims=True)) @ v[start:start + n, h]
        start += n
    assert not np.allclose(bad, ro, atol=1e-6)
