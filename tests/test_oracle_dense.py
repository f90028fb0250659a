"""CPU pins of the GEMM, LoRA, add-RMSNorm, unpad and cross-entropy oracles.

Each oracle is checked against something other than its own formula:
  gemm      brute-force triple loop; the EXP-002 gate rejects planted mistakes
            (transposed weight, dropped bias, an output off by one fp16 ulp
            everywhere is still accepted -- the gate's intended slack);
  lora      the reference's cancel-to-zero known answer
            (solution/tests/test_lora.py:41-49) fails a fused multiply-add;
            ideal gradients equal central finite differences;
  rmsnorm   backward equals torch.autograd (CPU, float64) of the forward
            written independently; rms(q) == 1 invariant;
  unpad     the reference's right-padding table and index example
            (solution/tests/test_unpad.py:23-37,183-184); round trips;
  ce        known answers of solution/tests/test_cross_entropy.py:331-360;
            chunked online statistics == one-shot logsumexp for any chunk;
            gradients equal torch.autograd (CPU, float64).
"""

import math

import numpy as np
import pytest
import torch

from oracle import cross_entropy as ce
from oracle import gemm, lora, rmsnorm, unpad


# ------------------------------------------------------------------ gemm ---

def test_linear_matches_brute_force():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((3, 5)).astype(np.float16)
    w = rng.standard_normal((4, 5)).astype(np.float16)
    b = rng.standard_normal(4).astype(np.float16)
    np.testing.assert_allclose(gemm.linear(x, w, b), gemm.brute_force_linear(x, w, b), rtol=1e-12)
    np.testing.assert_allclose(gemm.linear_dx(x[:, :4], w), x[:, :4].astype(np.float64) @ w,
                               rtol=1e-12)


def test_gate_rejects_planted_mistakes():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((32, 64)).astype(np.float16)
    w = (rng.standard_normal((48, 64)) * 0.1).astype(np.float16)
    b = rng.standard_normal(48).astype(np.float16)
    good = gemm.linear(x, w, b)
    assert gemm.gate(good.astype(np.float16), good)[0]
    ws = (rng.standard_normal((64, 64)) * 0.1).astype(np.float16)
    assert not gemm.gate(gemm.linear(x, ws.T), gemm.linear(x, ws))[0]   # transposed operand
    assert not gemm.gate(gemm.linear(x, w), good)[0]                       # dropped bias
    assert not gemm.gate(-good, good)[0]                                    # wrong sign


def test_exact_weight_decode_rounds_to_the_fp16_decode():
    from oracle import nf4

    rng = np.random.default_rng(2)
    state = nf4.quantize_nested((rng.standard_normal((40, 640)) * 0.02).astype(np.float16))
    exact = state.decode_exact()
    dec = state.decode()
    np.testing.assert_array_equal(exact.astype(np.float32).astype(np.float16).view(np.uint16),
                                  dec.view(np.uint16))
    half_ulp = np.spacing(np.abs(dec)).astype(np.float64) / 2
    assert np.all(np.abs(exact - dec.astype(np.float64)) <= half_ulp * (1 + 2 ** -10))


def test_no_worse_gate_accepts_reference_and_rejects_planted_mistakes():
    from oracle import nf4

    rng = np.random.default_rng(3)
    state = nf4.quantize_nested((rng.standard_normal((96, 4096)) * 0.02).astype(np.float16))
    x = rng.standard_normal((24, 4096)).astype(np.float16)
    exact = gemm.linear(x, state.decode_exact())
    ref = gemm.linear(x, state.decode()).astype(np.float16)
    assert gemm.no_worse_than_reference(ref, exact, ref)[0]
    # post-scaled blocks (sum of x * fp16(NF4) per 64-block, times the scale): one
    # rounding per weight like the reference, so within the slack
    n = state.n
    nib = nf4.unpack_nibbles(state.packed, n).reshape(96, 64, 64)
    scale = nf4.blockwise_absmax(state.qabs, state.absmax2, state.code2, state.offset,
                                 n // 64).astype(np.float64).reshape(96, 64)
    v16 = nf4.NF4_VALUES.astype(np.float16).astype(np.float64)[nib]
    post = np.einsum("tbk,nbk->tnb", x.astype(np.float64).reshape(24, 64, 64), v16)
    post = (post * scale[None]).sum(-1).astype(np.float16)
    assert gemm.no_worse_than_reference(post, exact, ref)[0]
    dropped = gemm.linear(x[:, 64:], state.decode_exact()[:, 64:]).astype(np.float16)
    assert not gemm.no_worse_than_reference(dropped, exact, ref)[0]       # one block dropped
    coarse = exact.astype(np.float16).astype(np.float32)
    coarse = (np.round(coarse * 64) / 64).astype(np.float16)
    assert not gemm.no_worse_than_reference(coarse, exact, ref)[0]       # 6-bit output rounding
    assert not gemm.no_worse_than_reference(-ref, exact, ref)[0]          # wrong sign


# ------------------------------------------------------------------ lora ---

def test_epilogue_rounded_product_cancels_to_zero():
    adapter = np.linspace(-2, 2, 2049).astype(np.float16)
    s = 1.3
    base = (adapter.astype(np.float32) * np.float32(s)).astype(np.float16)
    out = lora.epilogue_forward(-base, adapter, s)
    assert out.dtype == np.float16 and np.count_nonzero(out) == 0
    # a fused multiply-add (no intermediate rounding) does NOT cancel
    fused = (-base.astype(np.float64) + adapter.astype(np.float64) * s).astype(np.float16)
    assert np.count_nonzero(fused) > 0


def test_epilogue_dtypes():
    a = np.ones(4, np.float32)
    assert lora.epilogue_forward(np.ones(4, np.float16), a, 2.0).dtype == np.float32
    assert lora.epilogue_forward(np.ones(4, np.float16), a, 2.0, True).dtype == np.float16
    d_r, d_a = lora.epilogue_backward(np.full(3, 1.0 / 3, np.float32), np.float16, np.float16, 2.0)
    assert d_r.dtype == d_a.dtype == np.float16
    assert d_a[0] == np.float16(np.float32(np.float16(1.0 / 3)) * 2)


def test_ideal_projection_gradients_match_finite_differences():
    rng = np.random.default_rng(2)
    t, k, n, r, s = 3, 5, 4, 2, 2.0
    x, w = rng.standard_normal((t, k)), rng.standard_normal((n, k))
    a, b, g = rng.standard_normal((r, k)), rng.standard_normal((n, r)), rng.standard_normal((t, n))
    dx, da, db = lora.ideal_projection_backward(g, x, w, a, b, s)

    def f(x_, a_, b_):
        return float((lora.ideal_projection(x_, w, None, a_, b_, s) * g).sum())

    eps = 1e-6
    for arr, grad, fn in ((x, dx, lambda v: f(v, a, b)), (a, da, lambda v: f(x, v, b)),
                          (b, db, lambda v: f(x, a, v))):
        num = np.zeros_like(arr)
        for idx in np.ndindex(arr.shape):
            p, m = arr.copy(), arr.copy()
            p[idx] += eps
            m[idx] -= eps
            num[idx] = (fn(p) - fn(m)) / (2 * eps)
        np.testing.assert_allclose(grad, num, rtol=1e-6, atol=1e-6)


# --------------------------------------------------------------- rmsnorm ---

def test_rmsnorm_backward_matches_torch_autograd():
    rng = np.random.default_rng(3)
    rows, h, eps = 6, 40, 1e-6
    r = rng.standard_normal((rows, h))
    d = rng.standard_normal((rows, h))
    w = 1 + 0.1 * rng.standard_normal(h)
    gs = rng.standard_normal((rows, h))
    gy = rng.standard_normal((rows, h))
    rt, dt, wt = (torch.tensor(v, requires_grad=True) for v in (r, d, w))
    st = rt + dt
    yt = wt * (st * torch.rsqrt(st.pow(2).mean(-1, keepdim=True) + eps))
    torch.autograd.backward([st, yt], [torch.tensor(gs), torch.tensor(gy)])
    s, y, rstd = rmsnorm.add_rmsnorm_forward(r, d, w, eps)
    np.testing.assert_allclose(y, yt.detach().numpy(), rtol=1e-12)
    dr, dd, dg = rmsnorm.add_rmsnorm_backward(gs, gy, s, w, rstd, np.float64, np.float64,
                                              np.float64)
    np.testing.assert_allclose(dr, rt.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dd, dt.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dg, wt.grad.numpy(), rtol=1e-10, atol=1e-12)
    q = y / w
    np.testing.assert_allclose(np.sqrt((q ** 2).mean(-1)), 1.0, rtol=1e-6)


def test_rmsnorm_dtype_promotion():
    r16 = np.ones((2, 8), np.float16)
    s, y, _ = rmsnorm.add_rmsnorm_forward(r16, r16, np.ones(8, np.float32), 1e-6)
    assert s.dtype == np.float16 and y.dtype == np.float32
    _, y16, _ = rmsnorm.add_rmsnorm_forward(r16, r16, np.ones(8, np.float32), 1e-6, True)
    assert y16.dtype == np.float16


# ----------------------------------------------------------------- unpad ---

@pytest.mark.parametrize("rows,expected", [
    ([[1, 1, 1], [1, 0, 0]], (3, 1)), ([[1], [1]], (1, 1)), ([[1, 1], [1, 1]], (2, 2)),
    ([[True, False]], (1,)), ([[0, 1]], None), ([[1, 0, 1]], None), ([[0, 0]], None),
    ([[1, 2]], None), ([[1], [1, 0]], None), ([], None), ([[]], None),
])
def test_right_padding_table(rows, expected):
    assert unpad.right_padding_lengths(rows) == expected


def test_indices_example_and_round_trip():
    assert unpad.indices_from_lengths((1, 3), 3).tolist() == [0, 3, 4, 5]
    rng = np.random.default_rng(4)
    lengths = (5, 1, 7)
    x = rng.standard_normal((3, 7, 4)).astype(np.float16)
    idx = unpad.indices_from_lengths(lengths, 7)
    packed = unpad.pack(x, idx)
    assert packed.shape == (13, 4)
    back = unpad.scatter(packed, idx, 3, 7)
    mask = (np.arange(7)[None, :] < np.array(lengths)[:, None])[..., None]
    np.testing.assert_array_equal(back, np.where(mask, x, 0))
    np.testing.assert_array_equal(unpad.pack(back, idx), packed)


# -------------------------------------------------------------------- ce ---

def test_ce_tied_logits_known_answer():
    h = np.ones((1, 2), np.float16)
    w = np.array([[1.0, 0.0001], [1.0, 0.0002]], np.float16)
    loss, entropy, best, lse = ce.forward(h, w, np.array([1]))
    assert best[0] == 0
    assert loss[0] == pytest.approx(math.log(2), abs=1e-12)
    assert entropy[0] == pytest.approx(math.log(2), abs=1e-12)
    assert lse[0] == pytest.approx(math.log(2) + 1, abs=1e-12)


def test_ce_zero_weight_known_answer():
    rng = np.random.default_rng(5)
    h = rng.standard_normal((7, 16)).astype(np.float16)
    w = np.zeros((4103, 16), np.float16)
    t = rng.integers(0, 4103, 7)
    loss, entropy, best, lse = ce.forward(h, w, t, chunk=1000)
    np.testing.assert_allclose(entropy, math.log(4103), rtol=1e-12)
    assert np.all(best == 0)
    dx, dw = ce.backward(h, w, t, np.ones(7), lse)
    np.testing.assert_allclose(dx, 0, atol=1e-15)


@pytest.mark.parametrize("chunk", [1, 7, 256, 5000])
def test_ce_chunked_equals_one_shot(chunk):
    rng = np.random.default_rng(6)
    h = rng.standard_normal((9, 24)).astype(np.float16)
    w = (rng.standard_normal((1000, 24)) * 0.3).astype(np.float16)
    t = rng.integers(0, 1000, 9)
    t[::3] = -100
    got = ce.forward(h, w, t, chunk=chunk)
    ref = ce.forward_one_shot(h, w, t)
    for a, b in zip(got, ref):
        np.testing.assert_allclose(a, b, rtol=1e-12, atol=1e-12)


def test_ce_gradients_match_torch_autograd():
    """dz from torch's own cross_entropy backward at the fp16-rounded logits (the
    reference's straight-through cast convention), chained through both GEMMs."""
    rng = np.random.default_rng(7)
    h = rng.standard_normal((5, 12)).astype(np.float16)
    w = (rng.standard_normal((30, 12)) * 0.5).astype(np.float16)
    t = rng.integers(0, 30, 5)
    t[1] = -100
    g = rng.standard_normal(5)
    z16 = ce.logits_fp16(h, w).astype(np.float64)
    zt = torch.tensor(z16, requires_grad=True)
    losses = torch.nn.functional.cross_entropy(zt, torch.tensor(t), reduction="none",
                                               ignore_index=-100)
    (losses * torch.tensor(g)).sum().backward()
    dz = zt.grad.numpy()
    _, _, _, lse = ce.forward_one_shot(h, w, t)
    np.testing.assert_allclose(lse, torch.logsumexp(zt.detach(), -1).numpy(), rtol=1e-13)
    dx, dw = ce.backward(h, w, t, g, lse)
    np.testing.assert_allclose(dx, dz @ w.astype(np.float64), rtol=1e-10, atol=1e-13)
    np.testing.assert_allclose(dw, dz.T @ h.astype(np.float64), rtol=1e-10, atol=1e-13)
    assert np.all(dx[1] == 0)
