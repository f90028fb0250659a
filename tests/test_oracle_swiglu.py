"""CPU pins of the SwiGLU oracle (solution/kernels/swiglu_fused.py:20-46).

Checked against: closed forms at g = 0 and in both limits; a central finite
difference of the float64 forward; torch.nn.functional.silu and its autograd
(CPU, float64), written independently of the oracle's formula; and the fp32
operation order against the float64 value.  A planted mistake (the slope
without its act*(1-p) term) must fail the finite-difference pin.
"""

import numpy as np
import pytest
import torch

from oracle import swiglu as osw


def _inputs(shape, seed, scale=3.0):
    rng = np.random.default_rng(seed)
    g = (rng.standard_normal(shape) * scale).astype(np.float16)
    u = rng.standard_normal(shape).astype(np.float16)
    da = rng.standard_normal(shape).astype(np.float16)
    return g, u, da


def test_closed_forms_at_zero_and_limits():
    g = np.array([0.0, 0.0, 60.0, -60.0, 1e4, -1e4])
    u = np.array([1.0, -3.0, 2.0, 2.0, 1.0, 1.0])
    a = osw.swiglu_forward_exact(g, u, np.float64)
    assert a[0] == 0.0 and a[1] == 0.0
    assert a[2] == pytest.approx(120.0, rel=1e-15)
    assert abs(a[3]) < 1e-20 and abs(a[5]) == 0.0
    assert a[4] == 1e4
    dg, du = osw.swiglu_backward_exact(g, np.ones_like(g), np.ones_like(g), np.float64, np.float64)
    assert dg[0] == 0.5 and du[0] == 0.0            # slope(0) = p(0) = 1/2, act(0) = 0
    assert dg[2] == pytest.approx(1.0, rel=1e-12)   # slope -> 1
    assert abs(dg[3]) < 1e-20                        # slope -> 0
    assert du[2] == pytest.approx(60.0, rel=1e-15)


def _finite_difference(g, u, da, h=1e-6):
    g, u, da = (np.asarray(x, np.float64) for x in (g, u, da))
    f = lambda gg, uu: osw.swiglu_forward_exact(gg, uu, np.float64)  # noqa: E731
    dg = da * (f(g + h, u) - f(g - h, u)) / (2 * h)
    du = da * (f(g, u + h) - f(g, u - h)) / (2 * h)
    return dg, du


def test_backward_equals_finite_difference():
    g, u, da = _inputs((7, 33), 1)
    dg, du = osw.swiglu_backward_exact(g, u, da, np.float64, np.float64)
    fdg, fdu = _finite_difference(g, u, da)
    np.testing.assert_allclose(dg, fdg, rtol=1e-6, atol=1e-8)
    np.testing.assert_allclose(du, fdu, rtol=1e-6, atol=1e-8)


def test_planted_slope_mistake_fails_the_pin():
    g, u, da = _inputs((5, 17), 2)
    gf, uf, daf = (x.astype(np.float64) for x in (g, u, da))
    p = 1.0 / (1.0 + np.exp(-gf))
    wrong_dg = daf * uf * p                  # dropped act*(1-p)
    fdg, _ = _finite_difference(g, u, da)
    assert not np.allclose(wrong_dg, fdg, rtol=1e-3, atol=1e-6)


def test_matches_torch_silu_autograd_float64():
    g, u, da = _inputs((9, 65), 3)
    tg = torch.from_numpy(g.astype(np.float64)).requires_grad_()
    tu = torch.from_numpy(u.astype(np.float64)).requires_grad_()
    out = torch.nn.functional.silu(tg) * tu
    out.backward(torch.from_numpy(da.astype(np.float64)))
    a = osw.swiglu_forward_exact(g, u, np.float64)
    dg, du = osw.swiglu_backward_exact(g, u, da, np.float64, np.float64)
    np.testing.assert_allclose(a, out.detach().numpy(), rtol=1e-13, atol=1e-15)
    np.testing.assert_allclose(dg, tg.grad.numpy(), rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(du, tu.grad.numpy(), rtol=1e-13, atol=1e-15)


def test_fp32_order_within_an_fp16_ulp_of_exact():
    g, u, da = _inputs((64, 257), 4)
    a32 = osw.swiglu_forward_fp32(g, u, np.float32)
    a64 = osw.swiglu_forward_exact(g, u, np.float64)
    np.testing.assert_allclose(a32, a64, rtol=1e-5, atol=1e-30)
    a16 = osw.swiglu_forward_fp32(g, u).astype(np.float64)
    ulp = np.spacing(np.abs(a64).astype(np.float16)).astype(np.float64)
    assert (np.abs(a16 - a64) <= ulp).all()
    dg32, du32 = osw.swiglu_backward_fp32(g, u, da, np.float32, np.float32)
    dg64, du64 = osw.swiglu_backward_exact(g, u, da, np.float64, np.float64)
    # slope = p + act (1 - p) cancels near g = -1.28 (slope = 0): bound the fp32
    # error by the size of the summands, not of the result.
    gf, uf, daf = (x.astype(np.float64) for x in (g, u, da))
    p = 1.0 / (1.0 + np.exp(-gf))
    terms = np.abs(daf * uf) * (p + np.abs(gf * p * (1.0 - p)))
    assert (np.abs(dg32 - dg64) <= 1e-5 * np.abs(dg64) + 8 * 2.0 ** -24 * terms).all()
    np.testing.assert_allclose(du32, du64, rtol=1e-5, atol=1e-30)
