"""GPU parity of the SwiGLU kernels (ss_swiglu_fwd / ss_swiglu_bwd) against the oracle.

Bar (stated per dtype): an fp16 output is within one fp16 ulp of the float64
value of the same formula (oracle.swiglu.*_exact); an fp32 output is within a
relative 1e-5 of it.  dgate additionally gets the fp32 rounding slack of the
cancelling sum p + act (1 - p), 8 * 2^-24 * |da u| (p + |act (1 - p)|).
Cases follow the reference's use (solution/tests/test_mlp.py:63-89,
solution/tests/test_precompile.py:258,402-406): fp16 projection outputs,
fp32 outputs under autocast, fp16 saved gate/up with an fp32 upstream, 3-D
inputs, widths not a multiple of 8, strided and transposed views, and the
configs[1] MLP width (T = 990, I = 8960).
"""

import numpy as np
import pytest
import torch

from oracle import swiglu as osw
from soupsuck_amd.kernels.swiglu import swiglu, swiglu_fused_backward, swiglu_fused_forward

pytestmark = pytest.mark.gpu


def _host(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _inputs(shape, seed, device, dtype=torch.float16):
    gen = torch.Generator().manual_seed(seed)
    g = (torch.randn(shape, generator=gen) * 3).to(dtype)
    u = torch.randn(shape, generator=gen).to(dtype)
    da = torch.randn(shape, generator=gen).to(dtype)
    return g.to(device), u.to(device), da.to(device)


def _assert_close(dev, exact, slack=0.0):
    d = _host(dev)
    if dev.dtype == torch.float16:
        bound = np.spacing(np.abs(exact).astype(np.float16)).astype(np.float64)
    else:
        bound = 1e-5 * np.abs(exact)
    err = np.abs(d - exact) - bound - slack
    assert (err <= 0).all(), f"max excess {err.max():.3g} at {np.unravel_index(err.argmax(), err.shape)}"


def _dg_slack(g, u, da):
    g, u, da = _host(g), _host(u), _host(da)
    p = 1.0 / (1.0 + np.exp(-g))
    return 8 * 2.0 ** -24 * np.abs(da * u) * (p + np.abs(g * p * (1.0 - p)))


def _check(g, u, da, out, dg, du):
    gh, uh, dah = _host(g), _host(u), _host(da)
    _assert_close(out, osw.swiglu_forward_exact(gh, uh, np.float64))
    edg, edu = osw.swiglu_backward_exact(gh, uh, dah, np.float64, np.float64)
    _assert_close(dg, edg, _dg_slack(g, u, da))
    _assert_close(du, edu)


@pytest.mark.parametrize("shape", [(990, 8960), (2, 5, 1001), (3, 77, 64), (1, 8), (17, 3)])
def test_fp16_matches_oracle(device, shape):
    g, u, da = _inputs(shape, 11, device)
    out = swiglu_fused_forward(g, u)
    dg, du = swiglu_fused_backward(g, u, da)
    assert out.dtype == dg.dtype == du.dtype == torch.float16
    _check(g, u, da, out, dg, du)


def test_fp16_equals_fp32_operation_order_within_an_ulp(device):
    g, u, da = _inputs((64, 2048), 12, device)
    out = swiglu_fused_forward(g, u)
    ref = osw.swiglu_forward_fp32(g.cpu().numpy(), u.cpu().numpy()).astype(np.float64)
    diff = np.abs(_host(out) - ref)
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    assert (diff <= ulp).all()
    assert (diff == 0).mean() > 0.99


def test_fp32_projection_outputs(device):
    g, u, da = _inputs((4, 33, 256), 13, device, torch.float32)
    out = swiglu_fused_forward(g, u)
    dg, du = swiglu_fused_backward(g, u, da)
    assert out.dtype == dg.dtype == du.dtype == torch.float32
    _check(g, u, da, out, dg, du)


def test_fp16_saved_fp32_upstream_and_outputs(device):
    g, u, _ = _inputs((2, 77, 512), 14, device)
    da = torch.randn(g.shape, device=device, dtype=torch.float32)
    dg, du = swiglu_fused_backward(g, u, da, torch.float32, torch.float32)
    assert dg.dtype == du.dtype == torch.float32
    gh, uh, dah = _host(g), _host(u), _host(da)
    edg, edu = osw.swiglu_backward_exact(gh, uh, dah, np.float64, np.float64)
    _assert_close(dg, edg, _dg_slack(g, u, da))
    _assert_close(du, edu)


def test_strided_views_take_their_own_strides(device):
    # gate and up as halves of one [T, 2I] projection output (row stride 2I),
    # an output written into a column slice, and transposed (column-strided) views.
    t, i = 129, 520
    gen = torch.Generator().manual_seed(15)
    gu = (torch.randn((t, 2 * i), generator=gen) * 3).half().to(device)
    g, u = gu[:, :i], gu[:, i:]
    da = torch.randn((t, i), generator=gen).half().to(device)
    big = torch.zeros((t, i + 24), device=device, dtype=torch.float16)
    out = swiglu_fused_forward(g, u, out=big[:, 8:8 + i])
    assert out.data_ptr() == big[:, 8:].data_ptr()
    dg, du = swiglu_fused_backward(g, u, da)
    _check(g, u, da, out, dg, du)
    assert (big[:, :8] == 0).all() and (big[:, 8 + i:] == 0).all()
    gt, ut, dat = g.t(), u.t(), da.t()
    out_t = swiglu_fused_forward(gt, ut)
    dg_t, du_t = swiglu_fused_backward(gt, ut, dat)
    _check(gt, ut, dat, out_t, dg_t, du_t)


def test_empty_rows_are_a_no_op(device):
    g = torch.empty((0, 64), device=device, dtype=torch.float16)
    assert swiglu_fused_forward(g, g).shape == (0, 64)
    dg, du = swiglu_fused_backward(g, g, g)
    assert dg.shape == du.shape == (0, 64)


def test_rejects_mismatched_shapes_and_bf16(device):
    g = torch.zeros((4, 8), device=device, dtype=torch.float16)
    with pytest.raises(ValueError):
        swiglu_fused_forward(g, torch.zeros((4, 16), device=device, dtype=torch.float16))
    with pytest.raises(ValueError):
        swiglu_fused_forward(g.bfloat16(), g.bfloat16())


def test_autograd_matches_torch_float32(device):
    # solution/tests/test_mlp.py:12 tolerance, against eager silu(g) * u in fp32.
    g, u, _ = _inputs((2, 5, 1001), 16, device)
    g.requires_grad_()
    u.requires_grad_()
    out = swiglu(g, u)
    upstream = torch.randn_like(out)
    out.backward(upstream)
    rg = g.detach().float().requires_grad_()
    ru = u.detach().float().requires_grad_()
    ref = torch.nn.functional.silu(rg) * ru
    ref.backward(upstream.float())
    torch.testing.assert_close(out.float(), ref, rtol=2e-3, atol=2e-3)
    torch.testing.assert_close(g.grad.float(), rg.grad, rtol=2e-3, atol=2e-3)
    torch.testing.assert_close(u.grad.float(), ru.grad, rtol=2e-3, atol=2e-3)
