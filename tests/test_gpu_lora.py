"""GPU parity of the LoRA epilogue (bit-exact) and the QLoRA projection (toleranced).

Epilogue cases mirror solution/tests/test_lora.py:15-49 (every base/adapter
dtype pair, both cast modes, rtol = atol = 0; the rounded product must cancel
to exactly zero).  The projection forward is compared with the oracle's
autocast composition (fp16 after each GEMM) and the backward with the float64
ideal gradients, within a relative-norm bound of 1e-2.
"""

import numpy as np
import pytest
import torch

from oracle import lora as olora
from oracle import nf4 as onf4
from soupsuck_amd.kernels.lora_epilogue import lora_epilogue
from soupsuck_amd.lora import qlora_projection
from tests.gpu_util import bits, device_state, np16, random_weight, rel_norm

pytestmark = pytest.mark.gpu

NP = {torch.float16: np.float16, torch.float32: np.float32}


@pytest.mark.parametrize("base_dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("adapter_dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("cast_to_result", [False, True])
def test_epilogue_bit_exact(device, base_dtype, adapter_dtype, cast_to_result):
    rng = np.random.default_rng(175)
    base = rng.standard_normal((3, 7, 79)).astype(NP[base_dtype])
    adapter = rng.standard_normal((3, 7, 79)).astype(NP[adapter_dtype])
    bt = torch.from_numpy(base).to(device).requires_grad_()
    at = torch.from_numpy(adapter).to(device).requires_grad_()
    out = lora_epilogue(bt, at, 1.3, cast_to_result=cast_to_result)
    expected = olora.epilogue_forward(base, adapter, 1.3, cast_to_result)
    assert out.dtype == torch.from_numpy(expected).dtype
    np.testing.assert_array_equal(np16(out), expected)
    grad = rng.standard_normal(out.shape).astype(expected.dtype)
    out.backward(torch.from_numpy(grad).to(device))
    d_r, d_a = olora.epilogue_backward(grad, NP[base_dtype], NP[adapter_dtype], 1.3)
    np.testing.assert_array_equal(np16(bt.grad), d_r)
    np.testing.assert_array_equal(np16(at.grad), d_a)


def test_epilogue_rounded_product_cancels(device):
    adapter = torch.linspace(-2, 2, 2049, device=device, dtype=torch.float16)
    result = -(adapter * 1.3)
    assert torch.count_nonzero(lora_epilogue(result, adapter, 1.3)).item() == 0


@pytest.mark.parametrize("t,n,k,bias", [(96, 256, 1536, True), (200, 1536, 1536, False),
                                        (200, 512, 8960, False),
                                        (37, 8960, 1536, False), (64, 1536, 8960, False),
                                        (300, 256, 1536, True), (990, 8960, 1536, False),
                                        (990, 1536, 8960, False),
                                        # configs[1] q (bias), k / v (bias) and o at T = 990
                                        (990, 1536, 1536, True), (990, 256, 1536, True),
                                        (990, 1536, 1536, False), (2048, 8960, 256, True),
                                        (16, 8960, 1536, True), (29, 1000, 3584, False),
                                        # 592 tiles of 256x256 in the forward (LoRA
                                        # epilogue) and in the dX product (rank-16)
                                        (2048, 18944, 128, True),
                                        (2048, 128, 18944, False)])
def test_qlora_projection_matches_oracle(device, t, n, k, bias):
    rng = np.random.default_rng(t + n)
    state = onf4.quantize_nested(random_weight(n, k, seed=3))
    w = state.decode()
    packed, qs = device_state(state, device)
    x = rng.standard_normal((t, k)).astype(np.float16)
    a = ((rng.random((16, k)) * 2 - 1) / np.sqrt(k)).astype(np.float16)
    b = (rng.standard_normal((n, 16)) * 0.01).astype(np.float16)
    bvec = (rng.standard_normal(n) * 0.02).astype(np.float16) if bias else None
    g = (rng.standard_normal((t, n)) * 0.01).astype(np.float16)
    xt = torch.from_numpy(x).to(device).requires_grad_()
    at = torch.from_numpy(a).to(device).requires_grad_()
    bt = torch.from_numpy(b).to(device).requires_grad_()
    out = qlora_projection(xt, at, bt, packed, qs,
                           torch.from_numpy(bvec).to(device) if bias else None, scaling=2.0)
    # forward: oracle autocast composition
    base = (x.astype(np.float64) @ w.astype(np.float64).T
            + (bvec.astype(np.float64) if bias else 0)).astype(np.float16)
    _, lo = olora.branch_forward(x, a, b)
    expected = olora.epilogue_forward(base, lo, 2.0)
    got = np16(out)
    assert np.all(np.isfinite(got))
    np.testing.assert_allclose(got.astype(np.float64), expected.astype(np.float64),
                               rtol=2e-3, atol=2e-3)
    ideal = olora.ideal_projection(x, w, bvec, a, b, 2.0)
    assert rel_norm(got, ideal) < 1e-3
    out.backward(torch.from_numpy(g).to(device))
    dx, da, db = olora.ideal_projection_backward(g, x, w, a, b, 2.0)
    assert rel_norm(np16(xt.grad), dx) < 1e-2
    assert rel_norm(np16(at.grad), da) < 1e-2
    assert rel_norm(np16(bt.grad), db) < 1e-2


@pytest.mark.parametrize("m,k", [(37, 100), (990, 1536), (990, 8960), (1, 64), (130, 16),
                                 (16, 8960),     # few row blocks, long K: split form
                                 (500, 5000)])   # 32 row blocks: one launch, 16 waves
@pytest.mark.parametrize("w_kr", [False, True])
@pytest.mark.parametrize("scale", [None, 2.0, 1.3])
def test_rank_project_matches_numpy(device, m, k, w_kr, scale):
    from soupsuck_amd.lora import project16

    rng = np.random.default_rng(m + k)
    a = rng.standard_normal((m, k)).astype(np.float16)
    w = (rng.standard_normal((k, 16) if w_kr else (16, k)) * 0.1).astype(np.float16)
    out = project16(torch.from_numpy(a).to(device), torch.from_numpy(w).to(device), w_kr, scale)
    a_eff = a if scale is None else (a.astype(np.float32) * np.float32(scale)).astype(np.float16)
    wm = w.astype(np.float64) if w_kr else w.astype(np.float64).T
    expected = a_eff.astype(np.float64) @ wm
    np.testing.assert_allclose(np16(out).astype(np.float64), expected, rtol=2e-3, atol=2e-3)


@pytest.mark.parametrize("t,n", [(37, 100), (990, 1536), (990, 8960), (1, 64), (300, 16),
                                 (6000, 64),     # one column block, long T: split form
                                 (5000, 2048),   # 32 column blocks: one launch
                                 (0, 64)])       # empty reduction: zeros
@pytest.mark.parametrize("transpose", [False, True])
@pytest.mark.parametrize("scale", [None, 2.0])
def test_rank_grad_matches_numpy(device, t, n, transpose, scale):
    from soupsuck_amd.lora import grad16

    rng = np.random.default_rng(t * 7 + n)
    p = (rng.standard_normal((t, 16)) * 0.3).astype(np.float16)
    q = rng.standard_normal((t, n)).astype(np.float16)
    out = grad16(torch.from_numpy(p).to(device), torch.from_numpy(q).to(device), transpose, scale)
    q_eff = q if scale is None else (q.astype(np.float32) * np.float32(scale)).astype(np.float16)
    expected = p.astype(np.float64).T @ q_eff.astype(np.float64)
    if transpose:
        expected = expected.T
    np.testing.assert_allclose(np16(out).astype(np.float64), expected, rtol=2e-3,
                               atol=2e-3 * max(1.0, np.sqrt(t)))


def test_rank_ops_deterministic_and_leave_counters_zero(device):
    """Split reductions finished by the last workgroup to arrive: repeated calls
    give the same bits, and the workspace's arrival counters are zero again
    after every call (the contract that lets one zero-filled workspace serve
    all calls on a stream)."""
    from soupsuck_amd import lora

    rng = np.random.default_rng(12)
    a = torch.from_numpy(rng.standard_normal((990, 8960)).astype(np.float16)).to(device)
    w = torch.from_numpy((rng.standard_normal((8960, 16)) * 0.1).astype(np.float16)).to(device)
    z = torch.from_numpy((rng.standard_normal((990, 16)) * 0.3).astype(np.float16)).to(device)
    first_p = lora.project16(a, w, True, 2.0)
    first_g = lora.grad16(z, a, True, 2.0)
    for _ in range(3):
        assert torch.equal(lora.project16(a, w, True, 2.0), first_p)
        assert torch.equal(lora.grad16(z, a, True, 2.0), first_g)
    torch.cuda.synchronize()
    ws = lora._RANK_WORKSPACE[(device.index if device.index is not None else 0,
                               torch.cuda.current_stream(device).cuda_stream)]
    counters = ws[:256 * 1024].view(torch.int32)  # the fixed counter area
    assert int(torch.count_nonzero(counters)) == 0


def test_rank_ops_on_concurrent_streams(device):
    """Rank-16 ops queued on two side streams at once (each stream has its own
    counter workspace) give the single-stream results, and every workspace's
    counters are zero afterwards."""
    from soupsuck_amd import lora

    rng = np.random.default_rng(13)
    inputs = [torch.from_numpy(rng.standard_normal((990, 8960)).astype(np.float16)).to(device)
              for _ in range(2)]
    w = torch.from_numpy((rng.standard_normal((8960, 16)) * 0.1).astype(np.float16)).to(device)
    z = torch.from_numpy((rng.standard_normal((990, 16)) * 0.3).astype(np.float16)).to(device)
    ref = [(lora.project16(a, w, True, 2.0), lora.grad16(z, a, True, 2.0)) for a in inputs]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(device) for _ in inputs]
    results = [[], []]
    for _ in range(4):
        for i, (a, st) in enumerate(zip(inputs, streams)):
            with torch.cuda.stream(st):
                results[i].append((lora.project16(a, w, True, 2.0), lora.grad16(z, a, True, 2.0)))
    torch.cuda.synchronize()
    for i in range(2):
        for p, g in results[i]:
            assert torch.equal(p, ref[i][0]) and torch.equal(g, ref[i][1])
    for key, ws in lora._RANK_WORKSPACE.items():
        assert int(torch.count_nonzero(ws[:256 * 1024].view(torch.int32))) == 0, key


def test_general_path_matches_fused_and_dropout_runs(device):
    from soupsuck_amd.lora import _QLoRAProjection

    rng = np.random.default_rng(5)
    t, n, k = 64, 256, 1536
    state = onf4.quantize_nested(random_weight(n, k, seed=4))
    packed, qs = device_state(state, device)
    x = torch.from_numpy(rng.standard_normal((t, k)).astype(np.float16)).to(device)
    a = torch.from_numpy(((rng.random((16, k)) * 2 - 1) / 40).astype(np.float16)).to(device)
    b = torch.from_numpy((rng.standard_normal((n, 16)) * 0.01).astype(np.float16)).to(device)
    g = torch.from_numpy((rng.standard_normal((t, n)) * 0.01).astype(np.float16)).to(device)
    outs, grads = [], []
    for general in (False, True):
        xs, as_, bs = (v.clone().requires_grad_() for v in (x, a, b))
        if general:
            out = _QLoRAProjection.apply(xs, as_, bs, packed, qs, None, 2.0, 0.0, True)
        else:
            out = qlora_projection(xs, as_, bs, packed, qs, None, 2.0)
        out.backward(g)
        outs.append(np16(out).astype(np.float64))
        grads.append([np16(v.grad).astype(np.float64) for v in (xs, as_, bs)])
    np.testing.assert_allclose(outs[0], outs[1], rtol=2e-3, atol=2e-3)
    for g0, g1 in zip(*grads):
        assert rel_norm(g0, g1) < 1e-2
    xs = x.clone().requires_grad_()
    out = qlora_projection(xs, a.clone().requires_grad_(), b.clone().requires_grad_(), packed, qs,
                           None, 2.0, dropout_p=0.1)
    out.backward(g)
    assert torch.isfinite(out).all() and torch.isfinite(xs.grad).all()
