"""GPU parity of the NF4 GEMMs and the dense fp16 MFMA GEMM.

Bar (fixed before any GPU run; the reference's EXP-002 gate,
experiments/reports/EXP-002.md:60-76): assert_close(rtol=2e-3, atol=2e-3) on
the fp16 output against the float64 product of the bit-exact decoded weight
(oracle.gemm), finite output, relative L2 <= 1e-3.  Shapes: the reference's
EXP-002 table (W 1536x1536, 256x1536, 8960x1536, 1536x8960 at M = 800 and
2048), configs[0] (gate 8960x1536, X [1024, 1536]), small-T rows (1, 16, 128),
ragged sizes, the large-T decode-first path, and K % 64 != 0 (dense path).
"""

import numpy as np
import pytest
import torch

from oracle import gemm as ogemm
from oracle import nf4 as onf4
from soupsuck_amd import _lib
from soupsuck_amd.kernels.nf4_gemm import gemm_f16, nf4_dx_2d, nf4_forward_2d, nf4_matmul
from tests.gpu_util import device_state, np16, random_weight

pytestmark = pytest.mark.gpu

_CACHE = {}


def weight(n, k, seed=11):
    key = (n, k, seed)
    if key not in _CACHE:
        state = onf4.quantize_nested(random_weight(n, k, seed))
        _CACHE[key] = (state, state.decode())
    return _CACHE[key]


def x_of(t, k, seed, scale=1.0):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((t, k), dtype=np.float32) * scale).astype(np.float16)


def check(actual, expected, what):
    ok, max_abs, rel = ogemm.gate(np16(actual).astype(np.float64), expected)
    assert ok, f"{what}: max_abs={max_abs:.3e} rel_l2={rel:.3e}"


@pytest.mark.parametrize("t,n,k", [
    (1024, 8960, 1536),                                   # configs[0]
    (800, 1536, 1536), (800, 256, 1536), (800, 8960, 1536), (800, 1536, 8960),
    (2048, 256, 1536),
    (1, 1536, 1536), (16, 8960, 1536), (128, 256, 1536), (37, 320, 128), (130, 192, 64),
])
def test_forward_matches_oracle(device, t, n, k):
    state, w = weight(n, k)
    packed, qs = device_state(state, device)
    x = x_of(t, k, seed=t + n)
    bias = (np.random.default_rng(5).standard_normal(n) * 0.1).astype(np.float16)
    xt = torch.from_numpy(x).to(device)
    bt = torch.from_numpy(bias).to(device)
    y = nf4_matmul(xt, packed, qs, bias=bt)
    check(y, ogemm.linear(x, w, bias), f"fwd t={t} n={n} k={k}")
    y0 = nf4_matmul(xt.view(1, t, k), packed, qs)
    assert y0.shape == (1, t, n)
    check(y0[0], ogemm.linear(x, w), f"fwd nobias t={t}")


# The streaming T <= 32 forward (post-scaled MFMA on unscaled code values):
# one or two 16-row M tiles, ragged T and N, one stage (K = 256) up to several
# stage groups (K = 4608: 18 stages), few row tiles (many groups, tiles split
# between two workgroups) and many.
@pytest.mark.parametrize("t,n,k", [
    (1, 4000, 3584), (5, 200, 256), (16, 8960, 1536), (17, 1000, 3584), (32, 1536, 4608),
    (9, 64, 8960), (31, 2080, 1536),
])
def test_streaming_forward_small_t(device, t, n, k):
    state, w = weight(n, k)
    packed, qs = device_state(state, device)
    x = x_of(t, k, seed=7 * t + n)
    bias = (np.random.default_rng(6).standard_normal(n) * 0.1).astype(np.float16)
    xt = torch.from_numpy(x).to(device)
    y = nf4_matmul(xt, packed, qs, bias=torch.from_numpy(bias).to(device))
    check(y, ogemm.linear(x, w, bias), f"stream fwd t={t} n={n} k={k}")
    again = nf4_matmul(xt, packed, qs, bias=torch.from_numpy(bias).to(device))
    assert torch.equal(y, again), "streaming forward is not deterministic"


@pytest.mark.parametrize("t,n,k", [
    (1024, 8960, 1536), (800, 1536, 1536), (800, 256, 1536), (800, 1536, 8960),
    (1, 1536, 1536), (16, 8960, 1536), (37, 320, 128), (130, 192, 64),
])
def test_dx_matches_oracle(device, t, n, k):
    state, w = weight(n, k)
    packed, qs = device_state(state, device)
    dy = x_of(t, n, seed=3 * t + k)
    dx = nf4_matmul(torch.from_numpy(dy).to(device), packed, qs, transpose=True)
    check(dx, ogemm.linear_dx(dy, w), f"dx t={t} n={n} k={k}")


# Without scratch (NULL, 0 bytes) dX runs the fused kernel unsplit where it is
# taken (T = 200, 8960 dX columns) and the in-loop column decoder elsewhere;
# with the reported workspace it splits or decodes W^T first.  All match the
# oracle, accumulate included.
@pytest.mark.parametrize("t,n,k", [(200, 512, 1536), (200, 512, 8960), (130, 192, 64),
                                   (300, 1536, 256)])
def test_dx_without_workspace(device, t, n, k):
    state, w = weight(n, k)
    packed, qs = device_state(state, device)
    dy = x_of(t, n, seed=t + 17)
    dyt = torch.from_numpy(dy).to(device)
    base = x_of(t, k, seed=t + 18, scale=0.1)
    for accumulate in (0, 1):
        out = torch.from_numpy(base).to(device)
        _lib.call("ss_nf4_gemm_dx", dyt.data_ptr(), n, t, packed.data_ptr(), qs.absmax.data_ptr(),
                  qs.state2.absmax.data_ptr(), qs.state2.code.data_ptr(), qs.offset.data_ptr(),
                  n, k, out.data_ptr(), k, accumulate, None, 0, _lib.stream(device))
        expected = ogemm.linear_dx(dy, w) + (base.astype(np.float64) if accumulate else 0.0)
        check(out, expected, f"in-loop dx t={t} accumulate={accumulate}")
    check(nf4_matmul(dyt, packed, qs, transpose=True), ogemm.linear_dx(dy, w),
          f"decode-first dx t={t}")


# Fused dX for 16 < T <= 256 with dX columns % 128 == 0 and 128 or more
# workgroups: weight tiles decoded into LDS inside the GEMM (K-major B tiles,
# one scale per code piece), one or two 128-row tiles, ragged
# T, unsplit (a 512-row reduction) and split over the weight rows,
# accumulation.  Its rank-16 epilogue runs in the QLoRA projection tests.
@pytest.mark.parametrize("t,n,k", [(17, 8960, 1536), (64, 1536, 8960), (128, 8960, 1536),
                                   (130, 1536, 8960), (200, 512, 8960), (200, 3584, 3584),
                                   (256, 18944, 512)])
def test_fused_dx(device, t, n, k):
    state, w = weight(n, k)
    packed, qs = device_state(state, device)
    dy = x_of(t, n, seed=11 * t + n)
    dyt = torch.from_numpy(dy).to(device)
    dx = nf4_matmul(dyt, packed, qs, transpose=True)
    check(dx, ogemm.linear_dx(dy, w), f"fused dx t={t} n={n} k={k}")
    assert torch.equal(dx, nf4_matmul(dyt, packed, qs, transpose=True)), "fused dx not deterministic"
    base = x_of(t, k, seed=t + 5, scale=0.1)
    out = torch.from_numpy(base).to(device)
    nf4_dx_2d(dyt, packed, qs, n, k, out=out, accumulate=True)
    check(out, ogemm.linear_dx(dy, w) + base.astype(np.float64), f"fused dx accumulate t={t}")


# The streaming T <= 16 backward (transposed LDS reads of the codes, block
# scales folded into dY): ragged T, rows not a multiple of the 64-row unit,
# one to many row ranges, one column stage (K = 256) to many, N % 16 != 0
# (falls back to decode-first), and accumulation into dX.
@pytest.mark.parametrize("t,n,k", [
    (1, 4000, 3584), (16, 8960, 1536), (5, 1536, 256), (9, 64, 8960), (16, 3584, 4608),
    (3, 200, 512), (12, 1040, 768),
])
def test_streaming_dx_small_t(device, t, n, k):
    state, w = weight(n, k)
    packed, qs = device_state(state, device)
    dy = x_of(t, n, seed=5 * t + k)
    dyt = torch.from_numpy(dy).to(device)
    dx = nf4_matmul(dyt, packed, qs, transpose=True)
    check(dx, ogemm.linear_dx(dy, w), f"stream dx t={t} n={n} k={k}")
    assert torch.equal(dx, nf4_matmul(dyt, packed, qs, transpose=True)), "not deterministic"
    base = x_of(t, k, seed=t, scale=0.1)
    out = torch.from_numpy(base).to(device)
    nf4_dx_2d(dyt, packed, qs, n, k, out=out, accumulate=True)
    check(out, ogemm.linear_dx(dy, w) + base.astype(np.float64), f"stream dx accumulate t={t}")


# Decode-first products at the configs[1] layer shapes (T = 990: 256x256
# tiles for 990x8960x1536, split-K 128x128 for the long-K 990x1536x8960,
# 64x64 split-K for the narrow 990x256x1536), ragged T and N; split-K sums in
# split order, so two calls give the same bits; accumulation (beta = 1).
@pytest.mark.parametrize("t,n,k", [
    (990, 8960, 1536), (990, 1536, 1536), (990, 1536, 8960), (990, 256, 1536),
    (4100, 256, 1536), (300, 2000, 1536),
])
def test_decode_first_products(device, t, n, k):
    state, w = weight(n, k)
    packed, qs = device_state(state, device)
    x = x_of(t, k, seed=t + 2 * n)
    bias = (np.random.default_rng(9).standard_normal(n) * 0.1).astype(np.float16)
    xt = torch.from_numpy(x).to(device)
    bt = torch.from_numpy(bias).to(device)
    y = nf4_matmul(xt, packed, qs, bias=bt)
    check(y, ogemm.linear(x, w, bias), f"decode-first fwd t={t} n={n} k={k}")
    assert torch.equal(y, nf4_matmul(xt, packed, qs, bias=bt)), "decode-first fwd not deterministic"
    dy = x_of(t, n, seed=t + 3 * k)
    dyt = torch.from_numpy(dy).to(device)
    dx = nf4_matmul(dyt, packed, qs, transpose=True)
    check(dx, ogemm.linear_dx(dy, w), f"decode-first dx t={t} n={n} k={k}")
    assert torch.equal(dx, nf4_matmul(dyt, packed, qs, transpose=True)), "decode-first dx not deterministic"
    base = x_of(t, k, seed=t + 1, scale=0.1)
    out = torch.from_numpy(base).to(device)
    nf4_dx_2d(dyt, packed, qs, n, k, out=out, accumulate=True)
    check(out, ogemm.linear_dx(dy, w) + base.astype(np.float64), f"decode-first dx accumulate t={t}")


def test_dx_accumulate(device):
    state, w = weight(256, 1536)
    packed, qs = device_state(state, device)
    dy = x_of(64, 256, seed=1)
    base = x_of(64, 1536, seed=2, scale=0.1)
    out = torch.from_numpy(base).to(device)
    nf4_dx_2d(torch.from_numpy(dy).to(device), packed, qs, 256, 1536, out=out, accumulate=True)
    check(out, ogemm.linear_dx(dy, w) + base.astype(np.float64), "dx accumulate")


def test_large_t_decode_first_path(device):
    t, n, k = 4096, 512, 1536
    assert _lib.load().ss_nf4_gemm_workspace_size(t, n, k) == n * k * 2
    state, w = weight(n, k)
    packed, qs = device_state(state, device)
    x = x_of(t, k, seed=9)
    y = nf4_forward_2d(torch.from_numpy(x).to(device), packed, qs, n, k)
    check(y, ogemm.linear(x, w), "fwd decode-first")
    dy = x_of(t, n, seed=10)
    dx = nf4_dx_2d(torch.from_numpy(dy).to(device), packed, qs, n, k)
    check(dx, ogemm.linear_dx(dy, w), "dx decode-first")


def test_k_not_multiple_of_64_uses_dense_path(device):
    state, w = weight(96, 100)
    packed, qs = device_state(state, device)
    x = x_of(33, 100, seed=4)
    check(nf4_matmul(torch.from_numpy(x).to(device), packed, qs), ogemm.linear(x, w), "K=100")
    dy = x_of(33, 96, seed=5)
    check(nf4_matmul(torch.from_numpy(dy).to(device), packed, qs, transpose=True),
          ogemm.linear_dx(dy, w), "K=100 dx")


def test_validation_errors(device):
    state, _ = weight(64, 128)
    packed, qs = device_state(state, device)
    with pytest.raises(ValueError):
        nf4_matmul(torch.zeros((4, 64), device=device, dtype=torch.float16), packed, qs)
    with pytest.raises(ValueError):
        nf4_matmul(torch.zeros((4, 128), device=device, dtype=torch.float32), packed, qs)


@pytest.mark.parametrize("a_trans", [False, True])
@pytest.mark.parametrize("b_trans", [False, True])
@pytest.mark.parametrize("out_dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("m,n,k", [(37, 45, 70), (256, 16, 1536), (300, 1536, 16), (129, 200, 256)])
def test_dense_gemm_layouts(device, a_trans, b_trans, out_dtype, m, n, k):
    rng = np.random.default_rng(m * n + k)
    a = rng.standard_normal((m, k)).astype(np.float16)
    b = (rng.standard_normal((k, n)) * 0.1).astype(np.float16)
    bias = rng.standard_normal(n).astype(np.float16)
    ad = torch.from_numpy(np.ascontiguousarray(a.T if a_trans else a)).to(device)
    bd = torch.from_numpy(np.ascontiguousarray(b.T if b_trans else b)).to(device)
    c = gemm_f16(ad, bd, a_trans=a_trans, b_trans=b_trans, out_dtype=out_dtype, alpha=0.5,
                 bias=torch.from_numpy(bias).to(device))
    expected = 0.5 * (a.astype(np.float64) @ b.astype(np.float64)) + bias
    if out_dtype == torch.float16:
        check(c, expected, "dense f16")
    else:
        np.testing.assert_allclose(np16(c), expected, rtol=1e-5, atol=1e-4)
        # accumulate into the fp32 output
        gemm_f16(ad, bd, a_trans=a_trans, b_trans=b_trans, out=c, accumulate=True)
        np.testing.assert_allclose(np16(c), expected + a.astype(np.float64) @ b,
                                   rtol=1e-5, atol=2e-4)


@pytest.mark.parametrize("m,n,k", [(4100, 4128, 96),    # 256x256 tiles, ragged M and N
                                   (1000, 2000, 1536),  # 128x128 tiles
                                   (100, 300, 64),      # 64x64 tiles
                                   (990, 1536, 8960)])  # long K (a gate/up dX shape)
@pytest.mark.parametrize("out_dtype", [torch.float16, torch.float32])
def test_dense_nt_pipeline_tiles(device, m, n, k, out_dtype):
    """A [M,K] . B[N,K]^T with both operands K-contiguous and K % 32 == 0: the
    direct-to-LDS pipelined kernel at each of its tile sizes, plus beta = 1."""
    rng = np.random.default_rng(m + n + k)
    a = rng.standard_normal((m, k)).astype(np.float16)
    bt = (rng.standard_normal((n, k)) * 0.05).astype(np.float16)
    bias = rng.standard_normal(n).astype(np.float16)
    ad, bd = torch.from_numpy(a).to(device), torch.from_numpy(bt).to(device)
    c = gemm_f16(ad, bd, b_trans=True, out_dtype=out_dtype, bias=torch.from_numpy(bias).to(device))
    prod = a.astype(np.float64) @ bt.astype(np.float64).T
    expected = prod + bias
    if out_dtype == torch.float16:
        check(c, expected, f"nt {m}x{n}x{k}")
    else:
        np.testing.assert_allclose(np16(c), expected, rtol=1e-5, atol=2e-4)
    gemm_f16(ad, bd, b_trans=True, out=c, accumulate=True)
    if out_dtype == torch.float16:
        check(c, np16(torch.from_numpy(expected.astype(np.float16))).astype(np.float64) + prod,
              f"nt accumulate {m}x{n}x{k}")
    else:
        np.testing.assert_allclose(np16(c), expected + prod, rtol=1e-5, atol=4e-4)


@pytest.mark.parametrize("m,n,k", [(518, 1536, 8192),   # CE dX chunk: valid rows x H over a vocab chunk
                                   (64, 64, 4096), (200, 136, 1024), (300, 2000, 64)])
def test_dense_split_k(device, m, n, k):
    """ss_gemm_f16_split: the long reduction over few output tiles split over
    workgroups (partials in the caller's scratch), fp32 accumulate and fp16 out."""
    rng = np.random.default_rng(m * 7 + n + k)
    a = rng.standard_normal((m, k)).astype(np.float16)
    bt = (rng.standard_normal((n, k)) * 0.05).astype(np.float16)
    ad, bd = torch.from_numpy(a).to(device), torch.from_numpy(bt).to(device)
    prod = a.astype(np.float64) @ bt.astype(np.float64).T
    base = rng.standard_normal((m, n)).astype(np.float32)
    c = torch.from_numpy(base).to(device)
    gemm_f16(ad, bd, b_trans=True, out=c, accumulate=True, split_k=True)
    np.testing.assert_allclose(np16(c), base + prod, rtol=1e-5, atol=5e-4)
    h = gemm_f16(ad, bd, b_trans=True, alpha=0.25, split_k=True)
    check(h, 0.25 * prod, f"split fp16 {m}x{n}x{k}")


@pytest.mark.parametrize("t,n,k", [(990, 8960, 1536),   # 256x256 tiles, 4 M tiles
                                   (1024, 8960, 1536),  # configs[0]
                                   (800, 1536, 1536),   # 64x64 tiles
                                   (300, 256, 1536),    # 64x64 tiles split over k
                                   (990, 1536, 8960)])  # decode-first (long k)
def test_forward_bitwise_equals_decode_then_dense(device, t, n, k):
    """The NF4 forward (fused decode or decode-first, as dispatched) equals,
    bit for bit, the stand-alone decode followed by the dense NT GEMM with the
    same tile plan: the fused kernel's fp16 B tiles are the decoder's values
    and its k order is the dense kernel's."""
    state, _ = weight(n, k)
    packed, qs = device_state(state, device)
    x = torch.from_numpy(x_of(t, k, seed=7)).to(device)
    y = nf4_matmul(x, packed, qs)
    wd = torch.empty((n, k), device=device, dtype=torch.float16)
    _lib.call("ss_nf4_dequant_nested", packed.data_ptr(), qs.absmax.data_ptr(),
              qs.state2.absmax.data_ptr(), qs.state2.code.data_ptr(), qs.offset.data_ptr(),
              wd.data_ptr(), n * k, _lib.stream(device))
    ref = gemm_f16(x, wd, b_trans=True, split_k=True)
    assert torch.equal(y, ref)


@pytest.mark.parametrize("m,n,k,split", [
    (2048, 3584, 512, False),   # 128x256 tiles (8 waves)
    (4096, 4096, 128, False),   # 256x256 tiles, ping-pong main loop
    (1024, 2048, 256, False),   # 128x128 tiles
    (1000, 2008, 320, False),   # 128x128 tiles, ragged M and N
    (200, 136, 1024, False),    # 64x64 tiles
    (200, 136, 1024, True),     # 64x64 tiles split over K
    (990, 1536, 8960, True),    # 256x128 tiles split over K
    (1536, 1024, 4096, True),   # 128x128 tiles split over K
    (8, 16, 64, False),         # one 64x64 tile, 8-wide chunks clamped at M / N
])
@pytest.mark.parametrize("a_trans,b_trans", [(False, False), (True, False), (True, True)])
def test_dense_nt_k_major_operands(device, m, n, k, split, a_trans, b_trans):
    """K-major operands (a_trans: A stored [K,M]; b_trans False: B stored [K,N]) on the
    direct-to-LDS kernel, read with transposed LDS reads: the same tiles, splits and MFMA
    order as the K-contiguous layout, so the output equals that layout's bit for bit, and
    matches the float64 product (fp16 gate; fp32 out within 1e-5 relative).  A K-major
    operand whose M / N is not a multiple of 8 takes the general kernel (no bitwise
    comparison there)."""
    rng = np.random.default_rng(m * 3 + n * 5 + k)
    a = rng.standard_normal((m, k)).astype(np.float16)
    b = (rng.standard_normal((k, n)) * 0.05).astype(np.float16)
    ad = torch.from_numpy(np.ascontiguousarray(a.T if a_trans else a)).to(device)
    bd = torch.from_numpy(np.ascontiguousarray(b.T if b_trans else b)).to(device)
    a_row = torch.from_numpy(a).to(device)
    b_row = torch.from_numpy(np.ascontiguousarray(b.T)).to(device)
    prod = a.astype(np.float64) @ b.astype(np.float64)
    for out_dtype in (torch.float16, torch.float32):
        c = gemm_f16(ad, bd, a_trans=a_trans, b_trans=b_trans, out_dtype=out_dtype,
                     split_k=split)
        ref = gemm_f16(a_row, b_row, b_trans=True, out_dtype=out_dtype, split_k=split)
        torch.cuda.synchronize()
        if (not a_trans or m % 8 == 0) and (b_trans or n % 8 == 0):
            assert torch.equal(c, ref), f"layout {a_trans},{b_trans} differs from K-contiguous"
        if out_dtype == torch.float16:
            check(c, prod, f"k-major {m}x{n}x{k}")
        else:
            np.testing.assert_allclose(np16(c), prod, rtol=1e-5, atol=5e-4)
    base = rng.standard_normal((m, n)).astype(np.float32)
    acc = torch.from_numpy(base).to(device)
    gemm_f16(ad, bd, a_trans=a_trans, b_trans=b_trans, out=acc, accumulate=True, split_k=split)
    np.testing.assert_allclose(np16(acc), base + prod, rtol=1e-5, atol=5e-4)


@pytest.mark.parametrize("m,n,k,a_trans,b_trans,split", [
    (990, 1536, 8960, False, True, True),    # split-K: the reduce applies the scale
    (8192, 1536, 576, True, False, False),   # the CE head-gradient product (K-major operands)
    (300, 200, 100, False, False, False),    # K % 64 != 0: the general kernel
])
def test_dense_gemm_device_alpha(device, m, n, k, a_trans, b_trans, split):
    """alpha_dev (a device fp32 scalar) multiplies alpha in every dense path: the same bits
    as the host alpha of the product (0.5 x 3.0 = 1.5 exactly)."""
    rng = np.random.default_rng(m + n + k)
    a = rng.standard_normal((k, m) if a_trans else (m, k)).astype(np.float16)
    b = (rng.standard_normal((n, k) if b_trans else (k, n)) * 0.05).astype(np.float16)
    ad, bd = torch.from_numpy(a).to(device), torch.from_numpy(b).to(device)
    scale = torch.tensor([3.0], device=device, dtype=torch.float32)
    for out_dtype in (torch.float16, torch.float32):
        got = gemm_f16(ad, bd, a_trans=a_trans, b_trans=b_trans, out_dtype=out_dtype,
                       alpha=0.5, alpha_dev=scale, split_k=split)
        ref = gemm_f16(ad, bd, a_trans=a_trans, b_trans=b_trans, out_dtype=out_dtype,
                       alpha=1.5, split_k=split)
        torch.cuda.synchronize()
        assert torch.equal(got, ref)
