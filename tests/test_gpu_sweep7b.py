"""GPU parity of the NF4 forward and dX at BASELINE configs[4] (Qwen2.5-7B shapes).

Shapes, W [N, K]: q/o 3584x3584, k/v 512x3584, gate/up 18944x3584, down
3584x18944; T in {1, 16, 128, 2048, 16384}; both directions, through the same
C-ABI entry points (ss_nf4_gemm_fwd / ss_nf4_gemm_dx) and the same workspace
sizing the benchmark sweep uses, so every dispatched path of the sweep is the
one checked here: streaming (T <= 32), skinny / fused (T <= 256), decode-first
256x256 8-wave tiles at N = 18944, and split-K with the long K = 18944 of the
down projection.

Weights: seeded N(0, 0.02) fp16 quantized on the GPU (ss_nf4_quantize).  The
decoded weight is checked bit for bit against oracle/nf4.py on the first, a
middle and the last rows (its encoder-side state is whatever the kernel
wrote; the decoder is defined on any state), and the GEMM references are the
float64 products of that bit-exact decoded weight (oracle/gemm.py).

Bar: the reference's EXP-002 gate (experiments/reports/EXP-002.md:60-76),
rtol = atol = 2e-3 per element and relative L2 <= 1e-3 against the
decoded-weight product.  EXP-002 calibrated that element tolerance on
reductions up to 8960; over the 18944-long reductions here (down forward,
gate/up dX) the fp16 rounding of each decoded weight alone moves the
decoded-weight product by more than 2e-3 (the reference's own
decode-then-dense result misses the exact-weight product by ~4.4e-3).  There
the bar is the north star's "no worse than the reference's own error": the
relative L2 bound of EXP-002 still holds, and the largest element error and
the relative L2 error against the exact-weight product (oracle.nf4
decode_exact) are at most 1.25x those of the reference's fp16 decode-then-dense
result (oracle.gemm.no_worse_than_reference).  T <= 128: the full output.
T >= 2048: a seeded sample of 256 rows, plus the whole output finite and
bit-identical over two calls (split-K sums in split order).
"""

import numpy as np
import pytest
import torch

from oracle import gemm as ogemm
from oracle import nf4 as onf4
from soupsuck_amd.bnb_compat import quantize_4bit
from soupsuck_amd.kernels.nf4 import dequantize_nf4
from soupsuck_amd.kernels.nf4_gemm import nf4_dx_2d, nf4_forward_2d

pytestmark = pytest.mark.gpu

SHAPES = [("q_o", 3584, 3584), ("k_v", 512, 3584), ("gate_up", 18944, 3584),
          ("down", 3584, 18944)]
TS = [1, 16, 128, 2048, 16384]
SAMPLE_ROWS = 256


def _decode_rows_oracle(packed, qabs, absmax2, code2, offset, k, rows):
    """Oracle decode of whole rows ``rows`` of W [N, K] (K % 64 == 0)."""
    nblocks = qabs.size
    scale = onf4.blockwise_absmax(qabs, absmax2, code2, offset, nblocks)
    out = []
    for r in rows:
        lo, hi = r * k, (r + 1) * k
        out.append(onf4.decode_flat(packed[lo // 2:hi // 2], scale[lo // 64:hi // 64], k))
    return np.stack(out)


@pytest.fixture(scope="module", params=SHAPES, ids=[s[0] for s in SHAPES])
def weight7b(request, device):
    name, n, k = request.param
    gen = torch.Generator(device=device).manual_seed(1000 + n + k)
    w = (torch.randn((n, k), device=device, generator=gen) * 0.02).half()
    packed, state = quantize_4bit(w)
    del w
    decoded = dequantize_nf4(packed, state)
    rows = [0, 1, n // 2, n - 1]
    expect = _decode_rows_oracle(packed.cpu().numpy().reshape(-1), state.absmax.cpu().numpy(),
                                 state.state2.absmax.cpu().numpy(),
                                 state.state2.code.cpu().numpy(), state.offset.cpu().numpy(),
                                 k, rows)
    got = decoded[rows].cpu().numpy()
    np.testing.assert_array_equal(got.view(np.uint16), expect.view(np.uint16))
    w64 = decoded.cpu().numpy().astype(np.float64)
    del decoded
    wexact = onf4.decode_exact(packed.cpu().numpy().reshape(-1), state.absmax.cpu().numpy(),
                               state.state2.absmax.cpu().numpy(),
                               state.state2.code.cpu().numpy(), state.offset.cpu().numpy(),
                               n * k).reshape(n, k)
    yield name, n, k, packed, state, w64, wexact
    del packed, state, w64, wexact
    torch.cuda.empty_cache()


def _inputs(device, t, width, seed):
    gen = torch.Generator(device=device).manual_seed(seed)
    return torch.randn((t, width), device=device, generator=gen).half()


def _check(out, a64, w64, wexact, dx, reduction, what):
    prod = ogemm.linear_dx if dx else ogemm.linear
    ref = prod(a64, w64)
    got = out.cpu().numpy().astype(np.float64)
    ok, max_abs, rel = ogemm.gate(got, ref)
    if ok:
        return
    assert reduction > 8960 and rel <= ogemm.REL_L2, \
        f"{what}: max_abs={max_abs:.3e} rel_l2={rel:.3e}"
    exact = prod(a64, wexact)
    ok, ratio_max, ratio_l2 = ogemm.no_worse_than_reference(got, exact, ref.astype(np.float16))
    assert ok, (f"{what}: max_abs={max_abs:.3e} rel_l2={rel:.3e}; vs the exact-weight "
                f"product {ratio_max:.2f}x / {ratio_l2:.2f}x the reference's own error")


def _sample(t, seed):
    rng = np.random.default_rng(seed)
    rows = rng.choice(t, size=min(t, SAMPLE_ROWS), replace=False)
    rows.sort()
    return rows


@pytest.mark.parametrize("t", TS)
@pytest.mark.parametrize("mode", ["fwd", "dx"])
def test_configs4_shape(device, weight7b, t, mode):
    name, n, k, packed, state, w64, wexact = weight7b
    width_in = n if mode == "dx" else k
    a = _inputs(device, t, width_in, seed=7 * t + n + (1 if mode == "dx" else 0))
    what = f"{name} {mode} T={t} N={n} K={k}"
    print(what, flush=True)
    run = (lambda: nf4_dx_2d(a, packed, state, n, k)) if mode == "dx" else \
        (lambda: nf4_forward_2d(a, packed, state, n, k))
    out = run()
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all()), f"{what}: non-finite output"
    reduction = n if mode == "dx" else k
    if t <= 128:
        a64 = a.cpu().numpy().astype(np.float64)
        _check(out, a64, w64, wexact, mode == "dx", reduction, what)
    else:
        rows = _sample(t, seed=t + n + k)
        idx = torch.from_numpy(rows).to(device)
        a64 = a.index_select(0, idx).cpu().numpy().astype(np.float64)
        _check(out.index_select(0, idx), a64, w64, wexact, mode == "dx", reduction,
               what + f" ({rows.size} sampled rows)")
    again = run()
    assert torch.equal(out, again), f"{what}: two calls differ"
