"""GPU check of ss_nf4_gemm_fwd_noalloc (the forward with a fixed device scratch).

The entry point runs ss_nf4_gemm_fwd's kernels with the scratch in a static
device array instead of a caller workspace, so at every shape its output must
be bit-identical to ss_nf4_gemm_fwd's (a stronger bar than the GEMM tolerance:
the same kernels run on the same operands).  Cases cover every forward path
the scratch serves: streaming (T <= 32), skinny (T <= 128), the fused NF4 GEMM
(128 < T < 256) and decode-first (T >= 256, small weight).  Two calls run back
to back with nothing between them, the second on a smaller input, so the
second call meets the first call's leftovers in the shared scratch.  A shape
whose forward needs more scratch than the array holds is rejected with
ValueError before any launch.  All calls go through the C ABI.
"""

import pytest
import torch

from soupsuck_amd import _lib
from soupsuck_amd.bnb_compat import quantize_4bit

pytestmark = pytest.mark.gpu

# (N, K), then (T of the first call, T of the second, smaller, call).
CASES = [
    ((18944, 3584), (128, 17)),   # skinny, then streaming
    ((3584, 18944), (255, 16)),   # fused NF4 GEMM with split-K, then streaming
    ((8960, 1536), (200, 100)),   # fused, then skinny
    ((1536, 1536), (990, 300)),   # decode-first (decoded weight in the scratch), twice
    ((512, 3584), (32, 1)),       # streaming, twice
]


def _weight(n, k, device, seed):
    gen = torch.Generator(device=device).manual_seed(seed)
    w = (torch.randn((n, k), device=device, generator=gen) * 0.02).half()
    return quantize_4bit(w)


def _state_args(packed, st):
    return (packed.data_ptr(), st.absmax.data_ptr(), st.state2.absmax.data_ptr(),
            st.state2.code.data_ptr(), st.offset.data_ptr())


def _with_workspace(x, packed, st, n, k, bias):
    t = x.shape[0]
    y = torch.empty((t, n), device=x.device, dtype=torch.float16)
    size = _lib.load().ss_nf4_gemm_workspace_size(t, n, k)
    ws = torch.empty(max(size, 1), device=x.device, dtype=torch.uint8)
    _lib.call("ss_nf4_gemm_fwd", x.data_ptr(), x.stride(0), t, *_state_args(packed, st), n, k,
              _lib.ptr(bias), y.data_ptr(), y.stride(0), ws.data_ptr(), size,
              _lib.stream(x.device))
    return y


def _noalloc(x, packed, st, n, k, bias, y):
    _lib.call("ss_nf4_gemm_fwd_noalloc", x.data_ptr(), x.stride(0), x.shape[0],
              *_state_args(packed, st), n, k, _lib.ptr(bias), y.data_ptr(), y.stride(0),
              _lib.stream(x.device))


@pytest.mark.parametrize("shape,ts", CASES, ids=[f"{c[0][0]}x{c[0][1]}-T{c[1][0]}-{c[1][1]}"
                                                 for c in CASES])
def test_noalloc_forward_equals_workspace_forward(device, shape, ts):
    n, k = shape
    t1, t2 = ts
    print(f"case noalloc N={n} K={k} T={t1} then T={t2}", flush=True)
    packed, st = _weight(n, k, device, seed=n + k)
    gen = torch.Generator(device=device).manual_seed(t1 + t2)
    x1 = torch.randn((t1, k), device=device, generator=gen).half()
    x2 = torch.randn((t2, k), device=device, generator=gen).half()
    bias = (torch.randn(n, device=device, generator=gen) * 0.1).half()
    ref1 = _with_workspace(x1, packed, st, n, k, bias)
    ref2 = _with_workspace(x2, packed, st, n, k, None)
    torch.cuda.synchronize()
    y1 = torch.full((t1, n), float("nan"), device=device, dtype=torch.float16)
    y2 = torch.full((t2, n), float("nan"), device=device, dtype=torch.float16)
    _noalloc(x1, packed, st, n, k, bias, y1)
    _noalloc(x2, packed, st, n, k, None, y2)
    torch.cuda.synchronize()
    assert torch.equal(y1, ref1), f"first call (T={t1}) differs from ss_nf4_gemm_fwd"
    assert torch.equal(y2, ref2), f"second call (T={t2}) differs from ss_nf4_gemm_fwd"


def test_noalloc_rejects_shapes_beyond_its_scratch(device):
    n, k, t = 18944, 3584, 4096  # decode-first: the 136 MB decoded weight does not fit
    packed, st = _weight(n, k, device, seed=5)
    x = torch.zeros((t, k), device=device, dtype=torch.float16)
    y = torch.zeros((t, n), device=device, dtype=torch.float16)
    with pytest.raises(ValueError, match="scratch"):
        _noalloc(x, packed, st, n, k, None, y)
    torch.cuda.synchronize()
    assert not bool(y.any()), "rejected call must not launch"


def test_noalloc_unvectorisable_x_takes_the_workspace_path(device):
    """X rows 1540 halves apart (ldx % 8 != 0) rule out the 16-byte-load kernels; at T = 200
    both entry points then decode W first, so the scratch holds the decoded weight and the
    outputs stay bit-identical.  The second call (T = 100, dense X) is the skinny kernel."""
    n, k = 8960, 1536
    print(f"case noalloc unvectorisable X N={n} K={k} T=200 then T=100", flush=True)
    packed, st = _weight(n, k, device, seed=11)
    gen = torch.Generator(device=device).manual_seed(3)
    x1 = torch.randn((200, k + 4), device=device, generator=gen).half()[:, :k]
    x2 = torch.randn((100, k), device=device, generator=gen).half()
    assert x1.stride(0) % 8 != 0
    ref1 = _with_workspace(x1, packed, st, n, k, None)
    ref2 = _with_workspace(x2, packed, st, n, k, None)
    torch.cuda.synchronize()
    y1 = torch.full((200, n), float("nan"), device=device, dtype=torch.float16)
    y2 = torch.full((100, n), float("nan"), device=device, dtype=torch.float16)
    _noalloc(x1, packed, st, n, k, None, y1)
    _noalloc(x2, packed, st, n, k, None, y2)
    torch.cuda.synchronize()
    assert torch.equal(y1, ref1) and torch.equal(y2, ref2)
