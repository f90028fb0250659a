"""GPU parity of the joint q/k RoPE kernels (ss_rope_fwd / ss_rope_bwd).

Bar: bit-exact against oracle/rope.py (fp32 products rounded to the output
dtype before each add, no contraction), for the Qwen2.5-1.5B attention shapes
(12 q heads, 2 k heads, head_dim 128) at T = 990, transposed projection views
([B, S, H, D].transpose(1, 2), as Qwen2Attention passes them), B = 2 with
per-batch and broadcast cos/sin, mixed q/k/cos dtypes (solution/kernels/
rope.py:1-15), gradients for q only / k only, and the autograd node against
transformers' eager apply_rotary_pos_emb within fp16 tolerance.
"""

import numpy as np
import pytest
import torch

from oracle import rope as orope
from soupsuck_amd.kernels.rope import fused_rope, patch_qwen2_rope
from tests.gpu_util import np16

pytestmark = pytest.mark.gpu


def _angles(b, s, d, device, dtype, seed=0):
    inv = 1.0 / (1000000 ** (torch.arange(0, d, 2, dtype=torch.float64) / d))
    pos = torch.arange(s, dtype=torch.float64)[:, None] + seed
    emb = torch.cat([pos * inv, pos * inv], dim=-1)
    cos = emb.cos()[None].repeat(b, 1, 1).to(dtype).to(device)
    sin = emb.sin()[None].repeat(b, 1, 1).to(dtype).to(device)
    return cos, sin


def _proj(b, s, h, d, dtype, device, gen):
    # [B, S, H*D] projection output viewed as [B, H, S, D] (non-contiguous).
    x = torch.randn((b, s, h * d), generator=gen).to(dtype).to(device)
    return x.view(b, s, h, d).transpose(1, 2)


def _exact(t, ref):
    got = np16(t)
    if ref.dtype == np.float16:
        np.testing.assert_array_equal(got.view(np.int16), ref.view(np.int16))
    else:
        np.testing.assert_array_equal(got, ref)


@pytest.mark.parametrize("qdt,kdt,cdt", [(torch.float16, torch.float16, torch.float16),
                                         (torch.float16, torch.float16, torch.float32),
                                         (torch.float16, torch.float32, torch.float32),
                                         (torch.float32, torch.float16, torch.float16),
                                         (torch.float32, torch.float32, torch.float32)])
@pytest.mark.parametrize("b,s,cb", [(1, 990, 1), (2, 77, 2), (2, 33, 1)])
def test_bit_exact_against_oracle(device, qdt, kdt, cdt, b, s, cb):
    print(f"case rope b={b} s={s} cb={cb} q={qdt} k={kdt} c={cdt}", flush=True)
    gen = torch.Generator().manual_seed(s)
    q = _proj(b, s, 12, 128, qdt, device, gen).requires_grad_()
    k = _proj(b, s, 2, 128, kdt, device, gen).requires_grad_()
    cos, sin = _angles(cb, s, 128, device, cdt)
    yq, yk = fused_rope(q, k, cos, sin)
    assert yq.is_contiguous() and yk.is_contiguous()
    cn, sn = np16(cos), np16(sin)
    _exact(yq, orope.rope_forward(np16(q), cn, sn))
    _exact(yk, orope.rope_forward(np16(k), cn, sn))
    gq = torch.randn(yq.shape, generator=gen).to(yq.dtype).to(device)
    gk = torch.randn(yk.shape, generator=gen).to(yk.dtype).to(device)
    torch.autograd.backward([yq, yk], [gq, gk])
    assert q.grad.dtype == qdt and k.grad.dtype == kdt
    _exact(q.grad, orope.rope_backward(np16(gq), cn, sn, np16(q).dtype))
    _exact(k.grad, orope.rope_backward(np16(gk), cn, sn, np16(k).dtype))


def test_one_side_gradient_and_strided_upstream(device):
    gen = torch.Generator().manual_seed(5)
    q = _proj(1, 40, 12, 128, torch.float16, device, gen).requires_grad_()
    k = _proj(1, 40, 2, 128, torch.float16, device, gen)
    cos, sin = _angles(1, 40, 128, device, torch.float16)
    yq, yk = fused_rope(q, k, cos, sin)
    g = torch.randn((1, 40, 12, 128), generator=gen).half().to(device).transpose(1, 2)
    yq.backward(g)
    _exact(q.grad, orope.rope_backward(np16(g), np16(cos), np16(sin), np.float16))
    assert k.grad is None


def test_patched_apply_rotary_pos_emb_matches_eager(device):
    modeling = pytest.importorskip("transformers.models.qwen2.modeling_qwen2")
    gen = torch.Generator().manual_seed(9)
    q = _proj(1, 64, 12, 128, torch.float16, device, gen)
    k = _proj(1, 64, 2, 128, torch.float16, device, gen)
    cos, sin = _angles(1, 64, 128, device, torch.float16)
    original = modeling.apply_rotary_pos_emb
    eq, ek = original(q, k, cos, sin)
    assert patch_qwen2_rope(modeling)
    try:
        aq, ak = modeling.apply_rotary_pos_emb(q, k, cos, sin)
    finally:
        modeling.apply_rotary_pos_emb = original
    torch.testing.assert_close(aq, eq, rtol=2e-3, atol=2e-3)
    torch.testing.assert_close(ak, ek, rtol=2e-3, atol=2e-3)


def test_rejects_unsupported(device):
    q = torch.zeros((1, 2, 4, 7), device=device, dtype=torch.float16)
    cos = torch.zeros((1, 4, 7), device=device, dtype=torch.float16)
    with pytest.raises(ValueError):
        fused_rope(q, q, cos, cos)


# The element-wise kernel (rope_kernel): taken when half = D / 2 is not a
# multiple of 4, when the upstream gradient's last stride is not 1, or when a
# base address is not 16-byte aligned.  Same bit-exact bar.
def test_scalar_path_head_dim_12(device):
    gen = torch.Generator().manual_seed(21)
    q = _proj(2, 37, 3, 12, torch.float16, device, gen).requires_grad_()
    k = _proj(2, 37, 1, 12, torch.float32, device, gen).requires_grad_()
    cos, sin = _angles(2, 37, 12, device, torch.float16)
    yq, yk = fused_rope(q, k, cos, sin)
    cn, sn = np16(cos), np16(sin)
    _exact(yq, orope.rope_forward(np16(q), cn, sn))
    _exact(yk, orope.rope_forward(np16(k), cn, sn))
    gq = torch.randn(yq.shape, generator=gen).half().to(device)
    gk = torch.randn(yk.shape, generator=gen).float().to(device)
    torch.autograd.backward([yq, yk], [gq, gk])
    _exact(q.grad, orope.rope_backward(np16(gq), cn, sn, np.float16))
    _exact(k.grad, orope.rope_backward(np16(gk), cn, sn, np.float32))


def test_scalar_path_expanded_gradient(device):
    gen = torch.Generator().manual_seed(22)
    q = _proj(1, 50, 12, 128, torch.float16, device, gen).requires_grad_()
    k = _proj(1, 50, 2, 128, torch.float16, device, gen).requires_grad_()
    cos, sin = _angles(1, 50, 128, device, torch.float16)
    yq, yk = fused_rope(q, k, cos, sin)
    gq = torch.randn((1, 12, 50, 1), generator=gen).half().to(device).expand(1, 12, 50, 128)
    gk = torch.randn((1, 2, 50, 1), generator=gen).half().to(device).expand(1, 2, 50, 128)
    assert gq.stride(-1) == 0
    torch.autograd.backward([yq, yk], [gq, gk])
    cn, sn = np16(cos), np16(sin)
    _exact(q.grad, orope.rope_backward(np16(gq), cn, sn, np.float16))
    _exact(k.grad, orope.rope_backward(np16(gk), cn, sn, np.float16))


def test_scalar_path_unaligned_base(device):
    gen = torch.Generator().manual_seed(23)
    b, s, h, d = 1, 45, 12, 128
    buf = torch.randn(b * s * h * d + 1, generator=gen).half().to(device)
    q = buf[1:].view(b, s, h, d).transpose(1, 2).requires_grad_()
    assert q.data_ptr() % 16 != 0
    k = _proj(b, s, 2, d, torch.float16, device, gen).requires_grad_()
    cos, sin = _angles(1, s, d, device, torch.float16)
    yq, yk = fused_rope(q, k, cos, sin)
    cn, sn = np16(cos), np16(sin)
    _exact(yq, orope.rope_forward(np16(q), cn, sn))
    _exact(yk, orope.rope_forward(np16(k), cn, sn))
    gq = torch.randn(yq.shape, generator=gen).half().to(device)
    gk = torch.randn(yk.shape, generator=gen).half().to(device)
    torch.autograd.backward([yq, yk], [gq, gk])
    _exact(q.grad, orope.rope_backward(np16(gq), cn, sn, np.float16))
    _exact(k.grad, orope.rope_backward(np16(gk), cn, sn, np.float16))
