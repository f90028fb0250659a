"""GPU parity of the packed causal attention (ss_attn_varlen_fwd / _bwd).

Bar (fp16 inputs and outputs, fp32 softmax, P rounded to fp16 before P.V as in
flash attention): against the float64 oracle (oracle/attention.py) of the same
fp16 inputs, the output within atol = rtol = 2e-3 elementwise and relative L2
<= 2e-3; the base-2 lse within 1e-3 of lse / ln 2; gradients dQ, dK, dV within
relative L2 1e-2 (fp16 outputs of sums over up to ~400 keys).  Cases: the
configs[1] batch (4 rows, lengths uniform in [80, 400], seed 0, T = 990) with
Qwen2.5-1.5B's 12 q heads and 2 kv heads; ragged rows of length 1 .. 130
(block edges 64 / 65 / 128 / 129); no GQA and 8:1 GQA; transposed projection
views as inputs; two calls bit-identical.
"""

import numpy as np
import pytest
import torch

from oracle import attention as oattn
from soupsuck_amd.kernels.attention import packed_causal_attention

pytestmark = pytest.mark.gpu


def _lengths_config1():
    gen = torch.Generator(device="cpu").manual_seed(0)
    return [int(v) for v in torch.randint(80, 401, (4,), generator=gen)]


def _proj_view(t, h, device, gen, scale=1.0):
    # [1, T, H*128] projection output viewed as [1, H, T, 128] (non-contiguous)
    x = (torch.randn((1, t, h * 128), generator=gen) * scale).half().to(device)
    return x.view(1, t, h, 128).transpose(1, 2)


def _np(t):
    # [1, H, T, D] -> [T, H, D]
    return t.detach()[0].transpose(0, 1).float().cpu().numpy()


@pytest.mark.parametrize("lengths,hq,hk", [
    (None, 12, 2),
    ((1, 17, 64, 65, 130, 128, 129), 4, 4),
    ((200, 3, 77), 8, 1),
])
def test_matches_oracle(device, lengths, hq, hk):
    lengths = lengths or _lengths_config1()
    t = sum(lengths)
    print(f"case attention lengths={lengths} hq={hq} hk={hk}", flush=True)
    gen = torch.Generator().manual_seed(t + hq)
    q = _proj_view(t, hq, device, gen).requires_grad_()
    k = _proj_view(t, hk, device, gen).requires_grad_()
    v = _proj_view(t, hk, device, gen).requires_grad_()
    scale = 128 ** -0.5
    o = packed_causal_attention(q, k, v, lengths, scale)
    assert o.shape == (1, t, hq, 128) and o.is_contiguous()
    ref, lse = oattn.forward(_np(q), _np(k), _np(v), lengths, scale)
    got = o.detach()[0].float().cpu().numpy().astype(np.float64)
    np.testing.assert_allclose(got, ref, rtol=2e-3, atol=2e-3)
    assert np.linalg.norm(got - ref) <= 2e-3 * np.linalg.norm(ref)
    assert torch.equal(o, packed_causal_attention(q, k, v, lengths, scale))
    g = (torch.randn((1, t, hq, 128), generator=gen)).half().to(device)
    o.backward(g)
    dq, dk, dv = oattn.backward(_np(q), _np(k), _np(v), g[0].float().cpu().numpy(), lengths,
                                scale)
    for name, got_g, ref_g in (("dq", q.grad, dq), ("dk", k.grad, dk), ("dv", v.grad, dv)):
        arr = _np(got_g).astype(np.float64)
        err = np.linalg.norm(arr - ref_g) / np.linalg.norm(ref_g)
        assert err < 1e-2, f"{name}: rel L2 {err:.3e}"


def test_lse_and_delta_statistics(device):
    lengths = (70, 5, 140)
    t = sum(lengths)
    gen = torch.Generator().manual_seed(9)
    q = _proj_view(t, 4, device, gen)
    k = _proj_view(t, 2, device, gen)
    v = _proj_view(t, 2, device, gen)
    from soupsuck_amd import _lib
    from soupsuck_amd.kernels.attention import row_offsets

    cu = row_offsets(lengths, device)
    o = torch.empty((1, t, 4, 128), device=device, dtype=torch.float16)
    lse2 = torch.empty((4, t), device=device, dtype=torch.float32)
    ov = o.transpose(1, 2)
    _lib.call("ss_attn_varlen_fwd", q.data_ptr(), q.stride(2), q.stride(1), k.data_ptr(),
              k.stride(2), k.stride(1), v.data_ptr(), v.stride(2), v.stride(1), cu.data_ptr(),
              len(lengths), max(lengths), t, 4, 2, 128, 0.1, o.data_ptr(), ov.stride(2),
              ov.stride(1), lse2.data_ptr(), _lib.stream(device))
    _, lse = oattn.forward(_np(q), _np(k), _np(v), lengths, 0.1)
    np.testing.assert_allclose(lse2.cpu().numpy(), lse / np.log(2), rtol=1e-4, atol=1e-3)


def test_rejects_unsupported(device):
    q = torch.zeros((1, 2, 8, 64), device=device, dtype=torch.float16)
    with pytest.raises(ValueError):
        packed_causal_attention(q, q, q, [8], 0.1)                    # head_dim 64
    q = torch.zeros((1, 2, 8, 128), device=device, dtype=torch.float16)
    with pytest.raises(ValueError):
        packed_causal_attention(q, q, q, [3, 4], 0.1)                 # lengths do not sum to T
