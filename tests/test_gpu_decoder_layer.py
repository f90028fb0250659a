"""GPU check of the whole decoder layer (soupsuck_amd.layer.DecoderLayer) against an
fp32 PyTorch composition of the same layer on the same weights.

The reference composition uses the bit-exact dequantized NF4 weights, fp32
matmuls, Qwen2's RMSNorm / rotate-half RoPE / SwiGLU formulas and causal
softmax attention within each packed row, all in float32 on the GPU, with
autograd for the gradients.  Bar: output, input gradient and every LoRA A / B
gradient within relative L2 2e-2 (a chain of ten fp16-rounded ops against
fp32), and the output of two runs bit-identical.  configs[1] batch: 4 rows,
lengths uniform in [80, 400] (seed 0), T = 990.
"""

import pytest
import torch

from soupsuck_amd.kernels.nf4 import dequantize_nf4
from soupsuck_amd.layer import DecoderLayer

pytestmark = pytest.mark.gpu


def _lengths():
    gen = torch.Generator(device="cpu").manual_seed(0)
    return [int(v) for v in torch.randint(80, 401, (4,), generator=gen)]


def _rel(a, b):
    a, b = a.double(), b.double()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def _reference(layer, h, lengths):
    f = torch.float32
    p = {q.name: q for q in layer.proj.projections}
    leaves = {n: (q.lora_a.detach().float().requires_grad_(),
                  q.lora_b.detach().float().requires_grad_()) for n, q in p.items()}
    x0 = h.detach().float().requires_grad_()

    def norm(x, w):
        var = x.pow(2).mean(-1, keepdim=True)
        return w.float() * (x * torch.rsqrt(var + 1e-6))

    def proj(name, x):
        q = p[name]
        w = dequantize_nf4(q.packed, q.state).float()
        a, b = leaves[name]
        y = x @ w.t() + (x @ a.t()) @ b.t() * layer.proj.scaling
        return y + q.bias.float() if q.bias is not None else y

    def rope(x):
        c, s = layer.cos.float(), layer.sin.float()
        x1, x2 = x[..., :64], x[..., 64:]
        return x * c + torch.cat([-x2, x1], -1) * s

    t = h.shape[0]
    x = norm(x0, layer.norm_in)
    q = rope(proj("q_proj", x).view(t, 12, 128).transpose(0, 1))
    k = rope(proj("k_proj", x).view(t, 2, 128).transpose(0, 1))
    v = proj("v_proj", x).view(t, 2, 128).transpose(0, 1)
    k, v = k.repeat_interleave(6, 0), v.repeat_interleave(6, 0)
    outs, start = [], 0
    for n in lengths:
        rows = slice(start, start + n)
        s = q[:, rows] @ k[:, rows].transpose(1, 2) * 128 ** -0.5
        mask = torch.ones((n, n), dtype=torch.bool, device=h.device).tril()
        s = s.masked_fill(~mask, float("-inf"))
        outs.append(torch.softmax(s, -1) @ v[:, rows])
        start += n
    attn = torch.cat(outs, 1).transpose(0, 1).reshape(t, 1536)
    residual = x0 + proj("o_proj", attn)
    x2 = norm(residual, layer.norm_post)
    g, u = proj("gate_proj", x2), proj("up_proj", x2)
    out = residual + proj("down_proj", torch.nn.functional.silu(g) * u)
    return out, x0, leaves


def test_decoder_layer_matches_fp32_composition(device):
    lengths = _lengths()
    t = sum(lengths)
    layer = DecoderLayer(device, lengths)
    gen = torch.Generator(device="cpu").manual_seed(3)
    h = torch.randn((t, 1536), generator=gen).half().to(device).requires_grad_()
    g = (torch.randn((t, 1536), generator=gen) * 0.05).half().to(device)
    out = layer.step(h, g)
    again = layer.forward(h.detach().requires_grad_())
    assert torch.equal(out, again), "two runs differ"
    ref, x0, leaves = _reference(layer, h, lengths)
    ref.backward(g.float())
    assert _rel(out.detach(), ref.detach()) < 2e-2
    assert _rel(h.grad, x0.grad) < 2e-2, _rel(h.grad, x0.grad)
    for q in layer.proj.projections:
        a, b = leaves[q.name]
        assert _rel(q.lora_a.grad, a.grad) < 2e-2, (q.name, "A", _rel(q.lora_a.grad, a.grad))
        assert _rel(q.lora_b.grad, b.grad) < 2e-2, (q.name, "B", _rel(q.lora_b.grad, b.grad))
