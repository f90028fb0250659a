"""One Qwen2 decoder layer's seven QLoRA projections (the benchmark workload).

Shapes follow Qwen2.5 (hidden 1536, intermediate 8960, 12 query heads and 2
key/value heads of 128 -> k/v out 256; q/k/v have a bias, o/gate/up/down do
not).  Every projection is an NF4 weight (nested statistics, blocksize 64)
with a LoRA adapter (r = 16, alpha = 32 -> scaling 2.0, A Kaiming-uniform,
B ~ N(0, 0.01), fp16), run through ``qlora_projection``.  A step is the
forward of all seven projections on a packed batch of T tokens followed by
their backward (dX, dA, dB).  Work per step is reported by ``flops()`` and
``weight_bytes()``.
"""

import math
from dataclasses import dataclass

import torch

from .bnb_compat import quantize_4bit
from .lora import qlora_projection

QWEN_1_5B = dict(hidden=1536, intermediate=8960, kv=256)
QWEN_7B = dict(hidden=3584, intermediate=18944, kv=512)


def projection_shapes(hidden, intermediate, kv):
    """(name, in_features K, out_features N, has_bias) for the seven projections."""
    return [("q_proj", hidden, hidden, True), ("k_proj", hidden, kv, True),
            ("v_proj", hidden, kv, True), ("o_proj", hidden, hidden, False),
            ("gate_proj", hidden, intermediate, False), ("up_proj", hidden, intermediate, False),
            ("down_proj", intermediate, hidden, False)]


@dataclass
class Projection:
    name: str
    k: int
    n: int
    packed: torch.Tensor
    state: object
    bias: torch.Tensor
    lora_a: torch.Tensor
    lora_b: torch.Tensor


class QLoRALayer:
    def __init__(self, device, hidden=1536, intermediate=8960, kv=256, rank=16, alpha=32,
                 seed=0, dropout_p=0.0):
        gen = torch.Generator(device="cpu").manual_seed(seed)
        self.rank, self.scaling, self.dropout_p = rank, alpha / rank, dropout_p
        self.projections = []
        for name, k, n, has_bias in projection_shapes(hidden, intermediate, kv):
            w = (torch.randn((n, k), generator=gen) * 0.02).to(torch.float16).to(device)
            packed, state = quantize_4bit(w, blocksize=64, compress_statistics=True,
                                          quant_type="nf4")
            del w
            bias = ((torch.randn(n, generator=gen) * 0.02).to(torch.float16).to(device)
                    if has_bias else None)
            bound = 1.0 / math.sqrt(k)  # kaiming_uniform_(a=sqrt(5)) on [r, K]
            a = ((torch.rand((rank, k), generator=gen) * 2 - 1) * bound).to(torch.float16)
            b = (torch.randn((n, rank), generator=gen) * 0.01).to(torch.float16)
            self.projections.append(Projection(
                name, k, n, packed, state, bias,
                a.to(device).requires_grad_(), b.to(device).requires_grad_()))

    def inputs(self, tokens, device, seed=1):
        gen = torch.Generator(device="cpu").manual_seed(seed)
        xs, gs = [], []
        for p in self.projections:
            xs.append(torch.randn((tokens, p.k), generator=gen).to(torch.float16).to(device))
            gs.append((torch.randn((tokens, p.n), generator=gen) * 0.01)
                      .to(torch.float16).to(device))
        return xs, gs

    def step(self, xs, gs):
        """Forward all seven projections, then backward with upstream gradients gs."""
        outs = []
        for p, x in zip(self.projections, xs):
            x.requires_grad_(True)
            outs.append(qlora_projection(x, p.lora_a, p.lora_b, p.packed, p.state, p.bias,
                                         self.scaling, self.dropout_p))
        torch.autograd.backward(outs, gs)
        return outs

    def flops(self, tokens):
        """Algorithmic flops of one step: base fwd + dX, LoRA fwd (2 GEMMs) + bwd (4 GEMMs)."""
        total = 0
        for p in self.projections:
            base = 2 * tokens * p.n * p.k
            lora_fwd = 2 * tokens * self.rank * (p.k + p.n)
            total += 2 * base + 3 * lora_fwd
        return total

    def weight_bytes(self):
        """NF4 bytes read per pass over the seven weights (codes + statistics)."""
        total = 0
        for p in self.projections:
            nk = p.n * p.k
            total += nk // 2 + -(-nk // 64) + 4 * -(-nk // 16384) + 1024 + 4
        return total


class DecoderLayer:
    """A whole Qwen2.5-1.5B decoder layer on a packed batch, every op on this package's
    kernels: RMSNorm -> q/k/v QLoRA projections -> joint q/k RoPE -> causal attention
    within each packed row -> o projection -> residual add + RMSNorm -> gate/up
    projections -> SwiGLU -> down projection -> residual add.  Forward then backward
    of the whole layer from an upstream gradient (the north star's full-layer time).
    The seven projections are ``QLoRALayer``'s; norm weights ~ 1 + N(0, 0.1) fp16;
    RoPE angles are Qwen2's (theta 1e6) at each token's position within its row."""

    def __init__(self, device, lengths, hidden=1536, intermediate=8960, kv=256, heads=12,
                 kv_heads=2, seed=0):
        from .kernels.attention import row_offsets

        self.proj = QLoRALayer(device, hidden, intermediate, kv, seed=seed)
        gen = torch.Generator(device="cpu").manual_seed(seed + 7)
        self.norm_in = (1 + 0.1 * torch.randn(hidden, generator=gen)).half().to(device)
        self.norm_post = (1 + 0.1 * torch.randn(hidden, generator=gen)).half().to(device)
        self.lengths = [int(n) for n in lengths]
        self.heads, self.kv_heads, self.head_dim = heads, kv_heads, hidden // heads
        self.cu = row_offsets(self.lengths, device)
        pos = torch.cat([torch.arange(n, dtype=torch.float64) for n in self.lengths])
        inv = 1.0 / (1_000_000 ** (torch.arange(0, self.head_dim, 2, dtype=torch.float64)
                                    / self.head_dim))
        ang = pos[:, None] * inv[None, :]
        emb = torch.cat([ang, ang], dim=-1)
        self.cos = emb.cos()[None].half().to(device)
        self.sin = emb.sin()[None].half().to(device)

    def forward(self, h):
        from .kernels.add_rmsnorm import add_rms_norm
        from .kernels.attention import packed_causal_attention
        from .kernels.rmsnorm import rms_norm
        from .kernels.rope import fused_rope
        from .kernels.swiglu import swiglu

        p = {q.name: q for q in self.proj.projections}
        s = self.proj.scaling
        t, d = h.shape[0], self.head_dim

        def run(name, x):
            q = p[name]
            return qlora_projection(x, q.lora_a, q.lora_b, q.packed, q.state, q.bias, s)

        x = rms_norm(h, self.norm_in, 1e-6)
        q = run("q_proj", x).view(1, t, self.heads, d).transpose(1, 2)
        k = run("k_proj", x).view(1, t, self.kv_heads, d).transpose(1, 2)
        v = run("v_proj", x).view(1, t, self.kv_heads, d).transpose(1, 2)
        q, k = fused_rope(q, k, self.cos, self.sin)
        attn = packed_causal_attention(q, k, v, self.lengths, d ** -0.5, cu_seqlens=self.cu)
        o = run("o_proj", attn.view(t, self.heads * d))
        residual, x2 = add_rms_norm(h, o, self.norm_post, 1e-6)
        act = swiglu(run("gate_proj", x2), run("up_proj", x2))
        return residual + run("down_proj", act)

    def step(self, h, g):
        for q in self.proj.projections:
            q.lora_a.grad = None
            q.lora_b.grad = None
        h.grad = None
        out = self.forward(h)
        out.backward(g)
        return out

    def flops(self):
        """Projection flops (QLoRALayer.flops) + attention: 2 products forward and 4
        backward of 2 * head_dim flops per causal (query, key) pair per q head."""
        t = sum(self.lengths)
        pairs = sum(n * (n + 1) // 2 for n in self.lengths)
        return self.proj.flops(t) + 6 * 2 * self.head_dim * pairs * self.heads
