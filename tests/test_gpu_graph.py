"""HIP-graph capture of the QLoRA layer step (the benchmark's timed unit).

The step -- seven NF4 + LoRA projections forward, then dX / dA / dB -- is
captured once with torch.cuda.CUDAGraph and replayed.  Every replay must
reproduce the eager step bit for bit: the kernels are deterministic (split
reductions in a fixed order, no atomics) and none of them records a memset
or allocates.  Replays are interleaved with unrelated eager GPU work and
synchronisations, and each replay is checked.
"""

import pytest
import torch

from soupsuck_amd.layer import QLoRALayer

pytestmark = pytest.mark.gpu


def _grads(layer, xs):
    out = []
    for p, x in zip(layer.projections, xs):
        out += [p.lora_a.grad, p.lora_b.grad, x.grad]
    return out


def test_graph_replay_matches_eager(device):
    layer = QLoRALayer(device)
    xs, gs = layer.inputs(300, device)

    def step():
        for p in layer.projections:
            p.lora_a.grad = None
            p.lora_b.grad = None
        for x in xs:
            x.grad = None
        return layer.step(xs, gs)

    eager_out = [o.detach().clone() for o in step()]
    eager_grads = [g.clone() for g in _grads(layer, xs)]

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        graph_out = step()
    graph_grads = _grads(layer, xs)

    noise = torch.randn((512, 512), device=device)
    for replay in range(3):
        for o in graph_out:
            o.detach().zero_()   # same storage; the replay must rewrite it
        graph.replay()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(graph_out, eager_out)):
            assert torch.equal(a, b), f"replay {replay}: output {i} differs"
        for i, (a, b) in enumerate(zip(graph_grads, eager_grads)):
            assert torch.equal(a, b), f"replay {replay}: gradient {i} differs"
        noise = noise @ noise.t() / 512.0   # unrelated eager work between replays
        torch.cuda.synchronize()


def test_graph_replay_after_rank_workspace_growth(device):
    """A graph captured on a stream keeps addressing the rank-16 workspace it
    was captured with.  A larger eager step on the same stream then grows that
    stream's workspace; the old buffer must stay allocated (its counters at
    zero) so that replays, after fresh allocations that could reuse freed
    memory, still reproduce the eager step bit for bit."""
    layer = QLoRALayer(device, seed=3)
    small_x, small_g = layer.inputs(128, device, seed=5)
    big_x, big_g = layer.inputs(2048, device, seed=6)

    def step(xs, gs):
        for p in layer.projections:
            p.lora_a.grad = None
            p.lora_b.grad = None
        for x in xs:
            x.grad = None
        return layer.step(xs, gs)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        eager = [o.detach().clone() for o in step(small_x, small_g)]
        step(small_x, small_g)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        graph_out = step(small_x, small_g)
    with torch.cuda.stream(s):
        step(big_x, big_g)   # grows the stream's rank-16 workspace
    torch.cuda.synchronize()
    scribble = [torch.full((1 << 22,), 255, dtype=torch.uint8, device=device) for _ in range(8)]
    for replay in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(graph_out, eager)):
            assert torch.equal(a, b), f"replay {replay}: output {i} differs"
    del scribble


def test_decoder_layer_graph_replay_matches_eager(device):
    """The whole decoder layer (norms, seven QLoRA projections, RoPE, packed causal
    attention, SwiGLU, residual adds) captured as one HIP graph, as bench.py times it:
    every replay, with unrelated eager work and synchronisations between replays,
    reproduces the eager step bit for bit -- output, input gradient and every LoRA
    gradient -- on the configs[1] batch."""
    from soupsuck_amd.layer import DecoderLayer

    lengths = [382, 242, 208, 158]
    layer = DecoderLayer(device, lengths)
    t = sum(lengths)
    gen = torch.Generator(device="cpu").manual_seed(3)
    h = torch.randn((t, 1536), generator=gen).half().to(device).requires_grad_()
    g = (torch.randn((t, 1536), generator=gen) * 0.05).half().to(device)

    def grads():
        out = [h.grad]
        for q in layer.proj.projections:
            out += [q.lora_a.grad, q.lora_b.grad]
        return out

    eager_out = layer.step(h, g).detach().clone()
    eager_grads = [x.clone() for x in grads()]

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            layer.step(h, g)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        graph_out = layer.step(h, g)
    graph_grads = grads()

    noise = torch.randn((512, 512), device=device)
    for replay in range(3):
        graph_out.detach().zero_()   # same storage; the replay must rewrite it
        for x in graph_grads:
            x.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(graph_out.detach(), eager_out), f"replay {replay}: output differs"
        for i, (a, b) in enumerate(zip(graph_grads, eager_grads)):
            assert torch.equal(a, b), f"replay {replay}: gradient {i} differs"
        noise = noise @ noise.t() / 512.0   # unrelated eager work between replays
        torch.cuda.synchronize()
