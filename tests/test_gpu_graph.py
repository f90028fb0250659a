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
