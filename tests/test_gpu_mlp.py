"""GPU parity of the frozen NF4 MLP with the SwiGLU in the GEMM epilogues.

* ss_nf4_gemm_fwd_swiglu / ss_nf4_gemm_dx_swiglu equal, bit for bit, the
  unfused composition (ss_nf4_gemm_fwd or _dx, then ss_swiglu_fwd or _bwd,
  both pinned against the oracles in their own tests) at T values that take
  each GEMM path: streaming (T <= 32), skinny (33-128), fused NF4 (129-256),
  decode-first + dense NT (larger T), at the configs[1] shapes
  (gate/up 8960 x 1536, down 1536 x 8960).
* fused_qwen2_mlp against the eager fp32 module on the decoded weights, with
  the reference's tolerance (solution/tests/test_mlp.py:12, 63-89): outputs
  and input gradients within rtol = atol = 2e-3, relative L2 error of dX
  <= 1e-2, for fp16 and fp32 inputs, with and without recompute.
"""

import pytest
import torch

from soupsuck_amd import _lib
from soupsuck_amd.bnb_compat import Linear4bit, dequantize_4bit, quantize_4bit
from soupsuck_amd.kernels.nf4_gemm import nf4_dx_2d, nf4_forward_2d
from soupsuck_amd.kernels.swiglu import swiglu_fused_backward, swiglu_fused_forward
from soupsuck_amd.mlp import down_dx_swiglu, fused_qwen2_mlp, gate_up_swiglu, patch_qwen2_mlp_fused

pytestmark = pytest.mark.gpu

HIDDEN, INTER = 1536, 8960


def _weight(n, k, seed, device):
    gen = torch.Generator(device=device).manual_seed(seed)
    w = (torch.randn((n, k), device=device, generator=gen) * 0.02).half()
    packed, state = quantize_4bit(w)
    return packed, state, n, k


@pytest.fixture(scope="module")
def weights(device):
    return {"gate": _weight(INTER, HIDDEN, 1, device), "up": _weight(INTER, HIDDEN, 2, device),
            "down": _weight(HIDDEN, INTER, 3, device)}


def _bits(t):
    return t.contiguous().view(torch.int16)


@pytest.mark.parametrize("t", [1, 16, 100, 200, 990, 2048])
def test_forward_swiglu_bitwise_equals_gemm_then_swiglu(device, weights, t):
    print(f"case fwd_swiglu T={t}", flush=True)
    gen = torch.Generator(device=device).manual_seed(t)
    x = torch.randn((t, HIDDEN), device=device, generator=gen).half()
    gate, up, act = gate_up_swiglu(x, weights["gate"], weights["up"], keep=True, fuse=True)
    up_ref = nf4_forward_2d(x, *weights["up"])
    act_ref = swiglu_fused_forward(gate, up_ref)
    assert torch.equal(_bits(up), _bits(up_ref))
    assert torch.equal(_bits(act), _bits(act_ref))
    _, none_up, act2 = gate_up_swiglu(x, weights["gate"], weights["up"], keep=False,
                                      fuse=True)
    assert none_up is None and torch.equal(_bits(act2), _bits(act_ref))


@pytest.mark.parametrize("t", [1, 16, 100, 200, 990, 2048])
def test_dx_swiglu_bitwise_equals_dx_then_swiglu(device, weights, t):
    print(f"case dx_swiglu T={t}", flush=True)
    gen = torch.Generator(device=device).manual_seed(100 + t)
    dy = torch.randn((t, HIDDEN), device=device, generator=gen).half()
    gate = (torch.randn((t, INTER), device=device, generator=gen) * 3).half()
    up = torch.randn((t, INTER), device=device, generator=gen).half()
    dgate, dup = down_dx_swiglu(dy, weights["down"], gate, up, fuse=True)
    dact = nf4_dx_2d(dy, *weights["down"])
    dg_ref, du_ref = swiglu_fused_backward(gate, up, dact)
    assert torch.equal(_bits(dgate), _bits(dg_ref))
    assert torch.equal(_bits(dup), _bits(du_ref))


class _MLP(torch.nn.Module):
    def __init__(self, hidden, inter):
        super().__init__()
        self.config = type("Cfg", (), {"hidden_act": "silu"})()
        self.gate_proj = Linear4bit(hidden, inter, bias=False, compute_dtype=torch.float16)
        self.up_proj = Linear4bit(hidden, inter, bias=False, compute_dtype=torch.float16)
        self.down_proj = Linear4bit(inter, hidden, bias=False, compute_dtype=torch.float16)


def _dense(proj):
    st = proj.weight.quant_state
    return dequantize_4bit(proj.weight.data, st).float()


@pytest.mark.parametrize("epilogue", ["0", "1"])
@pytest.mark.parametrize("recompute", [False, True])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("shape", [(2, 5, 128), (3, 77, 128)])
def test_fused_mlp_matches_fp32_module(device, monkeypatch, epilogue, recompute, dtype, shape):
    print(f"case mlp epilogue={epilogue} recompute={recompute} dtype={dtype} shape={shape}",
          flush=True)
    from soupsuck_amd import mlp as fmlp

    monkeypatch.setattr(fmlp, "GLU_IN_EPILOGUE", epilogue == "1")
    torch.manual_seed(777)
    mlp = _MLP(128, 320).to(device)
    x = torch.randn(shape, device=device, dtype=dtype, requires_grad=True)
    out = fused_qwen2_mlp(mlp, x, recompute)
    assert out.dtype == dtype and out.shape == shape
    wg, wu, wd = (_dense(p) for p in (mlp.gate_proj, mlp.up_proj, mlp.down_proj))
    rx = x.detach().float().requires_grad_()
    ref = torch.nn.functional.linear(
        torch.nn.functional.silu(rx @ wg.t()) * (rx @ wu.t()), wd)
    torch.testing.assert_close(out.float(), ref, rtol=2e-3, atol=2e-3)
    upstream = torch.randn_like(out)
    out.backward(upstream)
    ref.backward(upstream.float())
    assert x.grad.dtype == dtype
    torch.testing.assert_close(x.grad.float(), rx.grad, rtol=2e-3, atol=2e-3)
    rel = (x.grad.float() - rx.grad).norm() / rx.grad.norm()
    assert rel.item() <= 1e-2


def test_offload_keeps_gate_up_on_host_and_matches_bitwise(device):
    """offload=True: the saved gate / up live in pinned host memory between
    forward and backward (no device tensors saved), the gradient equals the
    on-device node's bit for bit, and a second step reuses the pinned pair."""
    from soupsuck_amd import mlp as fmlp

    torch.manual_seed(778)
    mlp = _MLP(128, 320).to(device)
    x = torch.randn((3, 77, 128), device=device, dtype=torch.float16)
    upstream = torch.randn((3, 77, 128), device=device, dtype=torch.float16)
    # 231 rows take a pair of the 256-row capacity class.
    key = (device.index if device.index is not None else torch.cuda.current_device(), 256, 320)

    def pooled():
        torch.cuda.synchronize()
        return len(fmlp._HOST_FREE.get(key, [])) + sum(1 for _, k, _ in fmlp._HOST_PENDING
                                                        if k == key)

    before = pooled()
    grads = []
    for offload in (False, True, True):
        xi = x.clone().requires_grad_()
        out = fused_qwen2_mlp(mlp, xi, recompute=False, offload=offload)
        node = out.grad_fn
        if offload:
            assert len(node.saved_tensors) == 0
            pair = node.offloaded.pair if hasattr(node, "offloaded") else None
            assert pair is None or all(t.is_pinned() and not t.is_cuda for t in pair)
        out.backward(upstream)
        grads.append((out.detach().clone(), xi.grad.clone()))
        torch.cuda.synchronize()  # the copy back has finished: its pair is free again
    for out, grad in grads[1:]:
        assert torch.equal(_bits(out), _bits(grads[0][0]))
        assert torch.equal(_bits(grad), _bits(grads[0][1]))
    # The second offloaded step took the pair the first one returned.
    assert pooled() == max(before, 1)
    # Recomputation excludes offload.
    out = fused_qwen2_mlp(mlp, x.clone().requires_grad_(), recompute=True, offload=True)
    assert out.grad_fn.offloaded is None


def test_offload_prefetches_the_previous_node_during_backward(device):
    """Two offloaded MLP nodes in a row: restoring the second (first in the backward)
    starts the copy back of the first one's pair on the copy stream; the gradients equal
    the on-device nodes' bit for bit."""
    from soupsuck_amd import mlp as fmlp

    torch.manual_seed(779)
    m1, m2 = _MLP(128, 320).to(device), _MLP(128, 320).to(device)
    x = torch.randn((2, 90, 128), device=device, dtype=torch.float16)
    upstream = torch.randn((2, 90, 128), device=device, dtype=torch.float16)
    results = []
    for offload in (False, True):
        xi = x.clone().requires_grad_()
        h = fused_qwen2_mlp(m1, xi, recompute=False, offload=offload)
        out = fused_qwen2_mlp(m2, h, recompute=False, offload=offload)
        first = h.grad_fn.offloaded
        before = fmlp.PREFETCHES[0]
        out.backward(upstream)
        torch.cuda.synchronize()
        if offload:
            assert fmlp.PREFETCHES[0] >= before + 1
            assert first is not None and first.pair is None  # copied back ahead of need
        results.append((out.detach().clone(), xi.grad.clone()))
    assert torch.equal(_bits(results[0][0]), _bits(results[1][0]))
    assert torch.equal(_bits(results[0][1]), _bits(results[1][1]))


class _Stack(torch.nn.Module):
    def __init__(self, depth):
        super().__init__()
        self.layers = torch.nn.ModuleList([_MLP(128, 320) for _ in range(depth)])

    def forward(self, x):
        for layer in self.layers:
            x = x + fused_qwen2_mlp(layer, x)
        return x


def test_layer_policy_recompute_offload_and_tail(device, monkeypatch):
    """Four prepared layers under SOUP_MLP_OFFLOAD=1, SOUP_MLP_RECOMPUTE_LAYERS=1 and
    SOUP_EXP_OFFLOAD_TAIL=1: layer 0 saves only its input, layers 1-2 keep gate / up
    in pinned pairs reserved by prepare_mlp_offload (taken, not allocated, for a
    smaller T), layer 3 keeps them on the device; the step's output and input
    gradient equal the all-on-device step's bit for bit (solution/mlp.py:362-431)."""
    from soupsuck_amd import mlp as fmlp

    torch.manual_seed(780)
    model = _Stack(4).to(device)
    x = torch.randn((2, 60, 128), device=device, dtype=torch.float16)
    upstream = torch.randn_like(x)

    xi = x.clone().requires_grad_()
    ref_out = model(xi)
    ref_out.backward(upstream)
    ref_grad = xi.grad.clone()
    monkeypatch.setenv("SOUP_MLP_OFFLOAD", "1")
    monkeypatch.setenv("SOUP_MLP_RECOMPUTE_LAYERS", "1")
    monkeypatch.setenv("SOUP_EXP_OFFLOAD_TAIL", "1")
    torch.cuda.synchronize()
    monkeypatch.setattr(fmlp, "_HOST_FREE", {})  # a pool of this test's own
    monkeypatch.setattr(fmlp, "_HOST_PENDING", [])
    index = device.index if device.index is not None else torch.cuda.current_device()
    assert fmlp.prepare_mlp_offload(model, max_rows=256) == 4
    assert list(fmlp._HOST_FREE) == [(index, 256, 320)]
    reserved = {p[0].data_ptr() for p in fmlp._HOST_FREE[(index, 256, 320)]}
    assert len(reserved) == 2

    xi = x.clone().requires_grad_()
    h = [xi]
    for layer in model.layers:
        h.append(h[-1] + fused_qwen2_mlp(layer, h[-1]))
    nodes = [t.grad_fn.next_functions[1][0] for t in h[1:]]
    assert all("FrozenMLP" in type(n).__name__ for n in nodes)
    assert [n.recompute for n in nodes] == [True, False, False, False]
    assert [n.offloaded is not None for n in nodes] == [False, True, True, False]
    assert [len(n.saved_tensors) for n in nodes] == [1, 0, 0, 2]
    # 120 rows fit the reserved 256-row pairs: no pinned allocation.
    assert all(n.offloaded.pair[0].data_ptr() in reserved for n in nodes[1:3])
    h[-1].backward(upstream)
    torch.cuda.synchronize()
    assert torch.equal(_bits(h[-1].detach()), _bits(ref_out.detach()))
    assert torch.equal(_bits(xi.grad), _bits(ref_grad))


def test_rejects_ineligible_modules(device):
    mlp = _MLP(128, 320).to(device)
    mlp.down_proj = torch.nn.Linear(320, 128, bias=False).to(device).half()
    x = torch.randn((2, 128), device=device, dtype=torch.float16)
    with pytest.raises(ValueError):
        fused_qwen2_mlp(mlp, x)


def test_patched_qwen2_mlp_routes_through_the_fused_node(device):
    modeling = pytest.importorskip("transformers.models.qwen2.modeling_qwen2")
    config = modeling.Qwen2Config(hidden_size=128, intermediate_size=320, hidden_act="silu")
    layer = modeling.Qwen2MLP(config)
    for name, (i, o) in {"gate_proj": (128, 320), "up_proj": (128, 320),
                         "down_proj": (320, 128)}.items():
        setattr(layer, name, Linear4bit(i, o, bias=False, compute_dtype=torch.float16))
    layer = layer.to(device)
    x = torch.randn((2, 9, 128), device=device, dtype=torch.float16, requires_grad=True)
    original = modeling.Qwen2MLP.forward
    expected = original(layer, x)
    assert patch_qwen2_mlp_fused(modeling)
    try:
        assert modeling.Qwen2MLP.forward is not original
        actual = layer(x)
        assert actual.grad_fn is not None and "FrozenMLP" in type(actual.grad_fn).__name__
    finally:
        modeling.Qwen2MLP.forward = original
    torch.testing.assert_close(actual, expected, rtol=2e-3, atol=2e-3)
    assert _lib.load() is not None


def test_mlp_graph_replay_matches_eager(device):
    """The frozen NF4 MLP node forward + backward at the configs[1] shapes (T = 990,
    1536 -> 8960 -> 1536) captured as one HIP graph: every replay, with unrelated eager
    work between replays, reproduces the eager output and input gradient bit for bit."""
    torch.manual_seed(781)
    mlp = _MLP(HIDDEN, INTER).to(device)
    x = torch.randn((990, HIDDEN), device=device, dtype=torch.float16).requires_grad_()
    upstream = torch.randn((990, HIDDEN), device=device, dtype=torch.float16)

    def step():
        x.grad = None
        out = fused_qwen2_mlp(mlp, x, recompute=False, offload=False)
        out.backward(upstream)
        return out

    eager_out = step().detach().clone()
    eager_grad = x.grad.clone()
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
    graph_grad = x.grad
    noise = torch.randn((512, 512), device=device)
    for replay in range(3):
        graph_out.detach().zero_()
        graph_grad.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(graph_out.detach(), eager_out), f"replay {replay}: output differs"
        assert torch.equal(graph_grad, eager_grad), f"replay {replay}: gradient differs"
        noise = noise @ noise.t() / 512.0
        torch.cuda.synchronize()
