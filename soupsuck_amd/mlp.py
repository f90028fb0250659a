"""Frozen Qwen2 MLP on NF4 projections with the SwiGLU fused into the GEMMs.

Interface of the reference's solution/mlp.py:579-612 (``fused_qwen2_mlp``,
``patch_qwen2_mlp_fused``) over its node's semantics (:500-576): down(silu(gate(x)) * up(x))
for frozen bias-free NF4 Linear4bit projections, as one autograd node that
keeps gate and up (fp16) for the backward, or only x with ``recompute=True``
(gate and up are recomputed in the backward).  Kernels per direction:

  forward   gate = X Wg^T                         ss_nf4_gemm_fwd
            up, act = X Wu^T, silu(gate) * up     ss_nf4_gemm_fwd + ss_swiglu_fwd
                                                  (or ss_nf4_gemm_fwd_swiglu)
            out = act Wd^T                        ss_nf4_gemm_fwd
  backward  dgate, dup from dact = dY Wd          ss_nf4_gemm_dx + ss_swiglu_bwd
                                                  (or ss_nf4_gemm_dx_swiglu)
            dX = dgate Wg + dup Wu                ss_nf4_gemm_dx (twice, the
                                                  second accumulating in fp32)

The activation in the GEMM epilogue (the ``*_swiglu`` entry points,
``fuse=True``) gives bit-identical results; it is off by default
because it measured slower (see ``GLU_IN_EPILOGUE``).

Numerics follow the reference's node (bnb fp16 projections, the fp32 SwiGLU
tile engine of solution/kernels/swiglu_fused.py): every projection output is
rounded to fp16 before the activation reads it.  One difference: the two
input-gradient products are summed as fp16(fp16(dgate Wg) + fp32(dup Wu))
instead of two fp16 results added in fp16 (one rounding fewer).

``offload=True`` keeps the saved gate and up in pinned host memory instead of
HBM (the reference's pinned-host offload, solution/mlp.py:105-359): the
device-to-host copies run on a copy stream of default priority after the
producing stream; the copy back runs on that stream too and the backward waits
for it.  A node's restore also starts the copy back of the node created before
it (a lookahead of one: in a backward it is the next to restore), so that copy
overlaps the current node's backward.  The pinned buffers come in power-of-two
row classes and return to a free list once their copy back has completed.  The
default is off (``SOUP_MLP_OFFLOAD=1`` turns it on; the reference defaults to on):
with 288 GB of HBM per MI355X the activations fit, and the round trip costs PCIe
time.  Recomputation excludes offload, as in the reference.  Offload is refused
under HIP graph capture.

Per-layer placement (solution/mlp.py:362-431): ``SOUP_MLP_RECOMPUTE_LAYERS=k``
recomputes in the first k MLP layers, ``SOUP_EXP_OFFLOAD_TAIL=k`` keeps the last
k layers' gate / up on the device when offload is on, and
``prepare_mlp_offload(model, max_rows)`` numbers the layers and reserves their
pinned pairs up front.
"""

import os
import threading
import weakref

import torch
from torch.autograd.function import once_differentiable

from . import _lib
from .kernels.nf4 import _validate_state
from .kernels.nf4_gemm import nf4_dx_2d, nf4_forward_2d
from .kernels.swiglu import swiglu_fused_backward, swiglu_fused_forward


def _nf4(module):
    """(packed, state, n, k) of a frozen bias-free NF4 Linear4bit, else None."""
    weight = getattr(module, "weight", None)
    state = getattr(weight, "quant_state", None)
    if state is None or getattr(module, "bias", None) is not None:
        return None
    if weight.requires_grad or module._forward_hooks or module._forward_pre_hooks:
        return None
    packed = weight.data if isinstance(weight, torch.nn.Parameter) else weight
    try:
        n, k = _validate_state(packed, state, torch.float16)
    except ValueError:
        return None
    if k % 64 or packed.data_ptr() % 16:
        return None
    return packed, state, n, k


def _projections(mlp):
    parts = [_nf4(getattr(mlp, name, None)) for name in ("gate_proj", "up_proj", "down_proj")]
    return None if any(p is None for p in parts) else parts


def eligible_mlp(mlp, x):
    """Frozen bias-free NF4 gate/up/down of matching shapes on x's device, SiLU, CUDA fp16/fp32 x."""
    if not isinstance(x, torch.Tensor) or not x.is_cuda or x.dtype not in (torch.float16,
                                                                          torch.float32):
        return False
    act = getattr(getattr(mlp, "config", None), "hidden_act", "silu")
    if act != "silu":
        return False
    parts = _projections(mlp)
    if parts is None:
        return False
    (_, _, ng, kg), (_, _, nu, ku), (_, _, nd, kd) = parts
    return (kg == ku == nd == x.shape[-1] and ng == nu == kd
            and all(p[0].device == x.device for p in parts))


def _workspace(t, n, k, device):
    size = _lib.load().ss_nf4_gemm_workspace_size(t, n, k)
    ws = torch.empty(max(size, 1), dtype=torch.uint8, device=device) if size else None
    return ws, size


def _state_args(packed, state):
    return (packed.data_ptr(), state.absmax.data_ptr(), state.state2.absmax.data_ptr(),
            state.state2.code.data_ptr(), state.offset.data_ptr())


# Where the SwiGLU runs by default: its own HBM-bound kernels (False) or the
# GEMM epilogues (True; bit-identical).  Measured on MI355X at the configs[1]
# shapes (T = 990): alone, the down dX with the activation in its epilogue takes
# 66-70 us against 54-59 + 17 us for the product and the kernel; inside the
# whole MLP step the epilogue variant measured 398-414 us against 386-401 us in
# the same runs (every output tile reaches its epilogue at once, so the extra
# gate / up traffic there overlaps no MFMA work).  Callers choose per call with
# ``fuse=``.
GLU_IN_EPILOGUE = False


def gate_up_swiglu(x2d, gate_proj, up_proj, keep=True, fuse=None):
    """(gate, up, act) for x2d [T, H] fp16; gate/up are None unless ``keep``."""
    packed_g, state_g, n, k = gate_proj
    packed_u, state_u, _, _ = up_proj
    t = x2d.shape[0]
    gate = nf4_forward_2d(x2d, packed_g, state_g, n, k)
    if not (GLU_IN_EPILOGUE if fuse is None else fuse):
        up = nf4_forward_2d(x2d, packed_u, state_u, n, k)
        act = swiglu_fused_forward(gate, up)
        return (gate if keep else None), (up if keep else None), act
    act = torch.empty((t, n), device=x2d.device, dtype=torch.float16)
    up = torch.empty_like(act) if keep else None
    if t:
        ws, size = _workspace(t, n, k, x2d.device)
        _lib.call("ss_nf4_gemm_fwd_swiglu", x2d.data_ptr(), x2d.stride(0), t,
                  *_state_args(packed_u, state_u), n, k, gate.data_ptr(), gate.stride(0),
                  _lib.ptr(up), n, act.data_ptr(), n, _lib.ptr(ws), size,
                  _lib.stream(x2d.device))
    return (gate if keep else None), up, act


def down_dx_swiglu(dy2d, down_proj, gate, up, fuse=None):
    """(dgate, dup) from dact = dy2d . Wd, fp16 [T, I]."""
    packed, state, n, k = down_proj
    t = dy2d.shape[0]
    if not (GLU_IN_EPILOGUE if fuse is None else fuse):
        return swiglu_fused_backward(gate, up, nf4_dx_2d(dy2d, packed, state, n, k))
    dgate = torch.empty((t, k), device=dy2d.device, dtype=torch.float16)
    dup = torch.empty_like(dgate)
    if t:
        ws, size = _workspace(t, n, k, dy2d.device)
        _lib.call("ss_nf4_gemm_dx_swiglu", dy2d.data_ptr(), dy2d.stride(0), t,
                  *_state_args(packed, state), n, k, gate.data_ptr(), gate.stride(0),
                  up.data_ptr(), up.stride(0), dgate.data_ptr(), k, dup.data_ptr(), k,
                  _lib.ptr(ws), size, _lib.stream(dy2d.device))
    return dgate, dup


def mlp_forward_2d(x2d, parts, keep=True, fuse=None):
    """(out, gate, up) of the MLP on x2d [T, H] fp16 contiguous."""
    gate_p, up_p, down_p = parts
    gate, up, act = gate_up_swiglu(x2d, gate_p, up_p, keep, fuse)
    packed, state, n, k = down_p
    out = nf4_forward_2d(act, packed, state, n, k)
    return out, gate, up


def mlp_backward_2d(grad2d, parts, gate, up, fuse=None):
    """dX [T, H] fp16 of the MLP given the saved (or recomputed) gate and up."""
    gate_p, up_p, down_p = parts
    dgate, dup = down_dx_swiglu(grad2d, down_p, gate, up, fuse)
    dx = nf4_dx_2d(dgate, gate_p[0], gate_p[1], gate_p[2], gate_p[3])
    nf4_dx_2d(dup, up_p[0], up_p[1], up_p[2], up_p[3], out=dx, accumulate=True)
    return dx


_COPY_STREAMS = {}  # device index -> copy stream (default priority)
_HOST_FREE = {}     # (device index, capacity rows, width) -> free pinned (gate, up) pairs
_HOST_PENDING = []  # (event, key, pair): pairs whose copy back may still run


def _copy_stream(device):
    stream = _COPY_STREAMS.get(device.index)
    if stream is None:
        stream = _COPY_STREAMS[device.index] = torch.cuda.Stream(device=device)
    return stream


def _capacity(rows):
    """Pinned rows for `rows` of activations: the next power of two (at least 64), so
    that packed batches whose T changes every step reuse a few pairs."""
    return max(64, 1 << (max(rows, 1) - 1).bit_length())


def _host_pair(index, rows, width):
    """((gate, up) pinned pair, its key) holding at least `rows` x `width`: the free
    pair of the smallest capacity that fits, else a new one of _capacity(rows)."""
    still = []
    for event, k, pair in _HOST_PENDING:
        if event.query():
            _HOST_FREE.setdefault(k, []).append(pair)
        else:
            still.append((event, k, pair))
    _HOST_PENDING[:] = still
    fits = [k for k, free in _HOST_FREE.items()
            if free and k[0] == index and k[2] == width and k[1] >= rows]
    if fits:
        key = min(fits)
        return _HOST_FREE[key].pop(), key
    key = (index, _capacity(rows), width)
    return tuple(torch.empty(key[1:], dtype=torch.float16, pin_memory=True)
                 for _ in range(2)), key


_LAST_OFFLOAD = {}  # device index -> weakref to the newest HostOffload on that device
_OFFLOAD_LOCK = threading.Lock()  # forward (main thread) and backward (autograd thread)
PREFETCHES = [0]    # lookahead copies started (a counter the tests read)


class HostOffload:
    """gate and up of one MLP node held in pinned host memory until its backward.

    Nodes on a device are chained in creation order.  A backward runs them in the
    reverse order, so when a node restores its pair it also starts copying the pair
    of the node created before it back to the device on the copy stream (lookahead
    of one, the reference's prefetch chain, solution/mlp.py:203-252): that copy
    overlaps this node's backward and the next restore only waits for it."""

    def __init__(self, gate, up):
        device = gate.device
        self.device = device
        self.rows = gate.shape[0]
        self.prefetched = None  # (gate, up, ready event) once copied back
        with _OFFLOAD_LOCK:
            self.pair, self.key = _host_pair(device.index, self.rows, gate.shape[1])
            self.previous = _LAST_OFFLOAD.get(device.index)
            _LAST_OFFLOAD[device.index] = weakref.ref(self)
        producer = torch.cuda.current_stream(device)
        copy = _copy_stream(device)
        copy.wait_stream(producer)
        with torch.cuda.stream(copy):
            self.pair[0][:self.rows].copy_(gate, non_blocking=True)
            self.pair[1][:self.rows].copy_(up, non_blocking=True)
            self.stored = torch.cuda.Event()
            self.stored.record(copy)
        # The device tensors may be freed by the caller now: keep their memory
        # from being reused before the copy stream has read them.
        gate.record_stream(copy)
        up.record_stream(copy)

    def _fetch(self):
        """Copy the pair back to the device on the copy stream (caller holds the lock)."""
        copy = _copy_stream(self.device)
        with torch.cuda.stream(copy):
            copy.wait_event(self.stored)
            gate = self.pair[0][:self.rows].to(self.device, non_blocking=True)
            up = self.pair[1][:self.rows].to(self.device, non_blocking=True)
            ready = torch.cuda.Event()
            ready.record(copy)
        _HOST_PENDING.append((ready, self.key, self.pair))
        self.pair = None
        self.prefetched = (gate, up, ready)

    def restore(self):
        """(gate, up) back on the device, ordered on the current stream; starts the
        copy of the previous node's pair."""
        stream = torch.cuda.current_stream(self.device)
        with _OFFLOAD_LOCK:
            if self.prefetched is None:
                self._fetch()
            gate, up, ready = self.prefetched
            self.prefetched = None
            prev = self.previous() if self.previous is not None else None
            if prev is not None and prev.pair is not None:
                prev._fetch()
                PREFETCHES[0] += 1
        stream.wait_event(ready)
        # Allocated on the copy stream, read on this one from here on.
        gate.record_stream(stream)
        up.record_stream(stream)
        return gate, up


class _FrozenMLP(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, mlp, recompute, offload=False):
        parts = _projections(mlp)
        shape = x.shape
        x2d = x.reshape(-1, shape[-1]).to(torch.float16).contiguous()
        out, gate, up = mlp_forward_2d(x2d, parts, keep=not recompute)
        ctx.mlp, ctx.recompute, ctx.input_dtype, ctx.shape = mlp, recompute, x.dtype, shape
        ctx.offloaded = None
        if recompute:
            ctx.save_for_backward(x2d)
        elif offload:
            ctx.offloaded = HostOffload(gate, up)
            ctx.save_for_backward()
        else:
            ctx.save_for_backward(gate, up)
        return out.reshape(*shape[:-1], out.shape[-1]).to(x.dtype)

    @staticmethod
    @once_differentiable
    def backward(ctx, grad):
        parts = _projections(ctx.mlp)
        if parts is None:
            raise RuntimeError("MLP projections changed between forward and backward")
        grad2d = grad.reshape(-1, grad.shape[-1]).to(torch.float16).contiguous()
        if ctx.recompute:
            (x2d,) = ctx.saved_tensors
            gate = nf4_forward_2d(x2d, *parts[0])
            up = nf4_forward_2d(x2d, *parts[1])
        elif ctx.offloaded is not None:
            gate, up = ctx.offloaded.restore()
            ctx.offloaded = None
        else:
            gate, up = ctx.saved_tensors
        dx = mlp_backward_2d(grad2d, parts, gate, up)
        return dx.reshape(ctx.shape).to(ctx.input_dtype), None, None, None


# Per-layer placement of the saved activations (the reference's knobs,
# solution/mlp.py:360-430): SOUP_MLP_RECOMPUTE_LAYERS = k recomputes gate / up in the
# backward of the first k MLP layers; with offload on, SOUP_EXP_OFFLOAD_TAIL = k keeps
# the last k layers' gate / up on the device (their backward comes first).  A layer's
# index is its position in prepare_mlp_offload's module order, else its order of first
# forward among the MLPs sharing its config.
_LAYER_ORDER = {}  # id(config) -> WeakKeyDictionary(mlp -> index)


def _layer_index(mlp):
    index = getattr(mlp, "_soup_mlp_index", None)
    if index is not None:
        return index
    with _OFFLOAD_LOCK:
        for key in [k for k, group in _LAYER_ORDER.items() if not group]:
            del _LAYER_ORDER[key]
        group = _LAYER_ORDER.setdefault(id(getattr(mlp, "config", None)),
                                        weakref.WeakKeyDictionary())
        if mlp not in group:
            group[mlp] = len(group)
        return group[mlp]


def _layer_count(mlp):
    count = getattr(mlp, "_soup_mlp_count", None)
    if count is None:
        count = getattr(getattr(mlp, "config", None), "num_hidden_layers", None)
    return count


def _env_layers(name, mlp):
    """The layer count in environment variable `name` (0 when unset), checked against
    the model's depth."""
    value = os.environ.get(name, "0")
    try:
        k = int(value)
    except ValueError:
        raise ValueError(f"{name} must be a non-negative integer, got {value!r}") from None
    total = _layer_count(mlp)
    if k < 0 or (total is not None and k > total):
        raise ValueError(f"{name}={k} must be between 0 and the layer count ({total})")
    return k


def _recompute_layer(mlp):
    k = _env_layers("SOUP_MLP_RECOMPUTE_LAYERS", mlp)
    return k > 0 and _layer_index(mlp) < k


def _tail_layer(mlp):
    k = _env_layers("SOUP_EXP_OFFLOAD_TAIL", mlp)
    if k == 0:
        return False
    total = _layer_count(mlp)
    if total is None:
        raise ValueError("SOUP_EXP_OFFLOAD_TAIL needs the layer count: call "
                         "prepare_mlp_offload(model) first")
    return _layer_index(mlp) >= total - k


def _mlp_modules(model):
    names = ("gate_proj", "up_proj", "down_proj")
    return [m for m in model.modules() if all(hasattr(m, n) for n in names)]


def prepare_mlp_offload(model, max_rows=2048):
    """Number the model's MLP layers in module order and reserve, per (device, width),
    one pinned (gate, up) pair of `max_rows` capacity for every layer that will
    offload (neither recomputed nor kept by the tail policy), so steps of up to
    `max_rows` tokens allocate no pinned memory (solution/mlp.py:360-385)."""
    if max_rows < 1:
        raise ValueError("max_rows must be positive")
    layers = _mlp_modules(model)
    for index, layer in enumerate(layers):
        layer._soup_mlp_index = index
        layer._soup_mlp_count = len(layers)
    wanted = {}
    for layer in layers:
        device = layer.gate_proj.weight.device
        if device.type != "cuda" or os.environ.get("SOUP_MLP_RECOMPUTE") == "1":
            continue
        if _recompute_layer(layer) or _tail_layer(layer):
            continue
        key = (device.index, _capacity(max_rows), layer.gate_proj.out_features)
        wanted[key] = wanted.get(key, 0) + 1
    with _OFFLOAD_LOCK:
        for key, count in wanted.items():
            free = _HOST_FREE.setdefault(key, [])
            pending = sum(1 for _, k, _ in _HOST_PENDING if k == key)
            for _ in range(count - len(free) - pending):
                free.append(tuple(torch.empty(key[1:], dtype=torch.float16, pin_memory=True)
                                  for _ in range(2)))
    return len(layers)


def fused_qwen2_mlp(mlp, x, recompute=None, offload=None):
    """Run an eligible frozen NF4 MLP; raise ValueError otherwise (solution/mlp.py:579-612)."""
    if not eligible_mlp(mlp, x):
        raise ValueError("Expected frozen bias-free fp16 NF4 Linear4bit projections on CUDA")
    if recompute is None:
        recompute = os.environ.get("SOUP_MLP_RECOMPUTE") == "1" or _recompute_layer(mlp)
    if offload is None:
        offload = os.environ.get("SOUP_MLP_OFFLOAD") == "1"
    offload = bool(offload) and not recompute and not _tail_layer(mlp)
    if offload and torch.cuda.is_current_stream_capturing():
        raise ValueError("MLP activation offload cannot be captured in a HIP graph; "
                         "pass offload=False (or unset SOUP_MLP_OFFLOAD) for graph capture")
    with torch.cuda.device(x.device):
        if not torch.is_grad_enabled() or not x.requires_grad:
            shape = x.shape
            x2d = x.reshape(-1, shape[-1]).to(torch.float16).contiguous()
            out, _, _ = mlp_forward_2d(x2d, _projections(mlp), keep=False)
            return out.reshape(*shape[:-1], out.shape[-1]).to(x.dtype)
        return _FrozenMLP.apply(x, mlp, bool(recompute), offload)


def patch_qwen2_mlp_fused(module=None):
    """Route Qwen2MLP.forward through fused_qwen2_mlp for eligible modules (idempotent)."""
    from .patch import MLP_ROUTE, install_route

    return install_route(MLP_ROUTE, module)


def mlp_flops(t, hidden, inter):
    """Forward + backward (dX only) flops of the frozen MLP: 3 + 4 products of 2 t h i."""
    return 7 * 2 * t * hidden * inter


__all__ = ["fused_qwen2_mlp", "patch_qwen2_mlp_fused", "prepare_mlp_offload", "eligible_mlp",
           "gate_up_swiglu", "down_dx_swiglu", "mlp_forward_2d", "mlp_backward_2d", "mlp_flops",
           "HostOffload"]
