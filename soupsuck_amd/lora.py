"""QLoRA projection: frozen NF4 base GEMM + LoRA branch in one autograd node (A10-A12).

Forward (reference solution/lora.py:135-163 under CUDA fp16 autocast,
solution/kernels/lora_epilogue.py:24-34):
    result = fp16(X . Wdec^T + bias)                    ss_nf4_gemm_fwd
    Z      = fp16(drop(X) . A^T)                        ss_gemm_f16
    L      = fp16(Z . B^T)                              ss_gemm_f16
    out    = fp16(result + fp16(L * s))                 ss_lora_epilogue_fwd
Backward (reference solution/lora_pair.py:34-65 order, fp16 after each GEMM):
    dL = fp16(fp16(g) * s)                              ss_lora_epilogue_bwd
    dZ = fp16(dL . B),  dB = fp16(dL^T . Z),  dA = fp16(dZ^T . drop(X))
    dX = fp16(g . Wdec + mask * (dZ . A))               ss_nf4_gemm_dx, ss_gemm_f16
The frozen base contributes no weight gradient.

Fast path (rank 16, K % 64 == 0): two entry points per projection -- forward
ss_qlora_forward (Z, then the NF4 GEMM with the LoRA add in its epilogue; Z
runs in one launch with the NF4 decode); backward ss_qlora_backward (dZ from
fp16(g*s) and dB in one launch with the transposed decode, the dX GEMM
g.W + dZ.A in one accumulator, then dA).  With active dropout (p > 0,
training) the same steps run as ss_qlora_forward_dropout /
ss_qlora_backward_dropout: the keep mask of X is a counter-based (Philox)
function of a per-call seed drawn from torch's CPU generator, recomputed by
every kernel that reads X and never stored.  Its bits therefore differ from
those PEFT's own Dropout would draw from torch's CUDA RNG (same keep
probability and scaling, fp32(x) * fp32(1 / (1 - p)), as the reference's fp32
dropout; solution/lora.py:1-40).
Otherwise each GEMM and the epilogue run as separate kernels (torch's native
dropout on an fp32 copy of X for p > 0).  That is also the path of an active
dropout under HIP graph capture, where a seed fixed at capture would give
every replay the same mask, while torch's generator advances per replay.
"""

import contextlib
import math

import torch
from torch.autograd.function import once_differentiable

from . import _lib
from .kernels.nf4 import _validate_state
from .kernels.nf4_gemm import gemm_f16, nf4_dx_2d, nf4_forward_2d


def _nf4_args(packed, state):
    return (packed.data_ptr(), state.absmax.data_ptr(), state.state2.absmax.data_ptr(),
            state.state2.code.data_ptr(), state.offset.data_ptr())


def _on_device(device):
    """torch.cuda.device(device), or nothing when it is already the current device."""
    if device.index == torch.cuda.current_device():
        return contextlib.nullcontext()
    return torch.cuda.device(device)


_SIZES = {}


def _size_of(query, t, n, k, device):
    """Workspace size from the library (a pure function of the shape and the
    device's CU count), asked once per (query, shape, device)."""
    key = (query, t, n, k, device.index)
    size = _SIZES.get(key)
    if size is None:
        size = _SIZES[key] = int(getattr(_lib.load(), query)(t, n, k))
    return size


_GEMM_WORKSPACE = {}


def _gemm_ws(t, n, k, device, stream):
    """(workspace, bytes) of the NF4 GEMM for this shape: one buffer per (device, stream),
    grown on demand and reused by every call issued on that stream (calls on one stream
    run in order, and the workspace holds nothing between calls).  A buffer replaced by
    a larger one is kept alive, as the rank workspace's are, for HIP graphs captured
    with it."""
    size = _size_of("ss_nf4_gemm_workspace_size", t, n, k, device)
    if not size:
        return None, 0
    key = (device.index, stream)
    ws = _GEMM_WORKSPACE.get(key)
    if ws is None or ws.numel() < size:
        if ws is not None:
            _RETIRED_WORKSPACES.append(ws)
        grown = 2 * ws.numel() if ws is not None else 0
        ws = torch.empty(max(size, grown), dtype=torch.uint8, device=device)
        _GEMM_WORKSPACE[key] = ws
    return ws, ws.numel()


_CHECKED = {}


def _checked_state(packed, state):
    """(n, k, NF4 pointer arguments) of an accepted nested-NF4 state.  The full rule table
    runs once per (state, storage); later calls with the same objects and buffers (the
    frozen weight of a projection) reuse its verdict."""
    key = (id(state), id(packed), packed.data_ptr(), state.absmax.data_ptr(),
           state.state2.absmax.data_ptr(), state.state2.code.data_ptr(),
           state.offset.data_ptr())
    hit = _CHECKED.get(key)
    if hit is not None and hit[0] is state and hit[1] is packed:
        return hit[2]
    n, k = _validate_state(packed, state, torch.float16)
    verdict = (n, k, _nf4_args(packed, state))
    if len(_CHECKED) > 4096:
        _CHECKED.clear()
    _CHECKED[key] = (state, packed, verdict)
    return verdict


_RANK_WORKSPACE = {}
_RETIRED_WORKSPACES = []


def _rank_workspace(nbytes, device, stream=None):
    """Zero-filled workspace of the rank-16 ops, one per (device, stream), grown on demand.

    Its leading arrival counters must be zero when an op starts and the op
    leaves them zero, so one zero-filled buffer serves every call issued in
    order on one stream.  Calls on different streams can overlap in time, so
    each stream (torch's current stream at the call) gets its own buffer.  A
    buffer replaced by a larger one is kept alive, not released: a HIP graph
    captured on that stream still addresses it, and its replays must find
    the counters it left at zero, not whatever a later tensor wrote there.
    Growth at least doubles the size, so few buffers are ever retired.
    ``stream``: the raw stream handle when the caller already has it."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    key = (index, stream if stream is not None else _lib.stream(device))
    ws = _RANK_WORKSPACE.get(key)
    if ws is None or ws.numel() < nbytes:
        grown = 2 * ws.numel() if ws is not None else 0
        if ws is not None:
            _RETIRED_WORKSPACES.append(ws)
        ws = torch.zeros(max(int(nbytes), 1 << 16, grown), dtype=torch.uint8, device=device)
        _RANK_WORKSPACE[key] = ws
    return ws


def project16(a2d, w, w_kr, scale=None):
    """fp16 [M, 16] = A' . W (ss_lora_project); W is lora_A [16, K] or lora_B [N, 16]."""
    m, k = a2d.shape
    out = torch.empty((m, 16), device=a2d.device, dtype=torch.float16)
    size = _lib.load().ss_lora_workspace_size(m, 0)
    ws = _rank_workspace(size, a2d.device)
    _lib.call("ss_lora_project", a2d.data_ptr(), a2d.stride(0), m, k, w.data_ptr(), w.stride(0),
              int(w_kr), int(scale is not None), float(scale or 1.0), out.data_ptr(),
              ws.data_ptr(), ws.numel(), _lib.stream(a2d.device))
    return out


def grad16(p2d, q2d, transpose, scale=None):
    """fp16 P^T . Q' as [16, N] (or [N, 16] when transpose) (ss_lora_grad)."""
    t, n = q2d.shape
    out = torch.empty((n, 16) if transpose else (16, n), device=q2d.device, dtype=torch.float16)
    size = _lib.load().ss_lora_workspace_size(0, n)
    ws = _rank_workspace(size, q2d.device)
    _lib.call("ss_lora_grad", p2d.data_ptr(), p2d.stride(0), q2d.data_ptr(), q2d.stride(0), t, n,
              int(scale is not None), float(scale or 1.0), int(transpose), out.data_ptr(),
              ws.data_ptr(), ws.numel(), _lib.stream(q2d.device))
    return out


def _qlora_rank_ws(t, n, k, device, stream):
    return _rank_workspace(_size_of("ss_qlora_rank_workspace_size", t, n, k, device), device,
                           stream)


def _half(w):
    """fp16 contiguous copy of a LoRA weight (itself when it already is one)."""
    if w.dtype == torch.float16 and w.is_contiguous():
        return w
    return w.to(torch.float16).contiguous()


def _grads(ctx, dx, da, db):
    x_dtype, a_dtype, b_dtype = ctx.dtypes
    dx = dx.view(ctx.shape)
    return (dx if x_dtype == torch.float16 else dx.to(x_dtype),
            da if a_dtype == torch.float16 else da.to(a_dtype),
            db if b_dtype == torch.float16 else db.to(b_dtype))


class _QLoRAFused(torch.autograd.Function):
    """Rank-16 projection on the fused entry points: forward ss_qlora_forward (Z and the
    NF4 GEMM with the LoRA epilogue), backward ss_qlora_backward (dZ, dB, dX with the
    rank-16 update, dA); with a seed, the dropout variants of both (the keep mask is a
    Philox function of (seed, element of X), recomputed wherever X is used, so only the
    8-byte seed is saved for the backward).  ``nf4``: (n, k, NF4 pointer arguments) from
    _checked_state."""

    @staticmethod
    def forward(ctx, x, lora_a, lora_b, packed, state, bias, scaling, nf4, dropout):
        n, k, w_args = nf4
        t = x.numel() // k
        x2d = x.view(t, k)
        a16, b16 = _half(lora_a), _half(lora_b)
        dev = x.device
        z = torch.empty((t, 16), device=dev, dtype=torch.float16)
        y = torch.empty((t, n), device=dev, dtype=torch.float16)
        stream = _lib.stream(dev)
        ws, size = _gemm_ws(t, n, k, dev, stream)
        rws = _qlora_rank_ws(t, n, k, dev, stream)
        head = (x2d.data_ptr(), k, t, *w_args, n, k, _lib.ptr(bias), a16.data_ptr(),
                b16.data_ptr(), scaling)
        tail = (z.data_ptr(), y.data_ptr(), n, _lib.ptr(ws), size, rws.data_ptr(), rws.numel(),
                stream)
        if dropout is None:
            _lib.call("ss_qlora_forward", *head, *tail)
        else:
            _lib.call("ss_qlora_forward_dropout", *head, dropout[0], dropout[1], *tail)
        ctx.save_for_backward(x2d, z, a16, b16)
        # the NF4 arguments are raw pointers: the reference keeps the weight alive
        ctx.packed, ctx.nf4, ctx.scaling, ctx.dropout = packed, nf4, scaling, dropout
        ctx.shape, ctx.dtypes = x.shape, (x.dtype, lora_a.dtype, lora_b.dtype)
        return y.view(*x.shape[:-1], n)

    @staticmethod
    @once_differentiable
    def backward(ctx, grad):
        x2d, z, a16, b16 = ctx.saved_tensors
        n, k, w_args = ctx.nf4
        t = x2d.shape[0]
        g = grad.reshape(t, n)
        if g.dtype != torch.float16 or not g.is_contiguous():
            g = g.to(torch.float16).contiguous()
        dev = g.device
        # dZ (used inside the call), dB and dA in one allocation; dX apart
        rank = torch.empty(t * 16 + n * 16 + 16 * k, device=dev, dtype=torch.float16)
        dz = rank[:t * 16]
        db = rank[t * 16:t * 16 + n * 16].view(n, 16)   # fp16(fp16(g*s)^T . Z)
        da = rank[t * 16 + n * 16:].view(16, k)          # fp16(dZ^T . X)
        dx = torch.empty((t, k), device=dev, dtype=torch.float16)
        stream = _lib.stream(dev)
        ws, size = _gemm_ws(t, n, k, dev, stream)
        rws = _qlora_rank_ws(t, n, k, dev, stream)
        head = (g.data_ptr(), n, t, *w_args, n, k, x2d.data_ptr(), k, z.data_ptr(),
                a16.data_ptr(), b16.data_ptr(), ctx.scaling)
        tail = (dx.data_ptr(), k, dz.data_ptr(), da.data_ptr(), db.data_ptr(), _lib.ptr(ws),
                size, rws.data_ptr(), rws.numel(), stream)
        if ctx.dropout is None:
            _lib.call("ss_qlora_backward", *head, *tail)
        else:
            _lib.call("ss_qlora_backward_dropout", *head, *ctx.dropout, *tail)
        return (*_grads(ctx, dx, da, db), None, None, None, None, None, None)


def dropout_seed():
    """A 64-bit seed for one dropout call, drawn from torch's default CPU generator (so
    torch.manual_seed makes the masks reproducible)."""
    return int(torch.empty((), dtype=torch.int64).random_().item())


class _QLoRAProjection(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, lora_a, lora_b, packed, state, bias, scaling, dropout_p, training):
        n, k = state.shape
        t = x.numel() // k
        x2d = x.reshape(t, k)
        stream = _lib.stream(x.device)
        result = nf4_forward_2d(x2d, packed, state, n, k, bias=bias)
        mask = None
        if dropout_p > 0.0 and training:
            # torch's own dropout (graph-safe RNG); its mask, not dropped != 0, so a kept
            # zero of X still passes its gradient
            dropped, mask = torch.native_dropout(x2d.float(), dropout_p, True)
            x_in = dropped.to(torch.float16)
        else:
            x_in = x2d
        a16 = lora_a.to(torch.float16).contiguous()
        b16 = lora_b.to(torch.float16).contiguous()
        z = gemm_f16(x_in, a16, b_trans=True)
        lora = gemm_f16(z, b16, b_trans=True)
        out = torch.empty_like(result)
        if t:
            _lib.call("ss_lora_epilogue_fwd", result.data_ptr(), _lib.F16, lora.data_ptr(),
                      _lib.F16, out.data_ptr(), _lib.F16, result.numel(), float(scaling), 0,
                      stream)
        ctx.save_for_backward(x_in, z, a16, b16, packed, mask)
        ctx.state, ctx.scaling, ctx.dropout_p = state, float(scaling), dropout_p
        ctx.shape, ctx.dtypes = x.shape, (x.dtype, lora_a.dtype, lora_b.dtype)
        return out.reshape(*x.shape[:-1], n)

    @staticmethod
    @once_differentiable
    def backward(ctx, grad):
        x_in, z, a16, b16, packed, mask = ctx.saved_tensors
        state = ctx.state
        n, k = state.shape
        t = x_in.shape[0]
        g = grad.reshape(t, n).to(torch.float16).contiguous()
        stream = _lib.stream(g.device)
        d_lora = torch.empty_like(g)
        if t:
            _lib.call("ss_lora_epilogue_bwd", g.data_ptr(), _lib.F16, d_lora.data_ptr(), _lib.F16,
                      g.numel(), ctx.scaling, stream)
        dz = gemm_f16(d_lora, b16)                          # [T, r]
        db = gemm_f16(d_lora, z, a_trans=True)              # [N, r]
        da = gemm_f16(dz, x_in, a_trans=True)               # [r, K]
        dx = nf4_dx_2d(g, packed, state, n, k)              # [T, K]
        if mask is None:
            gemm_f16(dz, a16, out=dx, accumulate=True)
        else:
            dx_lora = gemm_f16(dz, a16, out_dtype=torch.float32)
            dx_lora = dx_lora * mask / (1.0 - ctx.dropout_p)
            dx = (dx.float() + dx_lora).to(torch.float16)
        x_dtype, a_dtype, b_dtype = ctx.dtypes
        return (dx.reshape(ctx.shape).to(x_dtype), da.to(a_dtype), db.to(b_dtype),
                None, None, None, None, None, None)


def qlora_projection(x, lora_a, lora_b, packed, state, bias=None, scaling=2.0, dropout_p=0.0,
                     training=True):
    """out = X . Wdec^T + bias + scaling * (drop(X) . A^T) . B^T with NF4 W (fp16 compute)."""
    nf4 = _checked_state(packed, state)
    n, k = nf4[0], nf4[1]
    if x.dtype != torch.float16 or not x.is_cuda or x.shape[-1] != k or not x.is_contiguous():
        raise ValueError("Expected contiguous CUDA fp16 X[..., K]")
    if lora_a.ndim != 2 or lora_b.ndim != 2 or lora_a.shape[1] != k or lora_b.shape[0] != n \
            or lora_a.shape[0] != lora_b.shape[1]:
        raise ValueError("Expected lora_A [r, K] and lora_B [N, r]")
    if bias is not None and (bias.dtype != torch.float16 or bias.shape != (n,)
                             or not bias.is_contiguous()):
        raise ValueError("Expected fp16 bias[N]")
    if not math.isfinite(scaling):
        raise ValueError("scaling must be finite")
    if not 0.0 <= dropout_p < 1.0:
        raise ValueError("dropout_p must be in [0, 1)")
    fused = lora_a.shape[0] == 16 and k % 64 == 0 and packed.data_ptr() % 16 == 0
    active = dropout_p > 0.0 and training
    with _on_device(x.device):
        if fused and not active:
            return _QLoRAFused.apply(x, lora_a, lora_b, packed, state, bias, float(scaling), nf4,
                                     None)
        # The fused dropout's seed is a kernel argument: a HIP graph would replay one mask
        # forever, so under capture the mask comes from torch's graph-safe generator.
        if fused and x.data_ptr() % 16 == 0 and not torch.cuda.is_current_stream_capturing():
            return _QLoRAFused.apply(x, lora_a, lora_b, packed, state, bias, float(scaling), nf4,
                                     (dropout_seed(), float(dropout_p)))
        return _QLoRAProjection.apply(x, lora_a, lora_b, packed, state, bias, float(scaling),
                                      float(dropout_p), bool(training))
