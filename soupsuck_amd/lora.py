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


def _workspace(nbytes, device):
    return torch.empty(max(int(nbytes), 16), dtype=torch.uint8, device=device)


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


def _gemm_ws(t, n, k, device):
    size = _size_of("ss_nf4_gemm_workspace_size", t, n, k, device)
    return (_workspace(size, device), size) if size else (None, 0)


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


class _QLoRAFused(torch.autograd.Function):
    """Rank-16, dropout-free projection on the fused entry points: forward
    ss_qlora_forward (Z and the NF4 GEMM with the LoRA epilogue), backward
    ss_qlora_backward (dZ, dB, dX with the rank-16 update, dA)."""

    @staticmethod
    def forward(ctx, x, lora_a, lora_b, packed, state, bias, scaling):
        n, k = state.shape
        t = x.numel() // k
        x2d = x.reshape(t, k)
        a16 = lora_a.to(torch.float16).contiguous()
        b16 = lora_b.to(torch.float16).contiguous()
        z = torch.empty((t, 16), device=x.device, dtype=torch.float16)
        y = torch.empty((t, n), device=x.device, dtype=torch.float16)
        stream = _lib.stream(x.device)
        ws, size = _gemm_ws(t, n, k, x.device)
        rws = _qlora_rank_ws(t, n, k, x.device, stream)
        _lib.call("ss_qlora_forward", x2d.data_ptr(), x2d.stride(0), t, *_nf4_args(packed, state),
                  n, k, _lib.ptr(bias), a16.data_ptr(), b16.data_ptr(), float(scaling),
                  z.data_ptr(), y.data_ptr(), y.stride(0), _lib.ptr(ws), size, rws.data_ptr(),
                  rws.numel(), stream)
        ctx.save_for_backward(x2d, z, a16, b16, packed)
        ctx.state, ctx.scaling = state, float(scaling)
        ctx.shape, ctx.dtypes = x.shape, (x.dtype, lora_a.dtype, lora_b.dtype)
        return y.reshape(*x.shape[:-1], n)

    @staticmethod
    @once_differentiable
    def backward(ctx, grad):
        x2d, z, a16, b16, packed = ctx.saved_tensors
        state = ctx.state
        n, k = state.shape
        t = x2d.shape[0]
        g = grad.reshape(t, n).to(torch.float16).contiguous()
        dev = g.device
        dz = torch.empty((t, 16), device=dev, dtype=torch.float16)   # fp16(fp16(g*s) . B)
        db = torch.empty((n, 16), device=dev, dtype=torch.float16)   # fp16(fp16(g*s)^T . Z)
        da = torch.empty((16, k), device=dev, dtype=torch.float16)   # fp16(dZ^T . X)
        dx = torch.empty((t, k), device=dev, dtype=torch.float16)
        stream = _lib.stream(dev)
        ws, size = _gemm_ws(t, n, k, dev)
        rws = _qlora_rank_ws(t, n, k, dev, stream)
        _lib.call("ss_qlora_backward", g.data_ptr(), g.stride(0), t, *_nf4_args(packed, state), n,
                  k, x2d.data_ptr(), x2d.stride(0), z.data_ptr(), a16.data_ptr(), b16.data_ptr(),
                  ctx.scaling, dx.data_ptr(), dx.stride(0), dz.data_ptr(), da.data_ptr(),
                  db.data_ptr(), _lib.ptr(ws), size, rws.data_ptr(), rws.numel(),
                  stream)
        x_dtype, a_dtype, b_dtype = ctx.dtypes
        return (dx.reshape(ctx.shape).to(x_dtype), da.to(a_dtype), db.to(b_dtype),
                None, None, None, None)


def dropout_seed():
    """A 64-bit seed for one dropout call, drawn from torch's default CPU generator (so
    torch.manual_seed makes the masks reproducible)."""
    return int(torch.empty((), dtype=torch.int64).random_().item())


class _QLoRAFusedDropout(torch.autograd.Function):
    """Rank-16 projection with LoRA dropout p > 0 on the fused entry points
    (ss_qlora_forward_dropout / ss_qlora_backward_dropout): the keep mask is a
    Philox function of (seed, element of X), drawn again wherever it is used,
    so only the 8-byte seed is saved for the backward."""

    @staticmethod
    def forward(ctx, x, lora_a, lora_b, packed, state, bias, scaling, dropout_p, seed):
        n, k = state.shape
        t = x.numel() // k
        x2d = x.reshape(t, k)
        a16 = lora_a.to(torch.float16).contiguous()
        b16 = lora_b.to(torch.float16).contiguous()
        z = torch.empty((t, 16), device=x.device, dtype=torch.float16)
        y = torch.empty((t, n), device=x.device, dtype=torch.float16)
        stream = _lib.stream(x.device)
        ws, size = _gemm_ws(t, n, k, x.device)
        rws = _qlora_rank_ws(t, n, k, x.device, stream)
        _lib.call("ss_qlora_forward_dropout", x2d.data_ptr(), x2d.stride(0), t,
                  *_nf4_args(packed, state), n, k, _lib.ptr(bias), a16.data_ptr(),
                  b16.data_ptr(), float(scaling), seed, float(dropout_p), z.data_ptr(),
                  y.data_ptr(), y.stride(0), _lib.ptr(ws), size, rws.data_ptr(), rws.numel(),
                  stream)
        ctx.save_for_backward(x2d, z, a16, b16, packed)
        ctx.state, ctx.scaling, ctx.dropout = state, float(scaling), (seed, float(dropout_p))
        ctx.shape, ctx.dtypes = x.shape, (x.dtype, lora_a.dtype, lora_b.dtype)
        return y.reshape(*x.shape[:-1], n)

    @staticmethod
    @once_differentiable
    def backward(ctx, grad):
        x2d, z, a16, b16, packed = ctx.saved_tensors
        state = ctx.state
        n, k = state.shape
        t = x2d.shape[0]
        seed, p = ctx.dropout
        g = grad.reshape(t, n).to(torch.float16).contiguous()
        dev = g.device
        dz = torch.empty((t, 16), device=dev, dtype=torch.float16)
        db = torch.empty((n, 16), device=dev, dtype=torch.float16)
        da = torch.empty((16, k), device=dev, dtype=torch.float16)
        dx = torch.empty((t, k), device=dev, dtype=torch.float16)
        stream = _lib.stream(dev)
        ws, size = _gemm_ws(t, n, k, dev)
        rws = _qlora_rank_ws(t, n, k, dev, stream)
        _lib.call("ss_qlora_backward_dropout", g.data_ptr(), g.stride(0), t,
                  *_nf4_args(packed, state), n, k, x2d.data_ptr(), x2d.stride(0), z.data_ptr(),
                  a16.data_ptr(), b16.data_ptr(), ctx.scaling, seed, p, dx.data_ptr(),
                  dx.stride(0), dz.data_ptr(), da.data_ptr(), db.data_ptr(), _lib.ptr(ws), size,
                  rws.data_ptr(), rws.numel(), stream)
        x_dtype, a_dtype, b_dtype = ctx.dtypes
        return (dx.reshape(ctx.shape).to(x_dtype), da.to(a_dtype), db.to(b_dtype),
                None, None, None, None, None, None)


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
    n, k = _validate_state(packed, state, torch.float16)
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
            return _QLoRAFused.apply(x, lora_a, lora_b, packed, state, bias, float(scaling))
        # The fused dropout's seed is a kernel argument: a HIP graph would replay one mask
        # forever, so under capture the mask comes from torch's graph-safe generator.
        if fused and x.data_ptr() % 16 == 0 and not torch.cuda.is_current_stream_capturing():
            return _QLoRAFusedDropout.apply(x, lora_a, lora_b, packed, state, bias,
                                            float(scaling), float(dropout_p), dropout_seed())
        return _QLoRAProjection.apply(x, lora_a, lora_b, packed, state, bias, float(scaling),
                                      float(dropout_p), bool(training))
