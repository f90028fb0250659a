"""Joint q/k rotary position embedding (Qwen2 ``apply_rotary_pos_emb``).

Interface of the reference's ``fused_rope`` (solution/kernels/rope.py:146-152)
and its route (solution/rope.py:55-80): q [B, Hq, S, D] and k [B, Hk, S, D]
with any batch / head / token strides (the transposed projection views), and
detached cos / sin [1|B, S, D].  Results are contiguous in promote(x, cos);
every product is rounded to that dtype before the add (eager PyTorch's order),
and the backward -- the inverse rotation -- rounds its products to the input
dtype.  Kernels: ss_rope_fwd / ss_rope_bwd; only cos and sin are saved.

Accepted inputs are the rule table ROPE_RULES; ``fused_rope`` raises
ValueError with the first broken rule, ``rope_supported`` answers without
raising (the route's eligibility test).
"""

from typing import NamedTuple

import torch
from torch.autograd.function import once_differentiable

from .. import _lib
from ..contract import Rule, enforce, is_tensor

_DTYPES = (torch.float16, torch.float32)


def _same_cuda_device(a):
    return a.q.is_cuda and all(t.device == a.q.device for t in (a.k, a.cos, a.sin))


def _pair_shapes(a):
    q, k = a.q, a.k
    return (q.ndim == 4 and k.ndim == 4 and q.shape[-1] % 2 == 0
            and k.shape[0] == q.shape[0] and tuple(k.shape[2:]) == tuple(q.shape[2:]))


def _table_shape(a):
    b, _, s, d = a.q.shape
    return (a.cos.ndim == 3 and a.sin.shape == a.cos.shape and a.cos.shape[0] in (1, b)
            and tuple(a.cos.shape[1:]) == (s, d))


ROPE_RULES = (
    Rule("fused_rope: q, k, cos and sin must be tensors", lambda a: is_tensor(a.q, a.k, a.cos,
                                                                             a.sin)),
    Rule("fused_rope: heads must be dimension 1 (unsqueeze_dim=1)", lambda a: a.unsqueeze == 1),
    Rule("fused_rope: all four tensors must live on one CUDA device", _same_cuda_device),
    Rule("fused_rope: q and k must be [B, H, S, D] sharing B, S and an even D", _pair_shapes),
    Rule("fused_rope: cos and sin must both be [1 or B, S, D]", _table_shape),
    Rule("fused_rope: cos and sin must not require grad",
         lambda a: not (a.cos.requires_grad or a.sin.requires_grad)),
    Rule("fused_rope: dtypes must be fp16 or fp32, with cos and sin alike",
         lambda a: all(t.dtype in _DTYPES for t in (a.q, a.k, a.cos, a.sin))
         and a.cos.dtype == a.sin.dtype),
    Rule("fused_rope: the last dimension of every tensor must be dense (stride 1)",
         lambda a: all(t.stride(-1) == 1 for t in (a.q, a.k, a.cos, a.sin))),
)


def rope_supported(q, k, cos, sin, unsqueeze_dim=1):
    try:
        enforce(ROPE_RULES, q=q, k=k, cos=cos, sin=sin, unsqueeze=unsqueeze_dim)
    except ValueError:
        return False
    return True


class _Geometry(NamedTuple):
    batches: int
    qheads: int
    kheads: int
    tokens: int
    half: int

    @property
    def empty(self):
        return not (self.batches and self.tokens and self.qheads + self.kheads)


def _operand(t, strides):
    """(pointer, dtype code, strides...) of one [B, H, S, D] operand; zeros when absent."""
    if t is None:
        return (None, 0) + (0,) * strides
    return (t.data_ptr(), _lib.dtype_code(t.dtype)) + tuple(t.stride()[:strides])


def _table(cos, sin):
    return (cos.data_ptr(), sin.data_ptr(), _lib.dtype_code(cos.dtype), cos.stride(0),
            cos.stride(1), sin.stride(0), sin.stride(1), cos.shape[0])


def _target(t):
    return (_lib.ptr(t), _lib.dtype_code(t.dtype) if t is not None else 0)


def _strided_target(t):
    """(pointer, dtype code, batch / head / token strides) of a gradient output."""
    if t is None:
        return (None, 0, 0, 0, 0)
    return (t.data_ptr(), _lib.dtype_code(t.dtype)) + tuple(t.stride()[:3])


def _layout_of(shape, stride, dtype, device):
    """An uninitialised [B, H, S, D] tensor in the memory order of `stride` when that is
    a dense permutation with a unit last stride (a head-split view of a projection's
    [B, S, H * D] output), else contiguous: a gradient written that way reaches the
    projection's backward without a copy."""
    expect, dense = 1, stride[-1] == 1 or shape[-1] == 1
    for i in sorted(range(len(shape)), key=lambda i: stride[i]):
        if shape[i] != 1:
            dense = dense and stride[i] == expect
            expect *= shape[i]
    if dense:
        return torch.empty_strided(shape, stride, device=device, dtype=dtype)
    return torch.empty(shape, device=device, dtype=dtype)


class _RotaryPair(torch.autograd.Function):
    """Both rotations in one launch each way; the backward rotates by -theta."""

    @staticmethod
    def forward(ctx, q, k, cos, sin):
        geo = _Geometry(q.shape[0], q.shape[1], k.shape[1], q.shape[2], q.shape[3] // 2)
        outs = tuple(torch.empty(x.shape, device=x.device,
                                 dtype=torch.promote_types(x.dtype, cos.dtype)) for x in (q, k))
        if not geo.empty:
            _lib.call("ss_rope_fwd", *_operand(q, 3), *_operand(k, 3), *_table(cos, sin),
                      *_target(outs[0]), *_target(outs[1]), *geo, _lib.stream(q.device))
        ctx.save_for_backward(cos, sin)
        ctx.geo = geo
        ctx.inputs = ((q.shape, q.stride(), q.dtype), (k.shape, k.stride(), k.dtype))
        ctx.set_materialize_grads(False)
        # an output whose input takes no gradient carries none, as in eager PyTorch
        frozen = [y for y, wanted in zip(outs, ctx.needs_input_grad) if not wanted]
        if frozen:
            ctx.mark_non_differentiable(*frozen)
        return outs

    @staticmethod
    @once_differentiable
    def backward(ctx, gq, gk):
        cos, sin = ctx.saved_tensors
        grads, results = [], []
        for g, wanted, (shape, stride, dtype) in zip((gq, gk), ctx.needs_input_grad,
                                                     ctx.inputs):
            live = g is not None and wanted
            grads.append(g if live else None)
            results.append(_layout_of(shape, stride, dtype, cos.device) if live else None)
        if any(r is not None for r in results) and not ctx.geo.empty:
            _lib.call("ss_rope_bwd", *_operand(grads[0], 4), *_operand(grads[1], 4),
                      *_table(cos, sin), *_strided_target(results[0]),
                      *_strided_target(results[1]), *ctx.geo, _lib.stream(cos.device))
        return results[0], results[1], None, None


def fused_rope(q, k, cos, sin):
    """(q', k') rotated on the GPU; cos / sin detached [1|B, S, D] (rope.py:146-152)."""
    enforce(ROPE_RULES, q=q, k=k, cos=cos, sin=sin, unsqueeze=1)
    with torch.cuda.device(q.device):
        return _RotaryPair.apply(q, k, cos, sin)


def patch_qwen2_rope(module=None):
    """Route modeling_qwen2.apply_rotary_pos_emb through fused_rope (idempotent)."""
    from ..patch import ROPE_ROUTE, install_route

    return install_route(ROPE_ROUTE, module)
