"""Joint q/k rotary position embedding (Qwen2 ``apply_rotary_pos_emb``).

Mirrors the reference's solution/kernels/rope.py:101-152 (``_RoPE`` and
``fused_rope``) and solution/rope.py:55-80 (``patch_qwen2_rope``): q [B, Hq,
S, D] and k [B, Hk, S, D] with any batch / head / token strides (e.g. the
transposed projection views), cos / sin [1|B, S, D] detached; outputs are
contiguous in promote(x, cos); every product is rounded to the output dtype
before the add (eager PyTorch's order), the backward rounds products to the
input dtype.  Kernels: ss_rope_fwd / ss_rope_bwd.  Saves only cos and sin.
"""

import torch
from torch.autograd.function import once_differentiable

from .. import _lib

_DTYPES = (torch.float16, torch.float32)


def rope_supported(q, k, cos, sin, unsqueeze_dim=1):
    tensors = (q, k, cos, sin)
    if not all(isinstance(t, torch.Tensor) for t in tensors) or unsqueeze_dim != 1:
        return False
    if not q.is_cuda or any(t.device != q.device for t in tensors):
        return False
    if q.ndim != 4 or k.ndim != 4 or cos.ndim != 3 or sin.shape != cos.shape:
        return False
    b, _, s, d = q.shape
    if d % 2 or k.shape[0] != b or k.shape[2:] != (s, d) or cos.shape[1:] != (s, d):
        return False
    if cos.shape[0] not in (1, b) or cos.requires_grad or sin.requires_grad:
        return False
    if any(t.dtype not in _DTYPES for t in tensors) or cos.dtype != sin.dtype:
        return False
    return all(t.stride(-1) == 1 for t in tensors)


def _cs_args(cos, sin):
    return (cos.data_ptr(), sin.data_ptr(), _lib.dtype_code(cos.dtype), cos.stride(0),
            cos.stride(1), sin.stride(0), sin.stride(1), cos.shape[0])


class _RoPE(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, cos, sin):
        b, hq, s, d = q.shape
        hk = k.shape[1]
        yq = torch.empty(q.shape, device=q.device, dtype=torch.promote_types(q.dtype, cos.dtype))
        yk = torch.empty(k.shape, device=k.device, dtype=torch.promote_types(k.dtype, cos.dtype))
        if b and s and hq + hk:
            _lib.call("ss_rope_fwd", q.data_ptr(), _lib.dtype_code(q.dtype), *q.stride()[:3],
                      k.data_ptr(), _lib.dtype_code(k.dtype), *k.stride()[:3],
                      *_cs_args(cos, sin), yq.data_ptr(), _lib.dtype_code(yq.dtype),
                      yk.data_ptr(), _lib.dtype_code(yk.dtype), b, hq, hk, s, d // 2,
                      _lib.stream(q.device))
        ctx.save_for_backward(cos, sin)
        ctx.qshape, ctx.kshape, ctx.qdtype, ctx.kdtype = q.shape, k.shape, q.dtype, k.dtype
        ctx.set_materialize_grads(False)
        frozen = tuple(o for o, req in zip((yq, yk), ctx.needs_input_grad[:2]) if not req)
        if frozen:
            ctx.mark_non_differentiable(*frozen)
        return yq, yk

    @staticmethod
    @once_differentiable
    def backward(ctx, gq, gk):
        cos, sin = ctx.saved_tensors
        b, hq, s, d = ctx.qshape
        hk = ctx.kshape[1]
        need_q = gq is not None and ctx.needs_input_grad[0]
        need_k = gk is not None and ctx.needs_input_grad[1]
        dq = torch.empty(ctx.qshape, device=cos.device, dtype=ctx.qdtype) if need_q else None
        dk = torch.empty(ctx.kshape, device=cos.device, dtype=ctx.kdtype) if need_k else None
        if (need_q or need_k) and b and s and hq + hk:
            qs = gq.stride() if need_q else (0, 0, 0, 0)
            ks = gk.stride() if need_k else (0, 0, 0, 0)
            _lib.call("ss_rope_bwd", gq.data_ptr() if need_q else None,
                      _lib.dtype_code(gq.dtype) if need_q else 0, *qs,
                      gk.data_ptr() if need_k else None,
                      _lib.dtype_code(gk.dtype) if need_k else 0, *ks, *_cs_args(cos, sin),
                      _lib.ptr(dq), _lib.dtype_code(ctx.qdtype), _lib.ptr(dk),
                      _lib.dtype_code(ctx.kdtype), b, hq, hk, s, d // 2, _lib.stream(cos.device))
        return dq, dk, None, None


def fused_rope(q, k, cos, sin):
    """Rotate q / k on the GPU; cos / sin are detached [1|B, S, D] (rope.py:146-152)."""
    if not rope_supported(q, k, cos, sin):
        raise ValueError("Expected CUDA q/k[B,H,S,even D] and detached cos/sin[1|B,S,D], "
                         "last stride 1")
    with torch.cuda.device(q.device):
        return _RoPE.apply(q, k, cos, sin)


def patch_qwen2_rope(module=None):
    """Route modeling_qwen2.apply_rotary_pos_emb through fused_rope (idempotent)."""
    from ..patch import ROPE_ROUTE, install_route

    return install_route(ROPE_ROUTE, module)
