"""Causal attention over packed rows (the attention of an unpadded batch).

Semantics of the reference's packed attention (solution/unpad.py:359-410): the
rows of a packed batch lie back to back on the token axis and each attends
causally to itself only, softmax(scale q.k) with GQA.  Here one launch covers
every row and head (ss_attn_varlen_fwd; backward ss_attn_varlen_bwd: dQ, then
dK / dV per q head, the GQA group's partials added in head order), instead of
one SDPA call per row.  fp16 in and out, fp32 softmax statistics.

Inputs follow Qwen2Attention's layout: q [1, Hq, T, 128], k / v [1, Hk, T, 128]
(any head / token strides with a unit last stride, e.g. the transposed
projection views); the output is [1, T, Hq, 128] contiguous, i.e. what
Qwen2Attention reshapes to [1, T, Hq * 128] for o_proj.
"""

import torch
from torch.autograd.function import once_differentiable

from .. import _lib
from ..contract import Rule, enforce

HEAD_DIM = 128


def row_offsets(lengths, device):
    """int32 cu_seqlens [rows + 1] on ``device`` from host row lengths (pinned, async copy)."""
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + int(n))
    host = torch.tensor(cu, dtype=torch.int32).pin_memory()
    return host.to(device, non_blocking=True)


def _aligned(t):
    return (t.data_ptr() % 16 == 0 and t.stride(-1) == 1 and t.stride(1) % 8 == 0
            and t.stride(2) % 8 == 0)


class PackedCausalAttention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, cu, max_len, scale):
        _, hq, total, d = q.shape
        hk = k.shape[1]
        rows = cu.numel() - 1
        o = torch.empty((1, total, hq, d), device=q.device, dtype=torch.float16)
        lse2 = torch.empty((hq, total), device=q.device, dtype=torch.float32)
        ov = o.transpose(1, 2)
        _lib.call("ss_attn_varlen_fwd", q.data_ptr(), q.stride(2), q.stride(1), k.data_ptr(),
                  k.stride(2), k.stride(1), v.data_ptr(), v.stride(2), v.stride(1),
                  cu.data_ptr(), rows, max_len, total, hq, hk, d, float(scale), o.data_ptr(),
                  ov.stride(2), ov.stride(1), lse2.data_ptr(), _lib.stream(q.device))
        ctx.save_for_backward(q, k, v, o, lse2, cu)
        ctx.shape_info = (max_len, float(scale))
        return o

    @staticmethod
    @once_differentiable
    def backward(ctx, grad):
        q, k, v, o, lse2, cu = ctx.saved_tensors
        max_len, scale = ctx.shape_info
        _, hq, total, d = q.shape
        hk = k.shape[1]
        g = grad.to(torch.float16)
        if not _aligned(g.transpose(1, 2)):
            g = g.contiguous()
        gv = g.transpose(1, 2)
        ov = o.transpose(1, 2)
        dq = torch.empty((1, total, hq, d), device=q.device, dtype=torch.float16)
        dk = torch.empty((1, total, hk, d), device=q.device, dtype=torch.float16)
        dv = torch.empty((1, total, hk, d), device=q.device, dtype=torch.float16)
        size = _lib.load().ss_attn_varlen_bwd_workspace_size(hq, hk, total)
        ws = torch.empty(max(size, 16), device=q.device, dtype=torch.uint8)
        dqv, dkv, dvv = dq.transpose(1, 2), dk.transpose(1, 2), dv.transpose(1, 2)
        _lib.call("ss_attn_varlen_bwd", q.data_ptr(), q.stride(2), q.stride(1), k.data_ptr(),
                  k.stride(2), k.stride(1), v.data_ptr(), v.stride(2), v.stride(1),
                  o.data_ptr(), ov.stride(2), ov.stride(1), g.data_ptr(), gv.stride(2),
                  gv.stride(1), lse2.data_ptr(), cu.data_ptr(), cu.numel() - 1, max_len, total,
                  hq, hk, d, scale, dq.data_ptr(), dqv.stride(2), dqv.stride(1), dk.data_ptr(),
                  dkv.stride(2), dkv.stride(1), dv.data_ptr(), dvv.stride(2), dvv.stride(1),
                  ws.data_ptr(), size, _lib.stream(q.device))
        return dqv, dkv, dvv, None, None, None


ATTENTION_RULES = (
    Rule("packed_causal_attention: q [1, Hq, T, 128] and k / v [1, Hk, T, 128] fp16 CUDA "
         "tensors on one device with Hq a multiple of Hk",
         lambda a: all(isinstance(t, torch.Tensor) and t.is_cuda and t.dtype == torch.float16
                       and t.ndim == 4 and t.shape[0] == 1 and t.shape[-1] == HEAD_DIM
                       and t.device == a.q.device for t in (a.q, a.k, a.v))
         and a.k.shape == a.v.shape and a.k.shape[2] == a.q.shape[2]
         and a.q.shape[1] % a.k.shape[1] == 0),
    Rule("packed_causal_attention: q / k / v need 16-byte aligned bases, a unit last stride and "
         "head / token strides that are multiples of 8",
         lambda a: all(_aligned(t) for t in (a.q, a.k, a.v))),
    Rule("packed_causal_attention: row lengths must be positive and sum to T",
         lambda a: len(a.lengths) > 0 and all(int(n) > 0 for n in a.lengths)
         and sum(int(n) for n in a.lengths) == a.q.shape[2]),
)


def packed_causal_attention(q, k, v, lengths, scale, cu_seqlens=None):
    """softmax(scale q k^T, causal within each row) v for a packed batch.

    ``lengths``: host row lengths (sum T); ``cu_seqlens``: their int32 device
    offsets when already built (see ``row_offsets``).  Returns [1, T, Hq, 128].
    """
    enforce(ATTENTION_RULES, q=q, k=k, v=v, lengths=lengths)
    with torch.cuda.device(q.device):
        cu = cu_seqlens if cu_seqlens is not None else row_offsets(lengths, q.device)
        return PackedCausalAttention.apply(q, k, v, cu, max(int(n) for n in lengths),
                                           float(scale))
