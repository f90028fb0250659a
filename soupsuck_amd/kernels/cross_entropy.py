"""Chunked fused linear cross-entropy without full-vocabulary logits (A17-A19).

Mirrors the reference's solution/kernels/cross_entropy.py:133-241
(``_FrozenLinearCrossEntropy`` / ``fused_linear_cross_entropy``):
  * logits of each vocabulary chunk are fp16(h16 . w16^T) (MFMA GEMM,
    ss_gemm_f16), and online statistics m, sum exp, sum exp*z, target logit
    and first argmax are merged chunk by chunk (ss_ce_stats); outputs
    lse, entropy and per-token loss (ss_ce_outputs);
  * backward compacts the rows with a target (one nonzero synchronisation),
    recomputes each chunk, forms dz = g (softmax - onehot) scaled per row by
    1/gain, gain = max(|g|, 1e-30)/1024, rounds it to fp16
    (ss_ce_derivative), accumulates dX in fp32 over chunks and undoes the gain
    while scattering back to all rows (ss_ce_finalize_dx).
Extension (``weight_grad=True``): the reference rejects a trainable head
(cross_entropy.py:221-222); here the lm_head gradient dW = dz^T . h is also
produced, from a second fp16 copy of dz scaled by one global gain
max_r |g_r| / 1024 (a per-row gain cannot be factored out of a sum over rows).
"""

import torch
from torch.autograd.function import once_differentiable

from .. import _lib
from .nf4_gemm import gemm_f16, transpose_f16


def _chunk_size(n, h):
    """Reference default (cross_entropy.py:125-130): <= 4096 and memory-capped, power of 2."""
    limit = min(4096, (64 * 1024 ** 2) // (2 * max(n, 1)), (32 * 1024 ** 2) // (2 * h))
    if limit < 1:
        raise ValueError("A single vocabulary column exceeds the temporary memory budget")
    return 1 << (limit.bit_length() - 1)


def _rows(src, index, row_bytes_per_elem):
    """Gather rows of a contiguous tensor by a device index (ss_unpad_gather)."""
    count = index.numel()
    out = torch.empty((count, *src.shape[1:]), device=src.device, dtype=src.dtype)
    row_bytes = src[0].numel() * src.element_size() if src.ndim > 1 else src.element_size()
    _lib.call("ss_unpad_gather", src.data_ptr(), src.shape[0], out.data_ptr(), index.data_ptr(),
              count, row_bytes, _lib.stream(src.device))
    return out


def _chunk_weight(weight, start, chunk):
    w = weight[start:start + chunk]
    if w.dtype != torch.float16 or not w.is_contiguous():
        w = w.to(torch.float16).contiguous()
    return w


class _LinearCrossEntropy(torch.autograd.Function):
    @staticmethod
    def forward(ctx, hidden, weight, targets, ignore_index, chunk, weight_grad):
        ctx.hidden_dtype = hidden.dtype
        hidden = hidden.to(torch.float16).contiguous()
        targets = targets.contiguous()
        n, h = hidden.shape
        v = weight.shape[0]
        chunk = chunk or _chunk_size(n, h)
        loss = torch.empty(n, device=hidden.device, dtype=torch.float32)
        entropy, lse = torch.empty_like(loss), torch.empty_like(loss)
        best = torch.empty(n, device=hidden.device, dtype=torch.int64)
        stream = _lib.stream(hidden.device)
        if n:
            state = torch.empty((n, 4), device=hidden.device, dtype=torch.float32)
            z = torch.empty((n, min(chunk, v)), device=hidden.device, dtype=torch.float16)
            for start in range(0, v, chunk):
                w = _chunk_weight(weight, start, chunk)
                width = w.shape[0]
                zc = z[:, :width]
                gemm_f16(hidden, w, b_trans=True, out=zc)
                _lib.call("ss_ce_stats", zc.data_ptr(), z.stride(0), targets.data_ptr(),
                          state.data_ptr(), best.data_ptr(), n, width, start, ignore_index,
                          int(start == 0), stream)
            _lib.call("ss_ce_outputs", state.data_ptr(), targets.data_ptr(), loss.data_ptr(),
                      entropy.data_ptr(), lse.data_ptr(), n, ignore_index, stream)
        ctx.save_for_backward(hidden, weight, targets, lse)
        ctx.ignore_index, ctx.chunk, ctx.weight_grad = ignore_index, chunk, weight_grad
        ctx.mark_non_differentiable(entropy, best, lse)
        ctx.set_materialize_grads(False)
        return loss, entropy, best, lse

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_loss, _grad_entropy, _grad_best, _grad_lse):
        hidden, weight, targets, lse = ctx.saved_tensors
        need_x = ctx.needs_input_grad[0]
        need_w = ctx.weight_grad and ctx.needs_input_grad[1]
        if grad_loss is None or not (need_x or need_w):
            return None, None, None, None, None, None
        n, h = hidden.shape
        v = weight.shape[0]
        device = hidden.device
        dx = torch.zeros((n, h), device=device, dtype=ctx.hidden_dtype) if need_x else None
        dw = torch.zeros(weight.shape, device=device, dtype=weight.dtype) if need_w else None
        if not n:
            return dx, dw, None, None, None, None
        valid_index = torch.nonzero(targets != ctx.ignore_index, as_tuple=False).flatten()
        valid_n = valid_index.numel()
        if not valid_n:
            # Ignored rows have zero gradient regardless of a non-finite upstream.
            return dx, dw, None, None, None, None
        stream = _lib.stream(device)
        grad = grad_loss.float().contiguous()
        work_hidden = _rows(hidden, valid_index, 2)
        work_targets = _rows(targets, valid_index, 8)
        work_lse = _rows(lse, valid_index, 4)
        work_grad = _rows(grad, valid_index, 4)
        inverse = torch.empty(n, device=device, dtype=torch.int32)
        _lib.call("ss_unpad_inverse", valid_index.data_ptr(), valid_n, inverse.data_ptr(), n,
                  stream)
        global_gain = 1.0
        if need_w:
            global_gain = max(work_grad.abs().max().item(), 1e-30) / 1024.0
        acc = torch.zeros((valid_n, h), device=device, dtype=torch.float32) if need_x else None
        width_max = min(ctx.chunk, v)
        z = torch.empty((valid_n, width_max), device=device, dtype=torch.float16)
        dz = torch.empty((valid_n, width_max), device=device, dtype=torch.float16)
        dzg = torch.empty_like(dz) if need_w else None
        # The chunk products go to the dense NT kernel, which wants both operands
        # contiguous along the reduced dimension: dX = dz . W_c reduces over the
        # chunk (W_c^T [H, width] per chunk), dW_c = dzg^T . h reduces over the
        # valid rows (dzg^T [width, T'] and h^T [H, T'], T' = valid rows padded
        # to 64 with zero columns, so K % 64 == 0).
        wt = torch.empty((h, width_max), device=device, dtype=torch.float16) if need_x else None
        if need_w:
            t_pad = -(-valid_n // 64) * 64
            ht = torch.zeros((h, t_pad), device=device, dtype=torch.float16)
            transpose_f16(work_hidden, out=ht[:, :valid_n])
            dzgt = torch.zeros((width_max, t_pad), device=device, dtype=torch.float16)
        for start in range(0, v, ctx.chunk):
            w = _chunk_weight(weight, start, ctx.chunk)
            width = w.shape[0]
            zc = z[:, :width]
            gemm_f16(work_hidden, w, b_trans=True, out=zc)
            dzc = dz.view(-1)[:valid_n * width].view(valid_n, width)
            dzgc = dzg.view(-1)[:valid_n * width].view(valid_n, width) if need_w else None
            _lib.call("ss_ce_derivative", zc.data_ptr(), z.stride(0), work_targets.data_ptr(),
                      work_lse.data_ptr(), work_grad.data_ptr(), dzc.data_ptr(),
                      _lib.ptr(dzgc), float(global_gain), valid_n, width, start,
                      ctx.ignore_index, stream)
            if need_x:
                wtc = transpose_f16(w, out=wt[:, :width])
                gemm_f16(dzc, wtc, b_trans=True, out=acc, accumulate=True, split_k=True)
            if need_w:
                dw_chunk = dw[start:start + width]
                transpose_f16(dzgc, out=dzgt[:width, :valid_n])
                dzgtc = dzgt[:width]
                if dw.dtype == torch.float16 or dw.dtype == torch.float32:
                    gemm_f16(dzgtc, ht, b_trans=True, out=dw_chunk, alpha=float(global_gain))
                else:
                    dw_chunk.copy_(gemm_f16(dzgtc, ht, b_trans=True, out_dtype=torch.float32,
                                            alpha=float(global_gain)))
        if need_x:
            _lib.call("ss_ce_finalize_dx", acc.data_ptr(), valid_n, grad.data_ptr(),
                      inverse.data_ptr(), dx.data_ptr(), _lib.dtype_code(dx.dtype), n, h, stream)
        return dx, dw, None, None, None, None


def fused_linear_cross_entropy(hidden, weight, targets, ignore_index=-100, *, chunk=None,
                               weight_grad=False):
    """Return per-token loss, entropy, first argmax and lse (reference cross_entropy.py:214-241).

    hidden[N,H] fp16/fp32, weight[V,H] fp16/fp32, targets[N] int64 (already
    shifted), all on one CUDA device.  Only ``loss`` has an autograd edge.
    ``weight_grad=True`` (extension) also differentiates w.r.t. a trainable
    weight; otherwise a weight that requires grad is rejected like the reference.
    """
    if weight.requires_grad and not weight_grad:
        raise ValueError("fused_linear_cross_entropy requires frozen weight")
    if hidden.ndim != 2 or weight.ndim != 2 or targets.ndim != 1:
        raise ValueError("Expected hidden[N,H], weight[V,H], targets[N]")
    if hidden.shape[1] != weight.shape[1] or hidden.shape[0] != targets.shape[0]:
        raise ValueError("Incompatible hidden, weight and targets shapes")
    if weight.shape[0] == 0 or weight.shape[1] == 0:
        raise ValueError("Vocabulary and hidden dimensions must be positive")
    if (hidden.dtype not in (torch.float16, torch.float32)
            or weight.dtype not in (torch.float16, torch.float32)):
        raise ValueError("Expected fp16/fp32 hidden and weight")
    if targets.dtype != torch.int64:
        raise ValueError("Expected int64 targets")
    if not hidden.is_cuda or weight.device != hidden.device or targets.device != hidden.device:
        raise ValueError("Inputs must be on the same CUDA device")
    if not isinstance(ignore_index, int):
        raise ValueError("ignore_index must be an integer")
    if chunk is not None and (not isinstance(chunk, int) or chunk <= 0):
        raise ValueError("chunk must be a positive integer")
    with torch.cuda.device(hidden.device):
        torch._assert_async(((targets == ignore_index)
                             | ((targets >= 0) & (targets < weight.shape[0]))).all(),
                            "Target outside vocabulary")
        return _LinearCrossEntropy.apply(hidden, weight, targets, ignore_index, chunk,
                                         bool(weight_grad))
