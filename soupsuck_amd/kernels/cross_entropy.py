"""``fused_linear_cross_entropy``: chunked linear + cross-entropy without full logits (A17-A19).

Interface of solution/kernels/cross_entropy.py:214-241 (arguments, the four
returned tensors loss / entropy / first argmax / lse with only ``loss``
differentiable, ValueError before launch) and its numerics (:1-43):

  forward   per vocabulary chunk c: z = fp16(h16 . W_c16^T) on the MFMA GEMM
            (ss_gemm_f16); per row and piece of at most 8192 columns of a chunk,
            the partial state (max m_p, sum e^(z-m_p), sum e^(z-m_p) z, target
            logit, first argmax; ss_ce_stats); the pieces folded in vocabulary
            order as the online softmax merges (m = max, s = sum s_p
            e^(m_p-m), ...), lse = m + log s, loss = lse - z_target (0 for
            ignored rows), entropy = lse - t/s (ss_ce_outputs);
  backward  rows with a target only (found and validated in the forward by one
            launch, ss_ce_rows, whose count is copied to pinned memory early, so
            no stall); each chunk
            is recomputed and dz = fp16((softmax - onehot) g / gain) with the
            per-row gain max(|g|, 1e-30)/1024 (ss_ce_derivative); dX = dz . W_c
            accumulated in fp32 over chunks, multiplied back by the gain and
            scattered to all rows (ss_ce_finalize_dx).  Ignored rows get zero
            gradient whatever the upstream value.

Extension (``weight_grad=True``, asked for by BASELINE configs[3]): the
reference only accepts a frozen head (ValueError "frozen"); here the head
gradient dW_c = dz'^T . h is also produced, from a second fp16 copy dz' of the
derivative scaled by one global gain max_r |g_r| / 1024 (a per-row gain cannot
be factored out of a sum over rows).

Kept logits: when the fp16 logits [N, V] fit KEEP_LOGITS_BUDGET (1 GiB; 251 MB
at configs[3]) and a backward may run, the forward's products write into one
[N, V] buffer and the backward reads the logits from there (rows picked through
the labelled-row indices) instead of recomputing h . W_c^T: one product per
chunk fewer.  The forward's products then span several chunks (as many as fill
one wave of 256 x 256 output tiles: two at configs[3]) and one statistics launch
follows them all; its pieces are those of a chunk-by-chunk forward, so the
outputs are the same bits.  The backward's
steps span as many chunks as DERIVATIVE_BUDGET holds of dz and dz' (the whole
vocabulary at configs[3]): one derivative launch and two long products.  Above
KEEP_LOGITS_BUDGET the backward recomputes, as the reference does, one [rows,
chunk] tile at a time.

Layout for the MFMA engine: the dense direct-to-LDS kernel reads operands stored
along the reduced dimension (K-major) through transposed LDS reads, so dX = dz .
W_c takes the head rows W_c [width, H] as they are, and dW_c = dz'^T . h takes
dz' [T', width] and h [T', H] as they are, T' = rows with a target padded to a
multiple of 64 with zero rows (the kernel reduces whole 64-deep steps).  No
operand is transposed in memory.
"""

import torch
from torch.autograd.function import once_differentiable

from .. import _lib
from ..contract import FLOAT_DTYPES, Rule, enforce, on_one_cuda_device
from .nf4_gemm import gemm_f16

MAX_CHUNK = 8192            # BASELINE configs[3]'s vocabulary chunk
TILE_BUDGET = 64 << 20      # bytes of one fp16 [rows, chunk] logits tile
# Bytes of fp16 logits [rows, V] the forward may keep for the backward, which
# then reads them instead of recomputing each chunk's product (the same bits:
# the backward's recomputed chunk equals the forward's).  Larger outputs are
# recomputed chunk by chunk, holding one [rows, chunk] tile at a time.
KEEP_LOGITS_BUDGET = 1 << 30
STATS_PIECE = 8192          # widest vocabulary piece one ss_ce_stats workgroup reduces
# Bytes of the backward's two fp16 derivative buffers when it reads kept logits.
DERIVATIVE_BUDGET = 1 << 30


def default_chunk(rows):
    """Vocabulary chunk when the caller gives none: the widest multiple of 256,
    at most MAX_CHUNK, whose fp16 logits tile fits TILE_BUDGET."""
    fit = TILE_BUDGET // (2 * max(rows, 1))
    return max(256, min(MAX_CHUNK, fit // 256 * 256))


def _vocab_chunks(vocab, chunk):
    for start in range(0, vocab, chunk):
        yield start, min(chunk, vocab - start)


def _head_rows(weight, start, width):
    w = weight.narrow(0, start, width)
    return w if (w.dtype == torch.float16 and w.is_contiguous()) else \
        w.to(torch.float16).contiguous()


def _gather_rows(src, index, out=None):
    """src[index] for a contiguous tensor and a device int64 index (ss_unpad_gather),
    into ``out`` (contiguous, index.numel() rows) when given."""
    if out is None:
        out = torch.empty((index.numel(), *src.shape[1:]), device=src.device, dtype=src.dtype)
    row_bytes = (src[0].numel() if src.ndim > 1 else 1) * src.element_size()
    _lib.call("ss_unpad_gather", src.data_ptr(), src.shape[0], out.data_ptr(), index.data_ptr(),
              index.numel(), row_bytes, _lib.stream(src.device))
    return out


_CUS = {}


def _product_span(rows, chunk, dev):
    """Vocabulary columns per logits product when the forward keeps its logits: whole
    chunks, as many as fit one wave of 256 x 256 output tiles on the device's CUs (T =
    826: two chunks of 8192, 256 tiles, against 224 tiles of 128 x 256 for one chunk).
    The statistics pieces do not change, and an output element does not depend on the
    product's width, so the results are the same bits."""
    if dev not in _CUS:
        _CUS[dev] = torch.cuda.get_device_properties(dev).multi_processor_count
    tiles = -(-rows // 256) * -(-chunk // 256)
    return max(1, _CUS[dev] // tiles) * chunk


def _backward_span(count, padded, chunk):
    """Vocabulary columns per backward step over kept logits: whole chunks whose fp16
    derivatives dz [count, span] and dz' [padded, span] fit DERIVATIVE_BUDGET together
    (T = 826 with 523 labelled rows: the whole vocabulary in one step).  dW's rows do
    not depend on the step's width; dX's fp32 sum over the vocabulary is split
    differently, so it matches a chunked backward to rounding."""
    return max(1, DERIVATIVE_BUDGET // (2 * (count + padded) * chunk)) * chunk


def _forward(hidden16, weight, targets, ignore_index, chunk, keep):
    """Loss, entropy, first argmax and lse; with ``keep`` also the fp16 logits [rows, V]
    (the products write straight into their columns, several chunks at a time), else
    None."""
    rows = hidden16.shape[0]
    dev = hidden16.device
    loss = torch.empty(rows, device=dev, dtype=torch.float32)
    entropy = torch.empty(rows, device=dev, dtype=torch.float32)
    lse = torch.empty(rows, device=dev, dtype=torch.float32)
    best = torch.empty(rows, device=dev, dtype=torch.int64)
    if rows == 0:
        return loss, entropy, best, lse, None
    stream = _lib.stream(dev)
    vocab = weight.shape[0]
    # Statistics pieces: each chunk splits into per_chunk pieces of `piece` columns
    # (the last narrower), each with a slot of partial state, folded in vocabulary
    # order by ss_ce_outputs.  The pieces depend only on the chunk, so a call over a
    # product of several chunks gives the bits of one call per chunk.
    piece = min(chunk, STATS_PIECE)
    per_chunk = -(-chunk // piece)
    last = vocab - (vocab - 1) // chunk * chunk
    slots = (vocab - 1) // chunk * per_chunk + -(-last // piece)
    partial = torch.empty((rows, slots, 4), device=dev, dtype=torch.float32)
    partial_arg = torch.empty((rows, slots), device=dev, dtype=torch.int64)
    tile = torch.empty((rows, vocab if keep else min(chunk, vocab)), device=dev,
                       dtype=torch.float16)

    def stats(z, start):
        _lib.call("ss_ce_stats", z.data_ptr(), tile.stride(0), targets.data_ptr(),
                  partial.data_ptr(), partial_arg.data_ptr(), rows, z.shape[1], piece, start,
                  start // chunk * per_chunk, slots, ignore_index, stream)

    if keep:
        for start, width in _vocab_chunks(vocab, _product_span(rows, chunk, dev)):
            gemm_f16(hidden16, _head_rows(weight, start, width), b_trans=True,
                     out=tile[:, start:start + width])
        # Every logit at hand: one statistics launch when the pieces tile whole chunks
        # (and fit one launch's grid).
        whole = chunk % piece == 0 and slots < 65536
        calls = [(0, vocab)] if whole else _vocab_chunks(vocab, chunk)
        for start, width in calls:
            stats(tile[:, start:start + width], start)
    else:
        for start, width in _vocab_chunks(vocab, chunk):
            gemm_f16(hidden16, _head_rows(weight, start, width), b_trans=True,
                     out=tile[:, :width])
            stats(tile[:, :width], start)
    _lib.call("ss_ce_outputs", partial.data_ptr(), partial_arg.data_ptr(), slots,
              targets.data_ptr(), loss.data_ptr(), entropy.data_ptr(), lse.data_ptr(),
              best.data_ptr(), rows, ignore_index, stream)
    return loss, entropy, best, lse, tile if keep else None


class _KeptRows:
    """Rows with a target, found and validated in the forward without a host
    synchronisation (ss_ce_rows, one launch).

    `order` lists the labelled rows in row order, then -1 up to a multiple of 64
    rows (the gather of the head-gradient product's operand writes zero rows
    there); their count is copied to pinned host memory as soon as it is
    computed, ahead of the forward's GEMMs, so by the time the backward needs it
    the copy has long completed and reading it does not stall the device.  `ok`
    is False when a target is outside [0, V) and not ignore_index."""

    def __init__(self, targets, ignore_index, vocab):
        rows = targets.numel()
        dev = targets.device
        self.order = torch.empty(-(-rows // 64) * 64, device=dev, dtype=torch.int64)
        count = torch.empty((), device=dev, dtype=torch.int64)
        self.ok = torch.empty((), device=dev, dtype=torch.bool)
        _lib.call("ss_ce_rows", targets.data_ptr(), rows, vocab, ignore_index,
                  self.order.data_ptr(), self.order.numel(), count.data_ptr(),
                  self.ok.data_ptr(), _lib.stream(dev))
        self.count_host = torch.empty((), dtype=torch.int64, pin_memory=True)
        self.count_host.copy_(count, non_blocking=True)
        self.ready = torch.cuda.Event()
        self.ready.record()

    def count(self):
        self.ready.synchronize()
        return int(self.count_host)


class _Backward:
    """Gradients of the summed loss w.r.t. hidden and (optionally) the head."""

    def __init__(self, hidden16, weight, targets, lse, grad, ignore_index, chunk, kept,
                 logits=None):
        self.weight, self.ignore, self.chunk = weight, ignore_index, chunk
        self.logits = logits  # the forward's fp16 [rows, V] logits, or None: recompute
        self.dev = hidden16.device
        self.stream = _lib.stream(self.dev)
        self.full_grad = grad
        self.count = kept.count()
        self.kept = kept.order[:self.count]
        if self.count:
            # Rows with a target, then zero rows up to a multiple of 64 (index -1): the
            # K of the head-gradient product.
            self.padded = -(-self.count // 64) * 64
            self.h_pad = _gather_rows(hidden16, kept.order[:self.padded])
            self.h = self.h_pad[:self.count]
            self.targets = _gather_rows(targets, self.kept)
            self.lse = _gather_rows(lse, self.kept)
            self.grad = _gather_rows(grad, self.kept)

    def run(self, dx, dw):
        count, padded = self.count, self.padded
        hdim = self.h.shape[1]
        kept_z = self.logits
        # With the kept logits a step spans as many chunks as the derivative buffers'
        # budget holds (the derivative is elementwise and the products take any width:
        # fewer, longer products); recomputing, one chunk at a time.
        span = self.chunk if kept_z is None else _backward_span(count, padded, self.chunk)
        width_max = min(span, self.weight.shape[0])
        if kept_z is None:
            logits = torch.empty((count, width_max), device=self.dev, dtype=torch.float16)
        dz = torch.empty((count, width_max), device=self.dev, dtype=torch.float16)
        # dX accumulates over the steps; the first one overwrites.
        acc = torch.empty((count, hdim), device=self.dev, dtype=torch.float32) \
            if dx is not None else None
        head_gain = None
        if dw is not None:
            # max_r |g_r| / 1024 as a device scalar (ss_ce_head_gain): no host round trip
            # between the forward and the backward's launches
            head_gain = torch.empty(1, device=self.dev, dtype=torch.float32)
            _lib.call("ss_ce_head_gain", self.grad.data_ptr(), count, head_gain.data_ptr(),
                      self.stream)
            # dz' per step as [padded, width] (dense rows); the derivative writes the rows
            # past `count` as zeros.
            dz_head = torch.empty(padded * width_max, device=self.dev, dtype=torch.float16)
        first = True
        for start, width in _vocab_chunks(self.weight.shape[0], span):
            w = _head_rows(self.weight, start, width)
            if kept_z is None:
                z, ldz, z_rows = logits[:, :width], logits.stride(0), None
                gemm_f16(self.h, w, b_trans=True, out=z)
            else:
                # The forward's logits of the step, rows picked through the kept-row indices.
                z, ldz, z_rows = kept_z[:, start:start + width], kept_z.stride(0), self.kept
            d = dz.view(-1)[:count * width].view(count, width)
            dh = None
            if dw is not None:
                dh = dz_head[:padded * width].view(padded, width)
            _lib.call("ss_ce_derivative", z.data_ptr(), ldz, _lib.ptr(z_rows),
                      self.targets.data_ptr(), self.lse.data_ptr(), self.grad.data_ptr(),
                      d.data_ptr(), _lib.ptr(dh), _lib.ptr(head_gain), count,
                      padded if dh is not None else count, width, start, self.ignore,
                      self.stream)
            if acc is not None:
                gemm_f16(d, w, out=acc, accumulate=not first, split_k=True)
            first = False
            if dw is not None:
                rows_w = dw.narrow(0, start, width)
                if rows_w.dtype in FLOAT_DTYPES:
                    gemm_f16(dh, self.h_pad, a_trans=True, out=rows_w, alpha_dev=head_gain)
                else:
                    rows_w.copy_(gemm_f16(dh, self.h_pad, a_trans=True,
                                          out_dtype=torch.float32, alpha_dev=head_gain))
        if acc is not None:
            rows, hd = dx.shape
            inverse = torch.empty(rows, device=self.dev, dtype=torch.int32)
            _lib.call("ss_unpad_inverse", self.kept.data_ptr(), self.count, inverse.data_ptr(),
                      rows, self.stream)
            _lib.call("ss_ce_finalize_dx", acc.data_ptr(), self.count, self.full_grad.data_ptr(),
                      inverse.data_ptr(), dx.data_ptr(), _lib.dtype_code(dx.dtype), rows, hd,
                      self.stream)


class LinearCrossEntropy(torch.autograd.Function):
    @staticmethod
    def forward(ctx, hidden, weight, targets, ignore_index, chunk, weight_grad, kept):
        hidden16 = hidden.to(torch.float16).contiguous()
        targets = targets.contiguous()
        chunk = chunk or default_chunk(hidden16.shape[0])
        ctx.kept = kept
        backward_may_run = ctx.needs_input_grad[0] or (weight_grad and ctx.needs_input_grad[1])
        keep = backward_may_run and \
            hidden16.shape[0] * weight.shape[0] * 2 <= KEEP_LOGITS_BUDGET
        loss, entropy, best, lse, ctx.logits = _forward(hidden16, weight, targets, ignore_index,
                                                        chunk, keep)
        ctx.save_for_backward(hidden16, weight, targets, lse)
        ctx.setup = (hidden.dtype, ignore_index, chunk, weight_grad)
        ctx.mark_non_differentiable(entropy, best, lse)
        ctx.set_materialize_grads(False)
        return loss, entropy, best, lse

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_loss, *_unused):
        hidden_dtype, ignore_index, chunk, weight_grad = ctx.setup
        logits, ctx.logits = ctx.logits, None  # kept logits serve one backward
        want_x = ctx.needs_input_grad[0]
        want_w = weight_grad and ctx.needs_input_grad[1]
        nothing = (None,) * 7
        if grad_loss is None or not (want_x or want_w):
            return nothing
        hidden16, weight, targets, lse = ctx.saved_tensors
        # Uninitialised: with a labelled row, ss_ce_finalize_dx writes every row of dX and
        # the chunk GEMMs every row of dW (a 467 MB fill at V = 151936 saved); without
        # one both gradients are zero.
        dx = torch.empty(hidden16.shape, device=hidden16.device, dtype=hidden_dtype) \
            if want_x else None
        dw = torch.empty(weight.shape, device=weight.device, dtype=weight.dtype) \
            if want_w else None
        back = None
        if hidden16.shape[0]:
            grad = grad_loss.float().contiguous()
            back = _Backward(hidden16, weight, targets, lse, grad, ignore_index, chunk, ctx.kept,
                             logits)
        if back is not None and back.count:
            back.run(dx, dw)
        else:
            for g in (dx, dw):
                if g is not None:
                    g.zero_()
        return dx, dw, None, None, None, None, None


CE_RULES = (
    Rule("fused_linear_cross_entropy: a trainable weight needs weight_grad=True (the "
         "reference requires a frozen weight)",
         lambda a: a.weight_grad or not getattr(a.weight, "requires_grad", False)),
    Rule("fused_linear_cross_entropy: expected hidden [N, H], weight [V, H], targets [N] with "
         "V, H > 0",
         lambda a: all(isinstance(t, torch.Tensor) for t in (a.hidden, a.weight, a.targets))
         and a.hidden.ndim == 2 and a.weight.ndim == 2 and a.targets.ndim == 1
         and a.hidden.shape[1] == a.weight.shape[1] and a.hidden.shape[0] == a.targets.shape[0]
         and a.weight.shape[0] > 0 and a.weight.shape[1] > 0),
    Rule("fused_linear_cross_entropy: hidden and weight must be fp16 or fp32, targets int64",
         lambda a: a.hidden.dtype in FLOAT_DTYPES and a.weight.dtype in FLOAT_DTYPES
         and a.targets.dtype == torch.int64),
    Rule("fused_linear_cross_entropy: hidden, weight and targets must be CUDA tensors on one "
         "device",
         lambda a: on_one_cuda_device(a.hidden, a.weight, a.targets)),
    Rule("fused_linear_cross_entropy: ignore_index must be an int",
         lambda a: isinstance(a.ignore_index, int) and not isinstance(a.ignore_index, bool)),
    Rule("fused_linear_cross_entropy: chunk must be None or a positive int",
         lambda a: a.chunk is None or (isinstance(a.chunk, int) and a.chunk > 0)),
)


def fused_linear_cross_entropy(hidden, weight, targets, ignore_index=-100, *, chunk=None,
                               weight_grad=False):
    """Per-token (loss, entropy, first argmax, lse) of softmax(hidden . weight^T).

    hidden [N, H] and weight [V, H] fp16/fp32, targets [N] int64 (already
    shifted), on one CUDA device.  Only ``loss`` carries a gradient.  A target
    outside [0, V) other than ignore_index fails a device-side assertion (no
    host synchronisation in the forward).
    """
    enforce(CE_RULES, hidden=hidden, weight=weight, targets=targets, ignore_index=ignore_index,
            chunk=chunk, weight_grad=weight_grad)
    with torch.cuda.device(hidden.device):
        targets = targets.contiguous()
        kept = None
        if targets.numel():
            # Labelled rows and the target check in one launch (ss_ce_rows).
            kept = _KeptRows(targets, ignore_index, weight.shape[0])
            torch._assert_async(kept.ok, "fused_linear_cross_entropy: target outside the "
                                         "vocabulary")
        return LinearCrossEntropy.apply(hidden, weight, targets, ignore_index, chunk,
                                        bool(weight_grad), kept)
