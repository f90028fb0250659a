"""Right-padding removal: packed gather / zero-filling scatter with autograd (A16).

Interface of the reference's solution/unpad.py: right_padding_lengths
(:51-72), packing into [1, T, ...] and scattering back with zero padding rows
(:149-161), and row-major indices of the real tokens built on the device
without a host-to-device copy (:184-199).  The row copies are the HIP kernels
ss_unpad_gather / ss_unpad_scatter (bit-exact); the scatter's zero rows and
copies are one pass, and each op's backward is the other op.
"""

from dataclasses import dataclass, field

import torch

from . import _lib


def right_padding_lengths(rows):
    """Real-token count of each right-padded mask row, or None if the mask is not one.

    ``rows`` is a sequence of equally long rows of 0/1 values (host data, e.g.
    a mask's ``tolist()``); a row qualifies when it is ones followed by zeros
    with at least one one.  Same accept/reject rule as the reference
    (solution/unpad.py:51-72); no device work.
    """
    if not rows or not len(rows[0]):
        return None
    width = len(rows[0])
    lengths = []
    for row in rows:
        values = list(row)
        if len(values) != width or any(v not in (0, 1) for v in values):
            return None
        ones = int(sum(values))
        if ones == 0 or values != [1] * ones + [0] * (width - ones):
            return None
        lengths.append(ones)
    return tuple(lengths)


def indices_from_lengths(lengths, sequence, device):
    """int64 indices row * sequence + t (t < length) of the real tokens, row-major.

    Built from per-row ``arange`` launches on the device, so no host-to-device
    copy (and no synchronisation) happens.
    """
    parts = [torch.arange(row * sequence, row * sequence + n, device=device, dtype=torch.long)
             for row, n in enumerate(lengths)]
    return torch.cat(parts) if parts else torch.empty(0, device=device, dtype=torch.long)


@dataclass
class PackedBatch:
    batch: int
    sequence: int
    lengths: tuple
    indices: torch.Tensor
    _inverse: torch.Tensor = field(default=None, repr=False)
    # set by the Qwen2Model route: int32 row offsets for the attention kernels, the
    # attention modules that run packed, and the LoRA dropouts bound to this batch
    cu_seqlens: torch.Tensor = field(default=None, repr=False)
    attention_ids: frozenset = frozenset()
    dropout_ids: frozenset = frozenset()

    @property
    def tokens(self):
        return sum(self.lengths)

    @property
    def rows(self):
        return self.batch * self.sequence

    def inverse(self):
        """int32[B*S]: packed position of each padded row, -1 for padding (cached)."""
        if self._inverse is None:
            inv = torch.empty(self.rows, device=self.indices.device, dtype=torch.int32)
            _lib.call("ss_unpad_inverse", self.indices.data_ptr(), self.tokens, inv.data_ptr(),
                      self.rows, _lib.stream(self.indices.device))
            self._inverse = inv
        return self._inverse


def make_batch(lengths, sequence, device):
    lengths = tuple(int(x) for x in lengths)
    if not lengths or any(x <= 0 or x > sequence for x in lengths):
        raise ValueError("lengths must be in [1, sequence]")
    return PackedBatch(len(lengths), sequence, lengths,
                       indices_from_lengths(lengths, sequence, device))


def _gather_rows(x2d, batch):
    out = torch.empty((batch.tokens, x2d.shape[1]), device=x2d.device, dtype=x2d.dtype)
    _lib.call("ss_unpad_gather", x2d.data_ptr(), x2d.shape[0], out.data_ptr(),
              batch.indices.data_ptr(), batch.tokens, x2d.shape[1] * x2d.element_size(),
              _lib.stream(x2d.device))
    return out


def _scatter_rows(p2d, batch):
    out = torch.empty((batch.rows, p2d.shape[1]), device=p2d.device, dtype=p2d.dtype)
    _lib.call("ss_unpad_scatter", p2d.data_ptr(), batch.tokens, out.data_ptr(),
              batch.inverse().data_ptr(), batch.rows, p2d.shape[1] * p2d.element_size(),
              _lib.stream(p2d.device))
    return out


class _Pack(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, batch):
        ctx.batch = batch
        tail = x.shape[2:]
        flat = x.reshape(batch.rows, -1).contiguous()
        return _gather_rows(flat, batch).reshape(1, batch.tokens, *tail)

    @staticmethod
    def backward(ctx, grad):
        batch = ctx.batch
        tail = grad.shape[2:]
        flat = grad.reshape(batch.tokens, -1).contiguous()
        return _scatter_rows(flat, batch).reshape(batch.batch, batch.sequence, *tail), None


class _Scatter(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, batch):
        ctx.batch = batch
        tail = x.shape[2:]
        flat = x.reshape(batch.tokens, -1).contiguous()
        return _scatter_rows(flat, batch).reshape(batch.batch, batch.sequence, *tail)

    @staticmethod
    def backward(ctx, grad):
        batch = ctx.batch
        tail = grad.shape[2:]
        flat = grad.reshape(batch.rows, -1).contiguous()
        return _gather_rows(flat, batch).reshape(1, batch.tokens, *tail), None


def _check(x, batch, leading):
    if not isinstance(x, torch.Tensor) or not x.is_cuda:
        raise ValueError("unpad expects a CUDA tensor")
    if tuple(x.shape[:2]) != leading:
        raise ValueError(f"expected leading shape {leading}, got {tuple(x.shape[:2])}")
    if x.element_size() * (x[0, 0].numel() if x.ndim > 2 else 1) % 2:
        raise ValueError("row size must be an even number of bytes")


def pack(x, batch):
    """[B, S, ...] -> [1, T, ...] keeping the real (unpadded) rows (reference _pack)."""
    _check(x, batch, (batch.batch, batch.sequence))
    with torch.cuda.device(x.device):
        if x.ndim > 2:
            return _Pack.apply(x, batch)
        return _Pack.apply(x.unsqueeze(-1), batch).squeeze(-1)


def scatter(x, batch):
    """[1, T, ...] -> [B, S, ...] with zero padding rows (reference _scatter)."""
    _check(x, batch, (1, batch.tokens))
    with torch.cuda.device(x.device):
        if x.ndim > 2:
            return _Scatter.apply(x, batch)
        return _Scatter.apply(x.unsqueeze(-1), batch).squeeze(-1)
