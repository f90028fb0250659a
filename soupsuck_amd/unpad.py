"""Right-padding removal: packed gather / zero-filling scatter with autograd (A16).

Mirrors the reference's solution/unpad.py:51-72 (right_padding_lengths),
:149-161 (_pack / _scatter) and :184-199 (row-major indices built on the
device without a host-to-device copy).  The row copies are the HIP kernels
ss_unpad_gather / ss_unpad_scatter (bit-exact); the scatter's zero rows and
copies are one pass, and each op's backward is the other op.
"""

from dataclasses import dataclass, field

import torch

from . import _lib


def right_padding_lengths(rows):
    """Validate binary nonempty right-padded rows; pure Python (reference unpad.py:51-72)."""
    if not rows or not rows[0]:
        return None
    width, lengths = len(rows[0]), []
    for row in rows:
        if len(row) != width:
            return None
        count, padding = 0, False
        for value in row:
            if value not in (0, 1):
                return None
            if value == 0:
                padding = True
            elif padding:
                return None
            else:
                count += 1
        if not count:
            return None
        lengths.append(count)
    return tuple(lengths)


def indices_from_lengths(lengths, sequence, device):
    """Row-major packed indices row*S + t (t < length), built on the device."""
    indices = torch.arange(sum(lengths), device=device, dtype=torch.long)
    start = 0
    for row, length in enumerate(lengths):
        offset = row * sequence - start
        if offset:
            indices.narrow(0, start, length).add_(offset)
        start += length
    return indices


@dataclass
class PackedBatch:
    batch: int
    sequence: int
    lengths: tuple
    indices: torch.Tensor
    _inverse: torch.Tensor = field(default=None, repr=False)

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
