"""NF4 decode entry points: ``dequantize_nf4`` and the backend's ``_dequantize_flat_into``.

Interface of solution/kernels/nf4.py:140-203 (names, arguments, accepted
states, ValueError before any launch, ``out=`` ownership and the transposed
view for a packed tensor stored as [1, n/2], nf4.py:203).  Accepted state
(the only one the reference decodes): fp16 NF4 with blocksize 64 and nested
statistics -- uint8 block codes ``absmax`` decoded through the fp32 block-256
``state2`` (absmax, 256-entry code) plus an fp32 ``offset``.  The decode is
ss_nf4_dequant_nested / ss_nf4_dequant_flat in the HIP library, bit-exact
against fp16(NF4[nibble] * fp32(fp32(code2[qabs] * absmax2) + offset)).
"""

import math

import torch

from .. import _lib
from ..contract import Rule, cdiv, enforce, frozen_buffer, is_tensor

NF4_VALUES = (
    -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
    -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
    0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
    0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0,
)


def _storage_ok(packed):
    return (is_tensor(packed) and packed.is_cuda and packed.dtype == torch.uint8
            and packed.is_contiguous() and packed.ndim in (1, 2))


def _matrix_shape(state):
    shape = getattr(state, "shape", None)
    if not isinstance(shape, (tuple, list, torch.Size)) or len(shape) != 2:
        return None
    if not all(isinstance(d, int) and d > 0 for d in shape):
        return None
    return tuple(shape)


def _nested_buffers_fit(packed, state, shape):
    """Every buffer of the nested state is present, frozen, on packed's device and long enough."""
    n = math.prod(shape)
    blocks = cdiv(n, 64)
    dev, second = packed.device, state.state2
    offset = getattr(state, "offset", None)
    return (packed.numel() * 2 >= n
            and frozen_buffer(getattr(state, "absmax", None), torch.uint8, dev, blocks)
            and frozen_buffer(getattr(second, "absmax", None), torch.float32, dev,
                              cdiv(blocks, 256))
            and frozen_buffer(getattr(second, "code", None), torch.float32, dev, 256)
            and frozen_buffer(offset, torch.float32, dev, 1) and offset.numel() == 1)


NESTED_STATE_RULES = (
    Rule("NF4 storage must be a contiguous one- or two-dimensional uint8 CUDA tensor",
         lambda a: _storage_ok(a.packed)),
    Rule("NF4 decode: only fp16 output is supported",
         lambda a: a.out_dtype == torch.float16),
    Rule("quant_state: expected fp16 NF4 with blocksize 64 and nested (compressed) statistics",
         lambda a: getattr(a.state, "quant_type", None) == "nf4"
         and getattr(a.state, "blocksize", None) == 64
         and getattr(a.state, "dtype", None) == torch.float16
         and bool(getattr(a.state, "nested", False))),
    Rule("quant_state.shape: expected two positive integers",
         lambda a: _matrix_shape(a.state) is not None),
    Rule("quant_state.state2: expected a non-nested fp32 state with blocksize 256",
         lambda a: getattr(getattr(a.state, "state2", None), "blocksize", None) == 256
         and getattr(a.state.state2, "dtype", None) == torch.float32
         and not getattr(a.state.state2, "nested", False)),
    Rule("quant_state buffers: packed codes, absmax, state2.absmax/code or offset do not fit "
         "the shape (each must be a contiguous frozen tensor on the storage's device)",
         lambda a: _nested_buffers_fit(a.packed, a.state, _matrix_shape(a.state))),
)


def _flat_out_ok(out, packed):
    return (is_tensor(out) and out.dtype == torch.float16 and out.device == packed.device
            and out.is_contiguous() and out.ndim == 2 and not out.requires_grad
            and packed.numel() * 2 >= out.numel())


FLAT_RULES = (
    Rule("flat NF4 decode: storage must be a contiguous one- or two-dimensional uint8 CUDA tensor",
         lambda a: _storage_ok(a.packed)),
    Rule("flat NF4 decode: out must be a contiguous frozen 2-D fp16 tensor on the storage's "
         "device, covered by the packed codes",
         lambda a: _flat_out_ok(a.out, a.packed)),
    Rule("flat NF4 decode: absmax must be a contiguous frozen fp32 tensor of one scale per "
         "64 elements",
         lambda a: frozen_buffer(a.absmax, torch.float32, a.packed.device,
                                 cdiv(a.out.numel(), 64))),
)


def _validate_state(packed, state, out_dtype):
    """Return the (N, K) shape of a supported nested NF4 state, else raise ValueError."""
    enforce(NESTED_STATE_RULES, packed=packed, state=state, out_dtype=out_dtype)
    return _matrix_shape(state)


def _decode_nested(packed, state, out):
    _lib.call("ss_nf4_dequant_nested", packed.data_ptr(), state.absmax.data_ptr(),
              state.state2.absmax.data_ptr(), state.state2.code.data_ptr(),
              state.offset.data_ptr(), out.data_ptr(), out.numel(), _lib.stream(packed.device))


def _dequantize_flat_into(packed, absmax, out):
    """Decode with an already reconstructed fp32 absmax (one per 64-block) into ``out``."""
    enforce(FLAT_RULES, packed=packed, absmax=absmax, out=out)
    if out.numel():
        with torch.cuda.device(packed.device):
            _lib.call("ss_nf4_dequant_flat", packed.data_ptr(), absmax.data_ptr(),
                      out.data_ptr(), out.numel(), _lib.stream(packed.device))
    return out


def dequantize_nf4(packed, quant_state, out_dtype=torch.float16, *, out=None):
    """Decode into ``out`` (allocated when None) of quant_state.shape.

    Returns ``out``, or its transpose when the packed codes are stored as a
    [1, n/2] row (the layout bitsandbytes gives a transposed weight).
    """
    shape = _validate_state(packed, quant_state, out_dtype)
    if out is not None:
        enforce((Rule("out must be a contiguous frozen fp16 tensor of quant_state.shape on the "
                      "storage's device",
                      lambda a: is_tensor(a.out) and tuple(a.out.shape) == shape
                      and a.out.device == packed.device and a.out.dtype == out_dtype
                      and a.out.is_contiguous() and not a.out.requires_grad),), out=out)
    with torch.cuda.device(packed.device):
        target = out if out is not None else torch.empty(shape, device=packed.device,
                                                         dtype=out_dtype)
        _decode_nested(packed, quant_state, target)
    return target.t() if packed.shape[0] == 1 else target
