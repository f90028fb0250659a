"""Routes for bitsandbytes 0.50.2's NF4 entry points (behaviour of solution/nf4_patch.py:1-125).

bitsandbytes reaches the 4-bit decode from two training paths: the
functional ``dequantize_4bit`` (MatMul4Bit.backward) and the CUDA backend's
``_dequant_linear_fallback``, which rebuilds the fp32 absmax of a nested state
itself and then calls the backend's ``_dequantize_4bit_impl``.  The routes:

  * ``functional.dequantize_4bit``: nested fp16 NF4 blocksize-64 states go to
    ``dequantize_nf4`` (statistics and codes decoded in one HIP pass, straight
    into ``out`` when given); anything else runs the original;
  * ``backends.cuda.ops._dequant_linear_fallback``: runs the original inside
    a scope that records whether the fp32 absmax it rebuilds came from nested
    statistics (``absmax_8bit`` given);
  * ``backends.cuda.ops._dequantize_4bit_impl``: inside such a nested scope,
    NF4 blocksize-64 fp16 decodes go to ``_dequantize_flat_into`` (writes
    ``out``, returns None like the original); standalone calls keep the original;
  * ``matmul_4bit`` (this package's addition over the reference, which left it
    on bitsandbytes): fp16 CUDA activations against a nested NF4 state with
    ``out=None`` run the fused NF4 GEMM node (forward and dX on the HIP
    kernels, saving only the packed weight); anything else runs the original.

The scope is a ContextVar, so it is per thread and per async task.  Kernel
errors propagate; only ValueError from a contract check selects the original.
The routes are built only for bitsandbytes 0.50.2 (the version the reference
pins, solution/nf4_patch.py:53).
"""

import sys
from contextlib import contextmanager
from contextvars import ContextVar

import torch

from .contract import frozen_buffer
from .utils import enabled

BNB_VERSION = "0.50.2"
_NESTED_ABSMAX = ContextVar("soupsuck_nested_absmax", default=False)


@contextmanager
def _absmax_provenance(nested):
    token = _NESTED_ABSMAX.set(bool(nested))
    try:
        yield
    finally:
        _NESTED_ABSMAX.reset(token)


def _pinned_version():
    bnb = sys.modules.get("bitsandbytes")
    return getattr(bnb, "__version__", None) == BNB_VERSION


def _nested_shape(A, state):
    """quant_state.shape if A / state are a supported nested NF4 pair, else None."""
    from .kernels.nf4 import _validate_state

    if not isinstance(A, torch.Tensor) or not A.is_cuda:
        return None
    try:
        return _validate_state(A, state, torch.float16)
    except ValueError:
        return None


def build_dequantize(original, module):
    if not _pinned_version():
        return None

    def dequantize_4bit(A, quant_state=None, absmax=None, out=None, blocksize=None,
                        quant_type="fp4"):
        kwargs = dict(quant_state=quant_state, absmax=absmax, out=out, blocksize=blocksize,
                      quant_type=quant_type)
        shape = _nested_shape(A, quant_state) if enabled() else None
        out_ok = out is None or (frozen_buffer(out, torch.float16, A.device, 0)
                                 and tuple(out.shape) == shape)
        if shape is None or not out_ok:
            # The original may reach the backend decode: not from nested statistics.
            with _absmax_provenance(False):
                return original(A, **kwargs)
        from .kernels.nf4 import dequantize_nf4

        return dequantize_nf4(A, quant_state, out=out)

    return dequantize_4bit


def build_backend_decode(original, module):
    if not _pinned_version():
        return None

    def _dequantize_4bit_impl(A, absmax, blocksize, quant_type, dtype, out):
        if (_NESTED_ABSMAX.get() and enabled() and blocksize == 64 and quant_type == "nf4"
                and dtype == torch.float16):
            from .kernels.nf4 import _dequantize_flat_into

            try:
                _dequantize_flat_into(A, absmax, out)
            except ValueError:
                return original(A, absmax, blocksize, quant_type, dtype, out)
            return None
        return original(A, absmax, blocksize, quant_type, dtype, out)

    return _dequantize_4bit_impl


def build_linear_fallback(original, module):
    if not _pinned_version():
        return None

    def _dequant_linear_fallback(A, B, shapeB, absmax, blocksize, quant_type, bias=None,
                                 absmax_8bit=None, absmax_code=None, absmax_offset=None):
        with _absmax_provenance(absmax_8bit is not None):
            return original(A, B, shapeB, absmax, blocksize, quant_type, bias=bias,
                            absmax_8bit=absmax_8bit, absmax_code=absmax_code,
                            absmax_offset=absmax_offset)

    return _dequant_linear_fallback


def _matmul_route_ok(A, packed, state, out, bias):
    shape = _nested_shape(packed, state)
    if shape is None or out is not None:
        return False
    n, k = shape
    if not (isinstance(A, torch.Tensor) and A.is_cuda and A.device == packed.device
            and A.dtype == torch.float16 and A.is_contiguous() and A.ndim >= 2
            and A.shape[-1] == k):
        return False
    return bias is None or (frozen_buffer(bias, torch.float16, A.device, n) and bias.shape == (n,))


def build_matmul(original, module):
    if getattr(module, "__version__", None) != BNB_VERSION:
        return None

    def matmul_4bit(A, B, quant_state, out=None, bias=None):
        packed = B.t() if isinstance(B, torch.Tensor) and B.ndim == 2 and B.shape[0] == 1 else B
        if enabled() and _matmul_route_ok(A, packed, quant_state, out, bias):
            from .kernels.nf4_gemm import NF4Linear

            return NF4Linear.apply(A, packed, quant_state, bias)
        return original(A, B, quant_state, out=out, bias=bias)

    return matmul_4bit
