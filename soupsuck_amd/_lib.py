"""ctypes binding of the C ABI in include/soupsuck_amd.h.

The shared library is built in-tree by ``soupsuck_amd.build`` (hipcc, gfx950)
and loaded here on first use.  There is no fallback: when the library is
missing or a call fails, a RuntimeError names the entry point and carries the
library's own error text.  Every call enqueues on torch's current HIP stream
of the tensors' device.
"""

import ctypes
import threading
from pathlib import Path

LIBRARY = Path(__file__).resolve().parent / "libsoupsuck_amd.so"

F16 = 0
F32 = 1

OK = 0
ERR_INVALID_ARGUMENT = -1
ERR_LAUNCH = -2
ERR_UNSUPPORTED = -3

_c_void_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_u64 = ctypes.c_uint64
_int = ctypes.c_int
_f32 = ctypes.c_float
_size = ctypes.c_size_t

# name -> argument types (restype is int unless listed in _RESTYPES)
SIGNATURES = {
    "ss_abi_version": [],
    "ss_last_error": [],
    "ss_nf4_dequant_nested": [_c_void_p] * 6 + [_i64, _c_void_p],
    "ss_nf4_dequant_flat": [_c_void_p] * 3 + [_i64, _c_void_p],
    "ss_nf4_dequant_nested_t": [_c_void_p] * 6 + [_i64, _i64, _c_void_p],
    "ss_nf4_gemm_fwd": [_c_void_p, _i64, _i64] + [_c_void_p] * 5 + [_i64, _i64, _c_void_p,
                                                                   _c_void_p, _i64, _c_void_p,
                                                                   _size, _c_void_p],
    "ss_nf4_gemm_fwd_noalloc": [_c_void_p, _i64, _i64] + [_c_void_p] * 5 + [_i64, _i64,
                                                                            _c_void_p, _c_void_p,
                                                                            _i64, _c_void_p],
    "ss_nf4_gemm_dx": [_c_void_p, _i64, _i64] + [_c_void_p] * 5 + [_i64, _i64, _c_void_p, _i64,
                                                                  _int, _c_void_p, _size,
                                                                  _c_void_p],
    "ss_nf4_gemm_workspace_size": [_i64, _i64, _i64],
    "ss_qlora_fwd": [_c_void_p, _i64, _i64] + [_c_void_p] * 5 + [_i64, _i64, _c_void_p, _c_void_p,
                                                                _c_void_p, _f32, _c_void_p, _i64,
                                                                _c_void_p, _size, _c_void_p],
    "ss_qlora_dx": [_c_void_p, _i64, _i64] + [_c_void_p] * 5 + [_i64, _i64, _c_void_p, _c_void_p,
                                                               _c_void_p, _i64, _c_void_p, _size,
                                                               _c_void_p],
    "ss_qlora_forward": [_c_void_p, _i64, _i64] + [_c_void_p] * 5 + [_i64, _i64] + [_c_void_p] * 3
                        + [_f32, _c_void_p, _c_void_p, _i64, _c_void_p, _size, _c_void_p, _size,
                           _c_void_p],
    "ss_qlora_backward": [_c_void_p, _i64, _i64] + [_c_void_p] * 5 + [_i64, _i64, _c_void_p, _i64]
                         + [_c_void_p] * 3 + [_f32, _c_void_p, _i64] + [_c_void_p] * 3
                         + [_c_void_p, _size, _c_void_p, _size, _c_void_p],
    "ss_qlora_forward_dropout": [_c_void_p, _i64, _i64] + [_c_void_p] * 5 + [_i64, _i64]
                                + [_c_void_p] * 3 + [_f32, _u64, _f32, _c_void_p, _c_void_p,
                                                      _i64, _c_void_p, _size, _c_void_p, _size,
                                                      _c_void_p],
    "ss_qlora_backward_dropout": [_c_void_p, _i64, _i64] + [_c_void_p] * 5
                                 + [_i64, _i64, _c_void_p, _i64] + [_c_void_p] * 3
                                 + [_f32, _u64, _f32, _c_void_p, _i64] + [_c_void_p] * 3
                                 + [_c_void_p, _size, _c_void_p, _size, _c_void_p],
    "ss_dropout_mask": [_u64, _f32, _i64, _i64, _c_void_p, _c_void_p],
    "ss_qlora_rank_workspace_size": [_i64, _i64, _i64],
    "ss_lora_workspace_size": [_i64, _i64],
    "ss_lora_project": [_c_void_p, _i64, _i64, _i64, _c_void_p, _i64, _int, _int, _f32,
                        _c_void_p, _c_void_p, _size, _c_void_p],
    "ss_lora_grad": [_c_void_p, _i64, _c_void_p, _i64, _i64, _i64, _int, _f32, _int, _c_void_p,
                     _c_void_p, _size, _c_void_p],
    "ss_nf4_quantize": [_c_void_p, _int, _i64, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                        _c_void_p, _c_void_p, _c_void_p],
    "ss_gemm_f16": [_int, _int, _i64, _i64, _i64, _f32, _c_void_p, _i64, _c_void_p, _i64,
                    _c_void_p, _f32, _c_void_p, _int, _i64, _c_void_p],
    "ss_gemm_f16_workspace_size": [_int, _int, _i64, _i64, _i64],
    "ss_gemm_f16_split": [_int, _int, _i64, _i64, _i64, _f32, _c_void_p, _c_void_p, _i64,
                          _c_void_p, _i64, _c_void_p, _f32, _c_void_p, _int, _i64, _c_void_p,
                          _size, _c_void_p],
    "ss_lora_epilogue_fwd": [_c_void_p, _int, _c_void_p, _int, _c_void_p, _int, _i64, _f32, _int,
                             _c_void_p],
    "ss_lora_epilogue_bwd": [_c_void_p, _int, _c_void_p, _int, _i64, _f32, _c_void_p],
    "ss_nf4_gemm_fwd_swiglu": [_c_void_p, _i64, _i64] + [_c_void_p] * 5 + [_i64, _i64, _c_void_p,
                                                                           _i64, _c_void_p, _i64,
                                                                           _c_void_p, _i64,
                                                                           _c_void_p, _size,
                                                                           _c_void_p],
    "ss_nf4_gemm_dx_swiglu": [_c_void_p, _i64, _i64] + [_c_void_p] * 5 + [_i64, _i64]
                             + [_c_void_p, _i64] * 4 + [_c_void_p, _size, _c_void_p],
    "ss_rope_fwd": [_c_void_p, _int, _i64, _i64, _i64] * 2 + [_c_void_p, _c_void_p, _int]
                   + [_i64] * 5 + [_c_void_p, _int] * 2 + [_i64] * 5 + [_c_void_p],
    "ss_rope_bwd": [_c_void_p, _int, _i64, _i64, _i64, _i64] * 2 + [_c_void_p, _c_void_p, _int]
                   + [_i64] * 5 + [_c_void_p, _int, _i64, _i64, _i64] * 2 + [_i64] * 5
                   + [_c_void_p],
    "ss_swiglu_fwd": ([_c_void_p, _int, _i64, _i64] * 3) + [_i64, _i64, _c_void_p],
    "ss_swiglu_bwd": ([_c_void_p, _int, _i64, _i64] * 5) + [_i64, _i64, _c_void_p],
    "ss_add_rmsnorm_fwd": [_c_void_p, _int, _c_void_p, _int, _c_void_p, _int, _i64, _c_void_p,
                           _int, _c_void_p, _int, _c_void_p, _i64, _i64, _f32, _c_void_p],
    "ss_add_rmsnorm_bwd": [_c_void_p, _int, _c_void_p, _int, _i64, _c_void_p, _c_void_p, _int,
                           _i64, _i64, _c_void_p, _int, _i64, _i64, _c_void_p, _int, _c_void_p,
                           _int, _i64, _i64, _c_void_p],
    "ss_rmsnorm_fwd": [_c_void_p, _int, _i64, _c_void_p, _int, _i64, _c_void_p, _int, _c_void_p,
                       _i64, _i64, _f32, _c_void_p],
    "ss_add_rmsnorm_dgamma_waves": [_i64],
    "ss_add_rmsnorm_bwd_dgamma": [_c_void_p, _int, _c_void_p, _int, _i64, _c_void_p, _c_void_p,
                                  _int, _i64, _i64, _c_void_p, _int, _i64, _i64, _c_void_p, _int,
                                  _c_void_p, _int, _int, _c_void_p, _c_void_p, _int, _i64, _i64,
                                  _c_void_p],
    "ss_rmsnorm_dgamma": [_c_void_p, _int, _c_void_p, _c_void_p, _int, _i64, _i64, _int,
                          _c_void_p, _c_void_p, _int, _i64, _i64, _c_void_p],
    "ss_unpad_gather": [_c_void_p, _i64, _c_void_p, _c_void_p, _i64, _i64, _c_void_p],
    "ss_unpad_inverse": [_c_void_p, _i64, _c_void_p, _i64, _c_void_p],
    "ss_unpad_scatter": [_c_void_p, _i64, _c_void_p, _c_void_p, _i64, _i64, _c_void_p],
    "ss_ce_stats": [_c_void_p, _i64, _c_void_p, _c_void_p, _c_void_p] + [_i64] * 7 +
                   [_c_void_p],
    "ss_ce_outputs": [_c_void_p, _c_void_p, _i64] + [_c_void_p] * 5 + [_i64, _i64, _c_void_p],
    "ss_ce_derivative": [_c_void_p, _i64, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                         _c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _i64, _c_void_p],
    "ss_ce_rows": [_c_void_p, _i64, _i64, _i64, _c_void_p, _i64, _c_void_p, _c_void_p, _c_void_p],
    "ss_ce_head_gain": [_c_void_p, _i64, _c_void_p, _c_void_p],
    "ss_attn_varlen_fwd": [_c_void_p, _i64, _i64] * 3 + [_c_void_p, _int, _int, _i64, _int,
                                                           _int, _int, _f32, _c_void_p, _i64,
                                                           _i64, _c_void_p, _c_void_p],
    "ss_attn_varlen_bwd": [_c_void_p, _i64, _i64] * 5 + [_c_void_p, _c_void_p, _int, _int, _i64,
                                                           _int, _int, _int, _f32]
                          + [_c_void_p, _i64, _i64] * 3 + [_c_void_p, _size, _c_void_p],
    "ss_attn_varlen_bwd_workspace_size": [_int, _int, _i64],
    "ss_f32_to_f16_exact": [_c_void_p, _c_void_p, _i64, _c_void_p, _c_void_p],
    "ss_hbm_read_probe": [_c_void_p, _i64, _i64, _c_void_p, _c_void_p],
    "ss_ce_finalize_dx": [_c_void_p, _i64, _c_void_p, _c_void_p, _c_void_p, _int, _i64, _i64,
                          _c_void_p],
}
_RESTYPES = {"ss_last_error": ctypes.c_char_p, "ss_nf4_gemm_workspace_size": _size,
             "ss_lora_workspace_size": _size, "ss_qlora_rank_workspace_size": _size,
             "ss_gemm_f16_workspace_size": _size, "ss_add_rmsnorm_dgamma_waves": _i64,
             "ss_attn_varlen_bwd_workspace_size": _size}

_lock = threading.Lock()
_lib = None

# Optional timing hooks: entry-point name -> (before, after) callables, run
# around the call on the calling thread.  Empty unless a benchmark installs one.
hooks = {}


def load(path=None):
    """Load (once) and return the ctypes handle; raise if the library is absent."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        target = Path(path) if path else LIBRARY
        if not target.exists():
            raise RuntimeError(
                f"soupsuck_amd: HIP library {target} is not built; run "
                "`python -m soupsuck_amd.build` (hipcc, gfx950) first")
        lib = ctypes.CDLL(str(target))
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = _RESTYPES.get(name, _int)
        if lib.ss_abi_version() != 1:
            raise RuntimeError("soupsuck_amd: ABI version mismatch")
        if path is None:
            _lib = lib
        return lib


def call(name, *args):
    """Invoke an entry point; raise RuntimeError (or ValueError for bad args) on failure."""
    lib = load()
    hook = hooks.get(name)
    if hook is None:
        rc = getattr(lib, name)(*args)
    else:
        hook[0](name, args)
        rc = getattr(lib, name)(*args)
        hook[1](name, args)
    if rc != OK:
        message = lib.ss_last_error().decode(errors="replace")
        if rc == ERR_INVALID_ARGUMENT:
            raise ValueError(f"{name}: {message}")
        raise RuntimeError(f"{name} failed ({rc}): {message}")
    return rc


def ptr(t):
    """Device address of a tensor (or None)."""
    return None if t is None else t.data_ptr()


def stream(device=None):
    """Raw hipStream_t of torch's current stream on ``device`` (a torch.device, an index,
    or None for the current device), read without building a Stream object."""
    import torch

    if isinstance(device, torch.device):
        index = device.index
    else:
        index = device
    if index is None:
        index = torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(index)


def dtype_code(dtype):
    import torch

    if dtype == torch.float16:
        return F16
    if dtype == torch.float32:
        return F32
    raise ValueError(f"unsupported dtype {dtype}; expected float16 or float32")
