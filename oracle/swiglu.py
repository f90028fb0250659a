"""SwiGLU activation oracle -- test infrastructure only.

Reference semantics (solution/kernels/swiglu_fused.py:20-46, the
``swiglu_tile_engine`` used by solution/mlp.py:500-612): gate g and up u are
read and widened to fp32, then
  p   = 1 / (1 + exp(-g))
  act = g * p
  forward   a  = act * u                          stored in the output's dtype
  backward  slope = p + act * (1 - p)
            dg = (da * u) * slope,  du = da * act  stored in each grad's dtype
(swiglu_fused.py:33-46; the tile engine is compiled with enable_fp_fusion=False,
so every product and sum is its own fp32 rounding).

Two restatements are kept: ``*_fp32`` follows the reference's fp32 operation
order exactly (numpy float32, one rounding per operation, exp in float32),
``*_exact`` evaluates the same formula in float64 and rounds once to the
output dtype.  A device kernel is held to both: within 1 fp16 ulp of the
float64 value for fp16 outputs, and within a relative 2e-6 of the fp32 order
for fp32 outputs (exp is not correctly rounded on either side).

Pins (tests/test_oracle_swiglu.py): closed forms silu(0) = 0 and slope(0) = 1/2,
the limits act -> g, slope -> 1 for g -> +inf and act -> 0, slope -> 0 for
g -> -inf; the backward against a central finite difference of the float64
forward; and the forward/backward against torch.nn.functional.silu and its
autograd in float64 on the CPU, a separately written formula for the same
quantities.
"""

import numpy as np

F32 = np.float32


def _sigmoid64(g):
    g = np.asarray(g, np.float64)
    with np.errstate(over="ignore"):
        return 1.0 / (1.0 + np.exp(-g))


def swiglu_forward_exact(gate, up, out_dtype=np.float16):
    """a = silu(g) * u in float64, rounded once to out_dtype."""
    g = np.asarray(gate).astype(np.float64)
    u = np.asarray(up).astype(np.float64)
    return (g * _sigmoid64(g) * u).astype(out_dtype)


def swiglu_backward_exact(gate, up, grad, gate_dtype=np.float16, up_dtype=np.float16):
    """(dg, du) of a = silu(g) * u in float64, each rounded once."""
    g = np.asarray(gate).astype(np.float64)
    u = np.asarray(up).astype(np.float64)
    da = np.asarray(grad).astype(np.float64)
    p = _sigmoid64(g)
    act = g * p
    slope = p + act * (1.0 - p)
    return (da * u * slope).astype(gate_dtype), (da * act).astype(up_dtype)


def _fp32_terms(gate):
    g = np.asarray(gate).astype(F32)
    with np.errstate(over="ignore"):
        e = np.exp(-g, dtype=F32)
    p = (F32(1.0) / (F32(1.0) + e)).astype(F32)
    act = (g * p).astype(F32)
    return g, p, act


def swiglu_forward_fp32(gate, up, out_dtype=np.float16):
    """The reference's fp32 operation order (swiglu_fused.py:33-46), unfused."""
    _, _, act = _fp32_terms(gate)
    u = np.asarray(up).astype(F32)
    return (act * u).astype(F32).astype(out_dtype)


def swiglu_backward_fp32(gate, up, grad, gate_dtype=np.float16, up_dtype=np.float16):
    _, p, act = _fp32_terms(gate)
    u = np.asarray(up).astype(F32)
    da = np.asarray(grad).astype(F32)
    slope = (p + (act * (F32(1.0) - p)).astype(F32)).astype(F32)
    dg = ((da * u).astype(F32) * slope).astype(F32)
    du = (da * act).astype(F32)
    return dg.astype(gate_dtype), du.astype(up_dtype)
