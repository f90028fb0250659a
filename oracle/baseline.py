"""CPU baseline of the QLoRA projection step -- test infrastructure only.

The reference's CPU-visible structure for a Linear4bit projection is
"dequantize, then dense matmul" (bitsandbytes fallback, reference
solution/nf4_patch.py:4-7,108-120, backward tasks/RUNTIME_AUDIT.md:113), with
the LoRA branch and epilogue of solution/lora.py:135-163.  This module runs
exactly that on the host: the A2 decode of oracle.nf4 followed by float32
numpy GEMMs (multi-threaded BLAS) for the forward and the dX/dA/dB backward.
It is timed by bench.py as the reported ``cpu_baseline`` (kind "port"); it is
never the measured product.
"""

import numpy as np

from . import nf4


def projection_step(x, state, a, b, bias, g, scaling):
    """One QLoRA projection forward + backward on the CPU; returns (out, dx, da, db)."""
    w = state.decode().astype(np.float32)                     # [N, K], bit-exact fp16 values
    x32 = x.astype(np.float32)
    a32, b32 = a.astype(np.float32), b.astype(np.float32)
    y = x32 @ w.T
    if bias is not None:
        y += bias.astype(np.float32)
    z = (x32 @ a32.T).astype(np.float16).astype(np.float32)
    lora = (z @ b32.T).astype(np.float16).astype(np.float32)
    out = (y.astype(np.float16).astype(np.float32)
           + (lora * np.float32(scaling)).astype(np.float16).astype(np.float32)).astype(np.float16)
    g32 = g.astype(np.float32)
    dl = (g32 * np.float32(scaling)).astype(np.float16).astype(np.float32)
    dz = dl @ b32
    db = dl.T @ z
    da = dz.T @ x32
    dx = g32 @ w + dz @ a32
    return out, dx.astype(np.float16), da.astype(np.float16), db.astype(np.float16)
