"""LoRA epilogue and LoRA branch oracles (A10-A12) -- test infrastructure only.

Reference semantics:
  * epilogue forward (solution/kernels/lora_epilogue.py:1-13,24-34,49-58):
        out_dtype = base dtype if cast_to_result else promote(base, adapter)
        scaled = cast_adapter(fp32(adapter) * s); if cast_to_result: scaled = cast_base(scaled)
        out = round_out(fp32(base) + fp32(scaled))
    i.e. the scaled product is rounded to the adapter dtype BEFORE the add;
  * epilogue backward (lora_epilogue.py:37-43,61-76):
        d_result = grad.to(base dtype); d_adapter = cast_adapter(fp32(cast_adapter(grad)) * s);
  * LoRA branch under fp16 autocast (solution/lora.py:151-163,
    solution/lora_pair.py:34-65): Z = fp16(X.A^T), L = fp16(Z.B^T); backward
    dZ = fp16(dL.B), dB = fp16(dL^T.Z), dA = fp16(dZ^T.X), dX = fp16(dZ.A),
    with dL the epilogue's d_adapter.

Pins: known answer "the rounded product cancels to exactly zero"
(solution/tests/test_lora.py:41-49: base = -(a*s) rounded, out == 0), which
an fused multiply-add or a missing intermediate rounding fails; the LoRA
gradients are checked against central finite differences in float64.
"""

import numpy as np

F16 = np.float16
F32 = np.float32


def _promote(a, b):
    return np.promote_types(a, b)


def epilogue_forward(base, adapter, s, cast_to_result=False):
    base = np.asarray(base)
    adapter = np.asarray(adapter)
    out_dtype = base.dtype if cast_to_result else _promote(base.dtype, adapter.dtype)
    scaled = (adapter.astype(F32) * F32(s)).astype(F32).astype(adapter.dtype).astype(F32)
    if cast_to_result:
        scaled = scaled.astype(base.dtype).astype(F32)
    return (base.astype(F32) + scaled).astype(F32).astype(out_dtype)


def epilogue_backward(grad, base_dtype, adapter_dtype, s):
    grad = np.asarray(grad)
    d_result = grad.astype(base_dtype)
    branch = grad.astype(adapter_dtype).astype(F32)
    d_adapter = (branch * F32(s)).astype(F32).astype(adapter_dtype)
    return d_result, d_adapter


def branch_forward(x, a, b):
    """Z = fp16(X.A^T), L = fp16(Z.B^T) with fp64 products (autocast fp16 GEMMs)."""
    z = (np.asarray(x, np.float64) @ np.asarray(a, np.float64).T).astype(F16)
    lora = (z.astype(np.float64) @ np.asarray(b, np.float64).T).astype(F16)
    return z, lora


def branch_backward(d_lora, x, a, b, z):
    """dZ, dB, dA, dX of the LoRA pair (solution/lora_pair.py:52-65), fp64 then fp16."""
    dl = np.asarray(d_lora, np.float64)
    dz = (dl @ np.asarray(b, np.float64)).astype(F16)
    db = (dl.T @ np.asarray(z, np.float64)).astype(F16)
    da = (dz.astype(np.float64).T @ np.asarray(x, np.float64)).astype(F16)
    dx = (dz.astype(np.float64) @ np.asarray(a, np.float64)).astype(F16)
    return dz, db, da, dx


def ideal_projection(x, w, bias, a, b, s):
    """float64 Y = X.W^T + bias + s * (X.A^T).B^T, the unrounded target."""
    x = np.asarray(x, np.float64)
    y = x @ np.asarray(w, np.float64).T
    if bias is not None:
        y = y + np.asarray(bias, np.float64)[None, :]
    return y + s * ((x @ np.asarray(a, np.float64).T) @ np.asarray(b, np.float64).T)


def ideal_projection_backward(g, x, w, a, b, s):
    """float64 gradients of ``ideal_projection`` w.r.t. X, A, B."""
    g = np.asarray(g, np.float64)
    x = np.asarray(x, np.float64)
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    z = x @ a.T
    dl = s * g
    dz = dl @ b
    dx = g @ np.asarray(w, np.float64) + dz @ a
    return dx, dz.T @ x, dl.T @ z
