"""Joint q/k rotary position embedding oracle -- test infrastructure only.

Reference semantics (solution/kernels/rope.py:1-15,24-98, ``fused_rope`` at
:146-152): q [B, Hq, S, D], k [B, Hk, S, D], cos/sin [1|B, S, D], D even,
half = D / 2, x1 = x[..., :half], x2 = x[..., half:]:
  forward   y1 = R(x1 c1) + R(-x2 s1),  y2 = R(x2 c2) + R(x1 s2)
            with R the rounding to promote(x.dtype, cos.dtype), the sum again
            rounded to that dtype on store;
  backward  d1 = R'(g1 c1) + R'(g2 s2),  d2 = R'(g2 c2) - R'(g1 s1)
            with R' the rounding to x.dtype (the gradient's dtype).
Every product and sum is one fp32 operation on the widened operands (a
product of two fp16 values is exact in fp32), so a device kernel following
this order without contraction is bit-exact against ``rope_forward`` /
``rope_backward`` here.

Pins (tests/test_oracle_rope.py): cos = 1, sin = 0 is the identity; cos = 0,
sin = 1 maps (x1, x2) to (-x2, x1); in float64 the forward equals
transformers' eager ``x * cos + rotate_half(x) * sin`` (a separately written
formula), and the backward is the exact adjoint of the forward
(<F(x), g> = <x, B(g)> for cos/sin of a real rotation).
"""

import numpy as np

F32 = np.float32


def _work(dtype):
    """fp32 arithmetic (the kernels'); float64 only for float64 pins."""
    return np.float64 if np.dtype(dtype) == np.float64 else F32


def _split(x):
    half = x.shape[-1] // 2
    return x[..., :half], x[..., half:]


def _cs(cos, sin, batches):
    c, s = np.asarray(cos), np.asarray(sin)
    if c.shape[0] == 1 and batches != 1:
        c = np.broadcast_to(c, (batches,) + c.shape[1:])
        s = np.broadcast_to(s, (batches,) + s.shape[1:])
    return c[:, None], s[:, None]  # [B, 1, S, D]: broadcast over heads


def rope_forward(x, cos, sin):
    """y of one operand (q or k) in promote(x.dtype, cos.dtype)."""
    x = np.asarray(x)
    out = np.promote_types(x.dtype, np.asarray(cos).dtype)
    w = _work(out)
    c, s = _cs(cos, sin, x.shape[0])
    c1, c2 = (v.astype(w) for v in _split(c))
    s1, s2 = (v.astype(w) for v in _split(s))
    x1, x2 = (v.astype(w) for v in _split(x))

    def r(v):
        return v.astype(w).astype(out).astype(w)

    lo = (r(x1 * c1) + r(-x2 * s1)).astype(out)
    hi = (r(x2 * c2) + r(x1 * s2)).astype(out)
    return np.concatenate([lo, hi], axis=-1)


def rope_backward(g, cos, sin, x_dtype):
    """dx of one operand given its output gradient g, in x_dtype."""
    g = np.asarray(g)
    w = _work(x_dtype)
    c, s = _cs(cos, sin, g.shape[0])
    c1, c2 = (v.astype(w) for v in _split(c))
    s1, s2 = (v.astype(w) for v in _split(s))
    g1, g2 = (v.astype(w) for v in _split(g))

    def r(v):
        return v.astype(w).astype(x_dtype).astype(w)

    lo = (r(g1 * c1) + r(g2 * s2)).astype(x_dtype)
    hi = (r(g2 * c2) - r(g1 * s1)).astype(x_dtype)
    return np.concatenate([lo, hi], axis=-1)
