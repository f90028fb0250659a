"""CPU pins of the RoPE oracle (solution/kernels/rope.py:24-98).

Closed forms (identity and the quarter turn), transformers' eager formula
x cos + rotate_half(x) sin in float64 (written independently of the oracle),
and the adjoint identity <F(x), g> = <x, B(g)> that ties the backward to the
forward; a planted sign mistake in the backward must break the adjoint pin.
"""

import numpy as np

from oracle import rope as orope


def _angles(b, s, d, seed=0):
    rng = np.random.default_rng(seed)
    inv = 1.0 / (10000 ** (np.arange(0, d, 2) / d))
    pos = np.arange(s)[:, None] + rng.integers(0, 50)
    freqs = pos * inv[None, :]
    emb = np.concatenate([freqs, freqs], axis=-1)
    return np.cos(emb)[None].repeat(b, 0), np.sin(emb)[None].repeat(b, 0)


def test_identity_and_quarter_turn():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((2, 3, 5, 8)).astype(np.float32)
    one, zero = np.ones((1, 5, 8), np.float32), np.zeros((1, 5, 8), np.float32)
    np.testing.assert_array_equal(orope.rope_forward(x, one, zero), x)
    y = orope.rope_forward(x, zero, one)
    np.testing.assert_array_equal(y[..., :4], -x[..., 4:])
    np.testing.assert_array_equal(y[..., 4:], x[..., :4])


def test_matches_eager_rotate_half_float64():
    b, h, s, d = 2, 3, 7, 16
    cos, sin = _angles(b, s, d)
    x = np.random.default_rng(2).standard_normal((b, h, s, d))
    half = d // 2
    rot = np.concatenate([-x[..., half:], x[..., :half]], axis=-1)
    eager = x * cos[:, None] + rot * sin[:, None]
    np.testing.assert_allclose(orope.rope_forward(x, cos, sin), eager, rtol=1e-14, atol=1e-15)


def _adjoint_gap(backward):
    b, h, s, d = 1, 2, 9, 32
    cos, sin = _angles(b, s, d, seed=3)
    rng = np.random.default_rng(4)
    x, g = rng.standard_normal((b, h, s, d)), rng.standard_normal((b, h, s, d))
    lhs = (orope.rope_forward(x, cos, sin) * g).sum()
    rhs = (x * backward(g, cos, sin, np.float64)).sum()
    return abs(lhs - rhs)


def test_backward_is_the_adjoint():
    assert _adjoint_gap(orope.rope_backward) < 1e-10


def test_planted_sign_mistake_breaks_the_adjoint():
    def wrong(g, cos, sin, dt):
        half = g.shape[-1] // 2
        c, s_ = cos[:, None], sin[:, None]
        g1, g2 = g[..., :half], g[..., half:]
        return np.concatenate([g1 * c[..., :half] - g2 * s_[..., half:],
                               g2 * c[..., half:] - g1 * s_[..., :half]], axis=-1)
    assert _adjoint_gap(wrong) > 1e-3


def test_dtype_promotion():
    x = np.ones((1, 1, 2, 4), np.float16)
    c32 = np.ones((1, 2, 4), np.float32)
    assert orope.rope_forward(x, c32, c32).dtype == np.float32
    assert orope.rope_forward(x, c32.astype(np.float16), c32.astype(np.float16)).dtype == np.float16
    assert orope.rope_backward(x, c32, c32, np.float16).dtype == np.float16
