"""The oracle's RoPE, RMSNorm and SwiGLU, pinned by invariants and closed
forms. CPU only."""

import math

import numpy as np

from oracle import pointwise


def test_rope_identity_norm_and_composition():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((3, 2, 16))
    np.testing.assert_allclose(pointwise.rope(x, np.zeros(3), 1e6), x, rtol=0, atol=0)
    r = pointwise.rope(x, np.array([5, 77, 32767]), 1e6)
    half = 8
    np.testing.assert_allclose(np.hypot(r[..., :half], r[..., half:]),
                               np.hypot(x[..., :half], x[..., half:]), rtol=1e-12)
    a, b = np.array([3, 100, 2000]), np.array([11, 7, 30000])
    np.testing.assert_allclose(pointwise.rope(pointwise.rope(x, a, 1e4), b, 1e4),
                               pointwise.rope(x, a + b, 1e4), rtol=1e-9, atol=1e-9)


def test_rmsnorm_closed_forms():
    w = np.linspace(0.5, 1.5, 8)
    x = np.full((1, 8), -3.0)
    want = -w / math.sqrt(1 + 1e-6 / 9.0)
    np.testing.assert_allclose(pointwise.rmsnorm(x, w, 1e-6)[0], want, rtol=1e-14)
    rng = np.random.default_rng(1)
    x = rng.standard_normal((4, 64))
    y = pointwise.rmsnorm(x, np.ones(64), 1e-6)
    ms = (x * x).mean(-1)
    np.testing.assert_allclose((y * y).mean(-1), ms / (ms + 1e-6), rtol=1e-12)


def test_swiglu_closed_forms():
    g = np.array([-100.0, -3.0, 0.0, 0.5, 20.0])
    np.testing.assert_array_equal(pointwise.swiglu(np.zeros(3), np.ones(3)), np.zeros(3))
    want = [x / (1 + math.exp(-x)) for x in g]
    np.testing.assert_allclose(pointwise.swiglu(g, np.ones(5)), want, rtol=1e-15)
