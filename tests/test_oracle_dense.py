"""The dense oracle pinned (no device): the projection by hand and by
identity, the term magnitudes by the triangle inequality, the argmax rule
against a scalar loop, the gather; and the gate the projection is held to
rejects fp16 accumulation (tests/test_linear.py:109-131)."""

import math

import numpy as np
import pytest

from conftest import accumulation_floor, assert_within_gate, fp16_exact
from oracle import dense


def test_linear_by_hand_by_identity_and_by_bias_alone():
    x = np.array([[1.0, 2.0, -3.0], [0.5, 0.0, 4.0]])
    w = np.array([[2.0, 0.0, 1.0], [-1.0, 1.0, 0.25]])
    got, terms = dense.linear(x, w, np.array([10.0, -1.0]))
    want = [[1 * 2 + 2 * 0 - 3 * 1 + 10, -1 + 2 - 0.75 - 1], [1 + 0 + 4 + 10, -0.5 + 0 + 1 - 1]]
    np.testing.assert_array_equal(got, want)
    np.testing.assert_array_equal(terms, [[2 + 0 + 3 + 10, 1 + 2 + 0.75 + 1],
                                          [1 + 0 + 4 + 10, 0.5 + 0 + 1 + 1]])
    rng = np.random.default_rng(0)
    x = rng.standard_normal((5, 7))
    np.testing.assert_array_equal(dense.linear(x, np.eye(7))[0], x)
    w = rng.standard_normal((9, 7))
    y, t = dense.linear(x, w, chunk=4)                   # slabs agree with one product
    np.testing.assert_allclose(y, x @ w.T, rtol=1e-12)
    assert np.all(np.abs(y) <= t * (1 + 1e-12))
    np.testing.assert_array_equal(dense.linear(np.zeros((2, 3)), np.zeros((4, 3)),
                                               np.arange(4.0))[0], [np.arange(4.0)] * 2)


def scalar_argmax(row):
    best, at = -dense.FLT_MAX, len(row)
    for i, v in enumerate(row):
        v = float(v)
        if v > best or (v == best and i < at):
            best, at = v, i
    return at


def test_argmax_is_the_scalar_rule_on_ties_nan_and_infinities():
    f = dense.FLT_MAX
    rows = np.array([
        [1.0, 3.0, 3.0, 2.0],
        [np.nan, 0.5, np.nan, 0.5],
        [-np.inf, -np.inf, -np.inf, -np.inf],
        [np.nan, np.nan, np.nan, np.nan],
        [-f, -np.inf, -f, np.nan],
        [np.inf, 1.0, np.inf, -1.0],
        [-2.0, -1.0, -3.0, -1.0],
    ], np.float32)
    want = [scalar_argmax(r) for r in rows]
    assert want == [1, 1, 4, 4, 0, 0, 1]
    np.testing.assert_array_equal(dense.argmax_rows(rows), want)
    rng = np.random.default_rng(3)
    x = rng.integers(-3, 4, size=(200, 37)).astype(np.float32)   # many ties
    x[rng.random(x.shape) < 0.1] = np.nan
    np.testing.assert_array_equal(dense.argmax_rows(x), [scalar_argmax(r) for r in x])


def test_embed_gathers_and_zeroes_unknown_ids():
    table = np.arange(12, dtype=np.float16).reshape(4, 3)
    got = dense.embed([2, -1, 0, 4, 3], table)
    np.testing.assert_array_equal(got, [[6, 7, 8], [0, 0, 0], [0, 1, 2], [0, 0, 0], [9, 10, 11]])


def test_the_gate_rejects_fp16_accumulation_and_holds_fp32():
    rng = np.random.default_rng(13)
    x = fp16_exact(rng.standard_normal((2, 4864)))
    w = fp16_exact(rng.standard_normal((256, 4864)) / math.sqrt(4864))
    want, terms = dense.linear(x, w)
    fp32 = (x.astype(np.float32) @ w.astype(np.float32).T).astype(np.float16)
    assert_within_gate(fp32, want, accumulation_floor(terms, x.shape[1]))
    products = (x[:, None, :] * w[None, :, :]).astype(np.float16)
    fp16_accumulated = np.cumsum(products, axis=-1, dtype=np.float16)[..., -1]
    with pytest.raises(AssertionError):
        assert_within_gate(fp16_accumulated, want, accumulation_floor(terms, x.shape[1]))
