"""The oracle's EWMA, pinned by the reference's known answer, the float64
EWMA and a scalar restatement. CPU only."""

import json

import numpy as np

from conftest import GOLDEN
from oracle import ewma

f32 = np.float32


def random_masses(rng, layers, heads, steps, start_pages):
    """tests/test_importance_scores.py:66-76."""
    out = []
    for t in range(steps):
        pages = start_pages + t // 3
        for layer in range(layers):
            m = rng.random((heads, pages)).astype(f32)
            out.append((layer, (m / m.sum(axis=1, keepdims=True)).astype(f32)))
    return out


def test_first_observation_known_answer():
    k = json.loads((GOLDEN / "known_answers.json").read_text())["ewma_first_observation"]
    mass = np.array(k["mass"], f32)
    scores = ewma.host_ewma([(k["layer"], mass)], k["layers"], k["max_pages"])
    np.testing.assert_array_equal(scores[1, :3], np.array(k["expected_first_pages"], f32))
    np.testing.assert_array_equal(scores[1, :3], ((mass[0] + mass[1]) / f32(2)).astype(f32))
    assert np.isnan(scores[1, 3:]).all() and np.isnan(scores[0]).all()


def test_within_four_ulps_of_float64():
    for alpha in (0.2, 0.5):
        steps = random_masses(np.random.default_rng(99), 3, 12, 30, 5)
        got = ewma.host_ewma(steps, 3, 40, f32(alpha))
        exact = ewma.float64_ewma(steps, 3, 40, float(f32(alpha)))
        assert (np.isnan(got) == np.isnan(exact)).all()
        seen = ~np.isnan(exact)
        assert np.abs(got[seen] - exact[seen]).max() < 4 * np.finfo(f32).eps


def test_scalar_restatement():
    """Each page folded with numpy float32 scalars, one operation at a time."""
    rng = np.random.default_rng(4)
    steps = random_masses(rng, 1, 5, 6, 3)
    got = ewma.host_ewma(steps, 1, 8)
    scores = [f32(np.nan)] * 8
    a = f32(0.2)
    keep = f32(f32(1) - a)
    for _, mass in steps:
        for p in range(mass.shape[1]):
            total = f32(0)
            for h in range(mass.shape[0]):
                total = f32(total + mass[h, p])
            obs = f32(total / f32(mass.shape[0]))
            old = scores[p]
            scores[p] = obs if np.isnan(old) else f32(f32(a * obs) + f32(keep * old))
    np.testing.assert_array_equal(got[0], np.array(scores, f32))
