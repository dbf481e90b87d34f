"""The standalone ImportanceScores.fold on the device (the call the
reference's PagedCache.attend makes after each scored decode step,
model.py:280-286): to the bit against the oracle's fp32 fold, at the default
alpha and another, over several layers and steps; a page's first observation
seeds its score; a refused fold changes nothing.

GPU parity tests. Scores are compared bit for bit (importance_scores.cu:31-50,
tests/test_importance_scores.py:85-115)."""

import numpy as np
import pytest

from conftest import announce, each
from oracle import ewma

pytestmark = pytest.mark.gpu

f32 = np.float32


def mi():
    from microinfer import _microinfer
    return _microinfer


def masses(rng, heads, pages):
    """Softmax shares per head over `pages` pages, with exact zeros (unread
    pages) and a few tiny values, fp32."""
    w = rng.exponential(1.0, (heads, pages)).astype(np.float64)
    w[:, rng.random(pages) < 0.1] = 0.0
    w[:, rng.random(pages) < 0.05] *= 1e-30
    w /= np.maximum(w.sum(1, keepdims=True), 1e-300)
    return w.astype(f32)


def test_standalone_fold_is_the_oracle_fold_to_the_bit():
    d = mi().device

    def check(alpha, heads):
        rng = np.random.default_rng(heads * 10 + (0 if alpha is None else 1))
        layers, max_pages = 4, 300
        scores = (d.ImportanceScores(layers, max_pages) if alpha is None
                  else d.ImportanceScores(layers, max_pages, alpha))
        a = ewma.DEFAULT_ALPHA if alpha is None else f32(alpha)
        assert scores.alpha == pytest.approx(float(a))
        steps = []
        # Contexts that grow: each step folds one page more than the last on
        # some layers, as a decode does every 32 tokens.
        for step in range(24):
            layer = step % layers
            pages = 200 + step * 4
            m = masses(rng, heads, pages)
            steps.append((layer, m))
            announce("fold", alpha, heads, step)
            scores.fold(layer, d.upload_f32(m.ravel()), heads, pages)
        got = scores.download()
        want = ewma.host_ewma(steps, layers, max_pages, a)
        np.testing.assert_array_equal(got, want)
        assert scores.downloads == 1

    each([(None, 12), (0.5, 12), (None, 14), (0.2, 32), (0.75, 1)], check)


def test_first_observation_seeds_and_the_known_answer():
    """tests/test_importance_scores.py:106-115: mass [[.5,.25,.25],
    [.7,.2,.1]] on layer 1 gives (0.6, 0.225, 0.175), the rest NaN."""
    d = mi().device
    scores = d.ImportanceScores(2, 8)
    mass = np.array([[0.5, 0.25, 0.25], [0.7, 0.2, 0.1]], f32)
    announce("fold known answer")
    scores.fold(1, d.upload_f32(mass.ravel()), 2, 3)
    got = scores.download()
    np.testing.assert_array_equal(got[1, :3], ((mass[0] + mass[1]) / f32(2)).astype(f32))
    np.testing.assert_allclose(got[1, :3], [0.6, 0.225, 0.175], rtol=1e-6)
    assert np.isnan(got[1, 3:]).all() and np.isnan(got[0]).all()


def test_a_refused_fold_changes_nothing():
    d = mi().device
    m = mi()
    scores = d.ImportanceScores(2, 8)
    mass = np.full((3, 8), 0.125, f32)
    scores.fold(0, d.upload_f32(mass.ravel()), 3, 8)
    before = scores.download()
    with pytest.raises(IndexError):
        scores.fold(2, d.upload_f32(mass.ravel()), 3, 8)
    with pytest.raises(ValueError):
        scores.fold(0, d.upload_f32(mass.ravel()), 3, 9)
    np.testing.assert_array_equal(scores.download(), before)
    assert isinstance(m.OutOfMemory("x"), MemoryError)
