"""The importance score's EWMA, in fp32, in the device's order.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Follows the reference:
  - fold:   src/core_kernels/importance_scores.cu:31-50 (per page: each head's
            mass added in head order, divided by the head count, then
            alpha*obs + (1-alpha)*old, every operation rounded once, a NaN
            old score seeded by the observation)
  - host:   tests/test_importance_scores.py:32-47 (host_ewma)

PINNED by (tests/test_oracle_ewma.py): the known answer of
tests/test_importance_scores.py:106-115 (mass [[.5,.25,.25],[.7,.2,.1]] ->
(0.6, 0.225, 0.175), the rest NaN); the float64 EWMA of :53-63 within 4 fp32
ulps; a scalar Python restatement with math.fsum-free sequential float32
steps on a few pages.
"""

from __future__ import annotations

import numpy as np

f32 = np.float32
DEFAULT_ALPHA = f32(0.2)   # importance_scores.h:31


def fold(scores: np.ndarray, layer: int, mass: np.ndarray, alpha=DEFAULT_ALPHA) -> None:
    """Fold one step's mass (heads, pages) fp32 into scores (layers,
    max_pages) fp32, in place, exactly as the fold kernel rounds."""
    mass = np.asarray(mass, f32)
    heads, pages = mass.shape
    total = np.zeros(pages, f32)
    for h in range(heads):
        total = (total + mass[h]).astype(f32)
    observed = (total / f32(heads)).astype(f32)
    alpha = f32(alpha)
    keep = (f32(1) - alpha).astype(f32)
    old = scores[layer, :pages]
    new = ((alpha * observed).astype(f32) + (keep * old).astype(f32)).astype(f32)
    scores[layer, :pages] = np.where(np.isnan(old), observed, new)


def host_ewma(steps, layers: int, max_pages: int, alpha=DEFAULT_ALPHA) -> np.ndarray:
    """The scores a sequence of (layer, mass) folds leaves, NaN-seeded."""
    scores = np.full((layers, max_pages), np.nan, f32)
    for layer, mass in steps:
        fold(scores, layer, mass, alpha)
    return scores


def float64_ewma(steps, layers: int, max_pages: int, alpha=0.2) -> np.ndarray:
    """tests/test_importance_scores.py:53-63: the same EWMA in float64."""
    scores = np.full((layers, max_pages), np.nan)
    for layer, mass in steps:
        mean = np.asarray(mass, np.float64).mean(axis=0)
        old = scores[layer, :mass.shape[1]]
        scores[layer, :mass.shape[1]] = np.where(np.isnan(old), mean,
                                                 alpha * mean + (1 - alpha) * old)
    return scores
