"""The dense projection, the embedding gather and the greedy argmax.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Follows the reference:
  - linear:  tests/test_linear.py:46-65 (float64 x @ w.T + bias, with the
             per-output magnitude of the summed terms, |x| @ |w|.T + |b|,
             which bounds the error where terms cancel); kernel
             src/core_kernels/linear.cu:85-138
  - embed:   src/core_kernels/embed.cu:17-40 (a gather; an id outside the
             vocabulary reads as a zero row)
  - argmax:  src/core_kernels/argmax.cu:17-68 (the larger value, the lower
             index on a tie, NaN never chosen, `cols` for a row with nothing
             >= -FLT_MAX)

PINNED by (tests/test_oracle_dense.py): linear against hand-computed 2x3
products, an identity weight returning x, and a bias-only row; the terms
against the triangle inequality; argmax against a scalar loop over rows
with ties, NaN, -inf and -FLT_MAX.
"""

from __future__ import annotations

import numpy as np

FLT_MAX = float(np.finfo(np.float32).max)


def linear(x, w, bias=None, chunk: int = 16384):
    """float64 x @ w.T (+ bias) and, per output, the summed magnitudes of its
    terms. Slabs of output features keep a large head's weight from being
    held in float64 whole."""
    x64 = np.asarray(x, np.float64)
    w = np.asarray(w)
    out = np.empty((x64.shape[0], w.shape[0]), np.float64)
    terms = np.empty_like(out)
    for start in range(0, w.shape[0], chunk):
        slab = w[start:start + chunk].astype(np.float64).T
        out[:, start:start + chunk] = x64 @ slab
        terms[:, start:start + chunk] = np.abs(x64) @ np.abs(slab)
    if bias is not None:
        b = np.asarray(bias, np.float64)
        out += b
        terms += np.abs(b)
    return out, terms


def embed(ids, table) -> np.ndarray:
    ids = np.asarray(ids, np.int64)
    table = np.asarray(table)
    known = (ids >= 0) & (ids < table.shape[0])
    out = np.zeros((ids.shape[0], table.shape[1]), table.dtype)
    out[known] = table[ids[known]]
    return out


def argmax_rows(x) -> np.ndarray:
    """Per row: the index of the largest value, the lowest index on a tie,
    NaN ignored; the row length for a row with nothing >= -FLT_MAX."""
    x = np.asarray(x, np.float32)
    rows, cols = x.shape
    usable = ~np.isnan(x) & (x >= -FLT_MAX)
    masked = np.where(usable, x, -np.inf)
    best = masked.max(axis=1, initial=-np.inf)
    hit = usable & (masked == best[:, None])
    first = np.where(hit.any(axis=1), hit.argmax(axis=1), cols)
    return first.astype(np.int32)
