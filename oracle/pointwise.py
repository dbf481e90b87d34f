"""RoPE, RMSNorm and SwiGLU in float64.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Follows the reference:
  - rope:    tests/test_rope.py:43-59 (rotate-half, complex form, fp64 angle
             pos * theta^(-2j/hd)); kernel src/core_kernels/rope.cu:32-54
  - rmsnorm: tests/test_rmsnorm.py:28-32; kernel src/core_kernels/rmsnorm.cu:33-84
  - swiglu:  tests/test_swiglu.py:23-25; kernel src/core_kernels/swiglu.cu:26-38

PINNED by (tests/test_oracle_pointwise.py): rope at position 0 is the
identity and preserves each pair's norm; two rotations compose (pos a then b
equals a + b); rmsnorm of a constant row is sign(x)*w/sqrt(1+eps/x^2), and
the output's mean square with w=1 is 1/(1+eps/ms); swiglu(0, u) = 0,
swiglu(g, 1) is g*sigmoid(g) checked against math.exp scalars.
"""

from __future__ import annotations

import numpy as np


def rope(x: np.ndarray, positions: np.ndarray, theta: float) -> np.ndarray:
    """x (seq, heads, hd) -> rotated, float64."""
    hd = x.shape[-1]
    half = hd // 2
    x64 = np.asarray(x, np.float64)
    inv_freq = theta ** (-np.arange(half, dtype=np.float64) * 2.0 / hd)
    angle = np.asarray(positions, np.float64)[:, None] * inv_freq[None, :]
    rot = np.exp(1j * angle)[:, None, :]
    z = (x64[..., :half] + 1j * x64[..., half:]) * rot
    return np.concatenate([z.real, z.imag], axis=-1)


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x64 = np.asarray(x, np.float64)
    ms = np.mean(x64 * x64, axis=-1, keepdims=True)
    return (x64 / np.sqrt(ms + eps)) * np.asarray(w, np.float64)


def swiglu(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    g = np.asarray(gate, np.float64)
    with np.errstate(over="ignore"):
        return g / (1.0 + np.exp(-g)) * np.asarray(up, np.float64)
