"""Shared test setup: the package on sys.path, the `gpu` marker, helpers.

`-m "not gpu"` runs here, on the CPU: the oracle against the reference's
known answers and fixtures, the host logic, and that the C ABI library loads
and exports every symbol its header declares. `-m gpu` runs on an MI355X:
the parity tests proper, HIP kernels through the C ABI against the oracle.
"""

import sys
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parent.parent
PACKAGE = REPO / "semantic-aware_adaptive_kv_cache_precision_amd"
for p in (str(REPO), str(PACKAGE)):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = Path(__file__).resolve().parent / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); parity tests")


def fp16_exact(a) -> np.ndarray:
    """Values an fp16 holds exactly, as float32."""
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


def each(cases, check, name=None):
    """Runs check(*case) for every case, reporting every failing case."""
    failures = []
    for case in cases:
        args = case if isinstance(case, tuple) else (case,)
        try:
            check(*args)
        except AssertionError as e:  # collect, then report all
            label = name(case) if name else repr(case)
            failures.append(f"{label}: {e}")
    if failures:
        raise AssertionError(f"{len(failures)} of {len(cases)} cases failed:\n" + "\n".join(failures))


#: Attention outputs: within 1e-3 relative of the float64 oracle (the
#: north_star's bar), with a floor of 1e-4 of the row's largest magnitude for
#: elements that cancel to near zero. The fp16 store alone costs 2^-11.
ATTN_RTOL = 1e-3
ATTN_FLOOR = 1e-4
#: Masses: within 1e-3 relative, plus 32 fp32 ulps at 1.0 absolute, the
#: reference's own mass tolerance (tests/test_attention_mass.py:35-38).
MASS_RTOL = 1e-3
MASS_ATOL = 32 * float(np.finfo(np.float32).eps)


def assert_attention_close(got, want, what=""):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    row = np.abs(want).max(axis=-1, keepdims=True)
    bound = ATTN_RTOL * np.abs(want) + ATTN_FLOOR * row
    err = np.abs(got - want)
    worst = float((err / np.maximum(bound, 1e-300)).max())
    assert np.all(err <= bound), f"{what}: error reaches {worst:.3g} of the bound"


def assert_mass_close(got, want, what=""):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.abs(got - want)
    bound = MASS_RTOL * np.abs(want) + MASS_ATOL
    assert np.all(err <= bound), f"{what}: mass error {err.max():.3g}"


def announce(*what) -> None:
    """Names the case before a GPU step, flushed, so a failed run says where."""
    print("[case]", *what, flush=True)
