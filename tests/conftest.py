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


#: Attention outputs: the reference's error gate (tests/ulp_gate.py:28-103,
#: tests/test_attention.py:58-115) held to the north_star's 1e-3: relative
#: error against the float64 oracle, its denominator floored at fp16's
#: smallest normal (below it the fp16 store errs in absolute terms) and, when
#: the oracle gives attention_bound's fp32 error bound, at the magnitude where
#: that bound spends the whole budget (outputs that cancel to near zero);
#: max below 1e-3 and mean below one fp16 ulp (2^-11).
ATTN_MAX_REL = 1e-3
ATTN_MEAN_REL = 2.0**-11
#: Masses: within 1e-3 relative, plus 32 fp32 ulps at 1.0 absolute, the
#: reference's own mass tolerance (tests/test_attention_mass.py:35-38).
MASS_RTOL = 1e-3
MASS_ATOL = 32 * float(np.finfo(np.float32).eps)


def attention_error(got, want, bound=None):
    """Per element, the gate's relative error (ATTN_MAX_REL's comment)."""
    from oracle.attention import FP16_MIN_NORMAL
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    floor = FP16_MIN_NORMAL
    if bound is not None:
        floor = np.maximum(FP16_MIN_NORMAL, np.asarray(bound, np.float64) / ATTN_MAX_REL)
    return np.abs(got - want) / np.maximum(np.abs(want), floor)


def assert_attention_close(got, want, what="", bound=None):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    err = attention_error(got, want, bound)
    assert err.max() < ATTN_MAX_REL, f"{what}: max relative error {err.max():.3e}"
    assert err.mean() < ATTN_MEAN_REL, f"{what}: mean relative error {err.mean():.3e}"


def assert_mass_close(got, want, what=""):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.abs(got - want)
    bound = MASS_RTOL * np.abs(want) + MASS_ATOL
    assert np.all(err <= bound), f"{what}: mass error {err.max():.3g}"


#: Dense projections: the reference's per-kernel gate (tests/ulp_gate.py:
#: 28-103) in ulps of the fp16 output, max relative error < 4 ulps and mean
#: < 1 ulp, the denominator floored at fp16's smallest normal and, for a
#: sum, at the magnitude where fp32 accumulation's probabilistic error
#: sqrt(n) * 2^-24 * terms (Higham and Mary 2019) spends the whole budget.
FP16_REL_ULP = 2.0**-11
ULP_MAX_REL = 4 * FP16_REL_ULP
ULP_MEAN_REL = FP16_REL_ULP


def accumulation_floor(terms, n: int) -> np.ndarray:
    return np.sqrt(n) * 2.0**-24 * np.asarray(terms, np.float64) / ULP_MAX_REL


def assert_within_gate(got, want, floor=None, what=""):
    from oracle.attention import FP16_MIN_NORMAL
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != reference {want.shape}"
    f = FP16_MIN_NORMAL if floor is None else np.maximum(FP16_MIN_NORMAL, floor)
    err = np.abs(got - want) / np.maximum(np.abs(want), f)
    assert err.max() < ULP_MAX_REL, \
        f"{what}: max relative error {err.max():.3e} ({err.max() / FP16_REL_ULP:.2f} ulp)"
    assert err.mean() < ULP_MEAN_REL, \
        f"{what}: mean relative error {err.mean():.3e} ({err.mean() / FP16_REL_ULP:.2f} ulp)"
    return err


def announce(*what) -> None:
    """Names the case before a GPU step, flushed, so a failed run says where."""
    print("[case]", *what, flush=True)
