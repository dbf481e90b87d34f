"""The C ABI library loads here, on the CPU, and exports every entry point
include/microinfer_hip.h declares; its host-side rounding helpers agree with
NumPy and the oracle. No device call is made."""

import re

import numpy as np

from conftest import REPO
from oracle import quant

HEADER = REPO / "include" / "microinfer_hip.h"


def declared() -> set:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(mi_[a-z0-9_]+)\s*\(", text))


def test_every_declared_symbol_is_exported():
    from microinfer import _microinfer
    names = declared()
    assert len(names) > 80
    missing = [n for n in sorted(names) if not hasattr(_microinfer.lib, n)]
    assert not missing, missing
    # And the shim binds a signature for each of them.
    unbound = sorted(names - set(_microinfer.SIGNATURES))
    assert not unbound, unbound


def test_half_rounding_from_double_is_numpy_s():
    from microinfer import _microinfer
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(20000) * np.exp(rng.uniform(-25, 12, 20000)),
        [0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e10, 2.0**-24, 2.0**-25, 2.0**-25 * 1.0001,
         2.0**-14, 2.0**-14 * (1 - 2.0**-12), 5.96e-8, np.inf, -np.inf]])
    # Values exactly halfway between neighbouring fp16s, both parities.
    h = np.arange(1, 0x7BFF, 97, dtype=np.uint16).view(np.float16).astype(np.float64)
    mids = (h + np.nextafter(h.astype(np.float16), np.float16(np.inf)).astype(np.float64)) / 2
    x = np.concatenate([x, mids, -mids])
    got = np.array([_microinfer.lib.mi_half_bits_from_double(float(v)) for v in x], np.uint16)
    with np.errstate(over="ignore"):  # values past fp16's range round to inf
        want = x.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(got, want)


def test_scale_bits_are_the_oracle_s():
    from microinfer import _microinfer
    rng = np.random.default_rng(1)
    lo = rng.normal(0, 5, 3000).astype(np.float16)
    hi = (lo.astype(np.float32) + np.abs(rng.normal(0, 1, 3000)).astype(np.float32)
          * rng.choice([1e-5, 1e-2, 1.0, 40.0], 3000).astype(np.float32)).astype(np.float16)
    for bits in (8, 4, 2):
        want = quant.scale_of(lo, hi, bits).view(np.uint16)
        got = np.array([_microinfer.lib.mi_scale_bits_of(float(a), float(b), bits)
                        for a, b in zip(lo, hi)], np.uint16)
        np.testing.assert_array_equal(got, want)


def test_layout_through_the_abi_is_the_oracle_s():
    from microinfer import _microinfer
    for kv, hd in ((2, 64), (2, 128), (8, 64), (1, 8)):
        for tier in (1, 2, 3):
            got = _microinfer.quantised_page_layout(tier, kv, hd)
            want = quant.layout(tier, kv, hd)
            assert {k: got[k] for k in want} == want


def test_errors_map_to_the_reference_exception_classes():
    import pytest
    from microinfer import _microinfer
    with pytest.raises(ValueError, match="FP16"):
        _microinfer.quantised_page_layout(_microinfer.Tier.FP16, 2, 64)
    with pytest.raises(ValueError, match="sharing a byte"):
        _microinfer.quantised_page_layout(_microinfer.Tier.INT2, 1, 2)
    assert issubclass(_microinfer.OpenPage, ValueError)
    assert issubclass(_microinfer.PageNotFound, KeyError)
    assert issubclass(_microinfer.OutOfMemory, MemoryError)
