"""The requantisation kernels against the oracle, to the bit.

GPU parity tests: every code, scale and zero-point of quantise_page, and
every fp16 of dequantise_page, must equal the NumPy restatement of the
reference's arithmetic (oracle/quant.py) exactly."""

import ctypes as C

import numpy as np
import pytest

from conftest import GOLDEN, announce, each, fp16_exact
from oracle import quant

pytestmark = pytest.mark.gpu

QUANTISED = (1, 2, 3)
SHAPES = ((2, 64, 32), (2, 128, 32), (8, 64, 32), (2, 64, 16), (2, 128, 48), (1, 8, 16))


def mi():
    from microinfer import _microinfer
    return _microinfer


def random_page(P, heads, hd, seed):
    rng = np.random.default_rng(seed)
    keys = rng.normal(0, 1, (P, heads, hd))
    keys[:, :, rng.choice(hd, min(3, hd), replace=False)] *= 40
    keys += rng.normal(0, 4, (1, heads, hd))
    values = rng.normal(0, 1, (P, heads, hd))
    values[rng.choice(P, 2, replace=False)] *= 25
    return fp16_exact(keys), fp16_exact(values)


def test_quantise_page_is_the_oracle_to_the_bit():
    m = mi()

    def check(kv, hd, P, tier, seed):
        announce("quantise_page", kv, hd, P, tier, seed)
        keys, values = random_page(P, kv, hd, seed)
        got = m.quantise_page(keys, values, tier, P)
        want = quant.quantise_page(keys.astype(np.float16), values.astype(np.float16), tier, P)
        np.testing.assert_array_equal(got, want)

    each([(kv, hd, P, t, s) for kv, hd, P in SHAPES for t in QUANTISED for s in range(3)], check)


def test_dequantise_page_is_the_oracle_to_the_bit():
    m = mi()

    def check(kv, hd, P, tier):
        announce("dequantise_page", kv, hd, P, tier)
        keys, values = random_page(P, kv, hd, 11)
        page = quant.quantise_page(keys.astype(np.float16), values.astype(np.float16), tier, P)
        gk, gv = m.dequantise_page(page, tier, kv, hd, P)
        wk, wv = quant.dequantise_page(page, tier, kv, hd, P)
        np.testing.assert_array_equal(gk, wk.astype(np.float32))
        np.testing.assert_array_equal(gv, wv.astype(np.float32))

    each([(kv, hd, P, t) for kv, hd, P in SHAPES for t in QUANTISED], check)


def test_known_answers_and_special_cases_on_the_device():
    """The on-level fixture packed by hand, and the reference's special cases
    (constant group, subnormal scale, huge outlier) through the kernel."""
    m = mi()
    data = np.load(GOLDEN / "quant_on_level.npz")
    for tier, name in ((1, "INT8"), (2, "INT4"), (3, "INT2")):
        announce("on-level", name)
        keys, values = data[f"{name}_keys"], data[f"{name}_values"]
        lay = quant.layout(tier, 2, 128)
        page = m.quantise_page(keys, values, tier)
        np.testing.assert_array_equal(page[lay["key_codes"]:lay["value_codes"]],
                                      data[f"{name}_key_codes"])
        np.testing.assert_array_equal(page[lay["value_codes"]:lay["key_scales"]],
                                      data[f"{name}_value_codes"])
        k, v = m.dequantise_page(page, tier, 2, 128)
        np.testing.assert_array_equal(k, keys)
        np.testing.assert_array_equal(v, values)
        special_k, special_v = random_page(32, 2, 128, 5)
        special_k[:, 1, 58] = fp16_exact(np.linspace(0.00554656982421875, 0.005672454833984375, 32))
        special_k[:, 0, 5] = -2.5
        special_v[3, 1] = 0.75
        special_k[5, 1, 7] = 3000.0
        special_v[9, 0, 3] = -3000.0
        got = m.quantise_page(special_k, special_v, tier)
        want = quant.quantise_page(special_k.astype(np.float16), special_v.astype(np.float16), tier)
        np.testing.assert_array_equal(got, want)


def test_a_batch_is_each_page_quantised_alone():
    """mi_quantise_pages over device address tables equals the one-page
    entry point, page for page."""
    m = mi()
    kv, hd, P, n = 2, 128, 32, 37
    fp16 = quant.fp16_page_bytes(P, kv * hd)
    rows = []
    for i in range(n):
        k, v = random_page(P, kv, hd, 100 + i)
        rows.append(quant.fp16_page(k.astype(np.float16), v.astype(np.float16)))
    for tier in QUANTISED:
        announce("quantise_pages batch", tier)
        lay = quant.layout(tier, kv, hd, P)
        src = m._Storage(n * fp16)
        dst = m._Storage(n * lay["page_bytes"])
        m._h2d(src.ptr, np.concatenate(rows))
        table = np.array([src.ptr + i * fp16 for i in range(n)] +
                         [dst.ptr + i * lay["page_bytes"] for i in range(n)], np.uint64)
        tab = m._Storage(table.nbytes)
        m._h2d(tab.ptr, table)
        m._check(m.lib.mi_quantise_pages(tab.ptr, tab.ptr + 8 * n, n, tier, P, kv, hd, None))
        out = np.empty(n * lay["page_bytes"], np.uint8)
        m._d2h(out, dst.ptr)
        for i in range(n):
            k, v = quant.read_fp16_page(rows[i], P, kv, hd)
            np.testing.assert_array_equal(out[i * lay["page_bytes"]:(i + 1) * lay["page_bytes"]],
                                          quant.quantise_page(k, v, tier, P))


def test_what_is_not_a_full_page_is_refused():
    m = mi()
    keys, values = random_page(32, 2, 64, 0)
    for tier in QUANTISED:
        for filled in (1, 31):
            with pytest.raises(m.OpenPage, match=f"{filled} of 32 positions.*FP16"):
                m.quantise_page(keys[:filled], values[:filled], tier)
        with pytest.raises(ValueError, match="positions"):
            m.quantise_page(np.concatenate([keys, keys]), np.concatenate([values, values]), tier)
        with pytest.raises(ValueError, match="shape"):
            m.quantise_page(keys, values[:, :1], tier)
        page = m.quantise_page(keys, values, tier)
        with pytest.raises(ValueError, match="bytes"):
            m.dequantise_page(page[:-1], tier, 2, 64)
    with pytest.raises(ValueError, match="FP16"):
        m.quantise_page(keys, values, m.Tier.FP16)


def tie_page(kv, hd, bits, seed):
    """Keys and values whose every group holds its minimum, its maximum and
    elements exactly on (and one fp16 ulp beside) the half-levels of a scale
    with an odd mantissa: quotients that are exact ties, where a code formed
    through 1 / scale could round the other way."""
    rng = np.random.default_rng(seed)
    levels = (1 << bits) - 1

    def group(n):
        s = np.float16(int(rng.choice(np.arange(3, 32, 2))) * 2.0 ** int(rng.integers(-14, 0)))
        lo = np.float16(int(rng.integers(-8, 8)) * np.float64(s))
        hi = np.float16(lo.astype(np.float64) + levels * np.float64(s))
        k = rng.integers(0, levels, n - 2).astype(np.float64)
        mid = (lo.astype(np.float64) + (k + 0.5) * np.float64(s)).astype(np.float16)
        step = rng.integers(-1, 2, n - 2).astype(np.int32)
        near = (mid.view(np.uint16).astype(np.int32) + np.where(mid >= 0, step, -step))
        near = near.astype(np.uint16).view(np.float16)
        out = np.concatenate([[lo, hi], near]).astype(np.float64)
        return np.clip(out, float(lo), float(hi))

    keys = np.stack([group(32) for _ in range(kv * hd)], axis=1).reshape(32, kv, hd)
    values = np.stack([group(hd) for _ in range(32 * kv)]).reshape(32, kv, hd)
    return fp16_exact(keys), fp16_exact(values)


def test_ties_quantise_as_the_oracle_to_the_bit():
    """Pages built from exact and near ties at every tier, through the
    quantiser the batch and single-page entry points take at the cache's
    shapes (32-token pages, head_dim 64 and 128)."""
    m = mi()

    def check(kv, hd, tier, seed):
        announce("quantise ties", kv, hd, tier, seed)
        keys, values = tie_page(kv, hd, 8 >> (tier - 1), seed)
        got = m.quantise_page(keys, values, tier, 32)
        want = quant.quantise_page(keys.astype(np.float16), values.astype(np.float16), tier, 32)
        np.testing.assert_array_equal(got, want)

    each([(kv, hd, t, s) for kv, hd in ((2, 128), (2, 64), (8, 64)) for t in QUANTISED
          for s in range(4)], check)
