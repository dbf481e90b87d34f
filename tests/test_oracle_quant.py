"""The oracle's quantiser and layout, pinned against the reference's known
answers, a brute-force search, and what the arithmetic fixes.

CPU only. These pin oracle/quant.py before anything is compared to it.
"""

import json
from fractions import Fraction

import numpy as np
import pytest

from conftest import GOLDEN, each, fp16_exact
from oracle import quant, slots

KNOWN = json.loads((GOLDEN / "known_answers.json").read_text())
QUANTISED = (quant.INT8, quant.INT4, quant.INT2)
NAMES = {quant.FP16: "FP16", quant.INT8: "INT8", quant.INT4: "INT4", quant.INT2: "INT2"}


def random_page(heads, head_dim, seed=0):
    """tests/test_quant.py:45-54: keys with outlier channels and a per-channel
    offset, values with outlier tokens; fp16-exact."""
    rng = np.random.default_rng(seed)
    keys = rng.normal(0, 1, (32, heads, head_dim))
    keys[:, :, rng.choice(head_dim, 3, replace=False)] *= 40
    keys += rng.normal(0, 4, (1, heads, head_dim))
    values = rng.normal(0, 1, (32, heads, head_dim))
    values[rng.choice(32, 2, replace=False)] *= 25
    return fp16_exact(keys).astype(np.float16), fp16_exact(values).astype(np.float16)


def test_layout_is_the_reference_known_answer():
    k = KNOWN["layout_1_5b"]
    for tier in QUANTISED:
        lay = quant.layout(tier, k["kv_heads"], k["head_dim"], k["page_tokens"])
        name = NAMES[tier]
        assert lay["metadata_bytes"] == k["metadata_bytes"]
        assert lay["effective_bits"] == k["effective_bits"][name]
        assert lay["page_bytes"] == k["page_bytes"][name]
        assert lay["value_codes"] - lay["key_codes"] == k["data_bytes"][name] // 2
        # Regions back to back in the documented order.
        width = k["kv_heads"] * k["head_dim"]
        sizes = [lay["value_codes"], lay["value_codes"], 2 * width, 2 * width,
                 2 * 32 * k["kv_heads"], 2 * 32 * k["kv_heads"]]
        starts = [lay[r] for r in ("key_codes", "value_codes", "key_scales", "key_zeros",
                                   "value_scales", "value_zeros")]
        assert starts == list(np.cumsum([0] + sizes[:-1]))
        assert starts[-1] + sizes[-1] == lay["page_bytes"]
    assert quant.page_bytes(quant.FP16, 2, 128) == k["page_bytes"]["FP16"]
    with pytest.raises(ValueError, match="FP16"):
        quant.layout(quant.FP16, 2, 64)
    with pytest.raises(ValueError, match="sharing a byte"):
        quant.layout(quant.INT2, 1, 2)


def test_footprint_at_32k_is_the_reference_measurement():
    """benchmark.jsonl:48-51: 28 layers at 32K, whole 2 MiB granules per
    tier range, two FP16 open pages a layer once a cache seals."""
    f = KNOWN["footprint_32k_1_5b"]
    page_bytes = [quant.page_bytes(t, 2, 128) for t in range(4)]
    for tier in range(4):
        seals = tier != quant.FP16
        ranges = slots.cache_ranges(f["layers"], f["context"], 32, page_bytes, tier=tier,
                                    seals=seals)
        name = NAMES[tier]
        assert sum(ranges) == f["payload_bytes"][name]
        assert slots.cache_bytes(ranges, f["granule"]) == f["bytes"][name]


def all_finite_fp16() -> np.ndarray:
    h = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16)
    return h.astype(np.float64)


def test_scale_of_is_the_least_fp16_reaching_the_range():
    """Brute force over every finite non-negative fp16: the stored scale is
    the nearest fp16 to range / levels, or the next one up if that is short;
    either way the least fp16 at or above it whenever the nearest is below."""
    grid = all_finite_fp16()
    rng = np.random.default_rng(1)
    lo = fp16_exact(rng.normal(0, 10, 4000) * rng.choice([1e-4, 1e-2, 1, 30], 4000))
    hi = lo + fp16_exact(np.abs(rng.normal(0, 1, 4000)) * rng.choice([1e-5, 1e-3, 1, 50], 4000))
    hi = fp16_exact(hi)
    for tier in QUANTISED:
        bits = quant.BITS[tier]
        exact = (hi.astype(np.float64) - lo.astype(np.float64)) / ((1 << bits) - 1)
        got = quant.scale_of(lo, hi, bits).astype(np.float64)
        at_or_above = grid[np.searchsorted(grid, exact, side="left")]
        nearest = exact.astype(np.float16).astype(np.float64)
        want = np.where(nearest >= exact, nearest, at_or_above)
        np.testing.assert_array_equal(got, want)
        assert np.all(got >= exact)


def test_codes_and_metadata_are_the_float64_reference_away_from_ties():
    """tests/test_quant.py:142-163: scales and zeros equal the float64
    reference; codes equal it but within a hair of a rounding tie."""
    def check(heads, hd, tier):
        keys, values = random_page(heads, hd)
        parts = quant.read_page(quant.quantise_page(keys, values, tier), tier, heads, hd)
        bits = parts["bits"]
        k_scale, k_zero, k_codes, k_exact = quant.reference64(keys, bits, axis=0)
        v_scale, v_zero, v_codes, v_exact = quant.reference64(values, bits, axis=2)
        np.testing.assert_array_equal(parts["key_scales"], k_scale[0])
        np.testing.assert_array_equal(parts["key_zeros"], k_zero[0])
        np.testing.assert_array_equal(parts["value_scales"], v_scale[..., 0])
        np.testing.assert_array_equal(parts["value_zeros"], v_zero[..., 0])
        for got, want, exact in ((parts["key_codes"], k_codes, k_exact),
                                 (parts["value_codes"], v_codes, v_exact)):
            differ = got != want
            near_tie = np.abs(exact - np.floor(exact) - 0.5) < 1e-3
            assert not np.any(differ & ~near_tie)
            assert np.all(np.abs(got.astype(np.int64) - want) <= 1)

    each([(h, d, t) for h, d in ((2, 64), (2, 128), (8, 64)) for t in QUANTISED], check)


def test_on_level_codes_are_packed_by_hand():
    """tests/test_quant.py:181-217, fixture tests/golden/quant_on_level.npz."""
    data = np.load(GOLDEN / "quant_on_level.npz")
    for tier in QUANTISED:
        name = NAMES[tier]
        keys, values = data[f"{name}_keys"], data[f"{name}_values"]
        lay = quant.layout(tier, 2, 128)
        page = quant.quantise_page(keys, values, tier)
        np.testing.assert_array_equal(page[lay["key_codes"]:lay["value_codes"]],
                                      data[f"{name}_key_codes"])
        np.testing.assert_array_equal(page[lay["value_codes"]:lay["key_scales"]],
                                      data[f"{name}_value_codes"])
        k, v = quant.dequantise_page(page, tier, 2, 128)
        np.testing.assert_array_equal(k.astype(np.float32), keys)
        np.testing.assert_array_equal(v.astype(np.float32), values)


def test_special_cases_of_the_reference():
    """tests/test_quant.py:241-303: outlier isolation, asymmetric range,
    subnormal scale rounded up, constant group."""
    def per_channel(tier):
        keys, values = random_page(2, 64, seed=2)
        base_k, base_v = quant.dequantise_page(quant.quantise_page(keys, values, tier), tier, 2, 64)
        k2, v2 = keys.copy(), values.copy()
        k2[5, 1, 7] = 3000.0
        v2[9, 0, 3] = -3000.0
        got_k, got_v = quant.dequantise_page(quant.quantise_page(k2, v2, tier), tier, 2, 64)
        other = np.ones((2, 64), bool)
        other[1, 7] = False
        np.testing.assert_array_equal(got_k[:, other], base_k[:, other])
        groups = np.ones((32, 2), bool)
        groups[9, 0] = False
        np.testing.assert_array_equal(got_v[groups], base_v[groups])
        assert not np.array_equal(got_k[:, 1, 7], base_k[:, 1, 7])

    def asymmetric(tier):
        keys, values = random_page(2, 64, seed=3)
        keys[:, 0, 0] = np.linspace(100, 101, 32).astype(np.float16)
        values[4, 1] = np.linspace(-51, -50, 64).astype(np.float16)
        page = quant.quantise_page(keys, values, tier)
        parts = quant.read_page(page, tier, 2, 64)
        assert parts["key_zeros"][0, 0] == 100 and parts["value_zeros"][4, 1] == -51
        k, v = quant.dequantise_page(page, tier, 2, 64)
        steps = (1 << quant.BITS[tier]) - 1
        assert np.abs(k[:, 0, 0].astype(np.float64) - keys[:, 0, 0]).max() <= 1 / steps
        assert np.abs(v[4, 1].astype(np.float64) - values[4, 1]).max() <= 1 / steps

    def narrow(tier):
        keys, values = random_page(2, 128, seed=5)
        channel = np.linspace(0.00554656982421875, 0.005672454833984375, 32).astype(np.float16)
        keys[:, 1, 58] = channel
        page = quant.quantise_page(keys, values, tier)
        scale = quant.read_page(page, tier, 2, 128)["key_scales"][1, 58]
        steps = (1 << quant.BITS[tier]) - 1
        c64 = channel.astype(np.float64)
        assert scale < 2.0**-14 and steps * scale >= c64.max() - c64.min()
        k, _ = quant.dequantise_page(page, tier, 2, 128)
        err = np.abs(k[:, 1, 58].astype(np.float64) - c64)
        assert err.max() <= scale / 2 + np.spacing(np.float16(0.0057)) / 2

    def constant(tier):
        keys, values = random_page(2, 64, seed=4)
        keys[:, 0, 5] = -2.5
        values[3, 1] = 0.75
        page = quant.quantise_page(keys, values, tier)
        parts = quant.read_page(page, tier, 2, 64)
        k, v = quant.dequantise_page(page, tier, 2, 64)
        assert parts["key_scales"][0, 5] == 0 and np.all(k[:, 0, 5] == keys[:, 0, 5])
        assert parts["value_scales"][3, 1] == 0 and np.all(v[3, 1] == values[3, 1])

    each([(c, t) for c in (per_channel, asymmetric, narrow, constant) for t in QUANTISED],
         lambda c, t: c(t), name=lambda c: f"{c[0].__name__} {NAMES[c[1]]}")


def test_dequantise_emulates_one_fma_exactly():
    """Every q*s + z the dequantiser meets is exact in float64, so rounding
    it to fp32 is fmaf's single rounding: checked with exact rationals."""
    for tier in QUANTISED:
        keys, values = random_page(2, 128, seed=7)
        parts = quant.read_page(quant.quantise_page(keys, values, tier), tier, 2, 128)
        q = parts["key_codes"].astype(np.float64)
        s = np.broadcast_to(parts["key_scales"][None], q.shape)
        z = np.broadcast_to(parts["key_zeros"][None], q.shape)
        idx = np.random.default_rng(0).choice(q.size, 500, replace=False)
        for i in idx:
            qi, si, zi = q.flat[i], s.flat[i], z.flat[i]
            assert Fraction(qi * si + zi) == Fraction(qi) * Fraction(si) + Fraction(zi)


def test_round_trip_within_half_a_step_and_worse_as_tiers_narrow():
    """tests/test_quant.py:223-238."""
    pages = [random_page(2, 128, seed) for seed in range(4)]
    relative = []
    for tier in QUANTISED:
        errs = []
        for keys, values in pages:
            page = quant.quantise_page(keys, values, tier)
            parts = quant.read_page(page, tier, 2, 128)
            k, v = quant.dequantise_page(page, tier, 2, 128)
            kb = quant.round_trip_bound(keys, k, parts["key_scales"][None])
            vb = quant.round_trip_bound(values, v, parts["value_scales"][..., None])
            ke = np.abs(k.astype(np.float64) - keys)
            ve = np.abs(v.astype(np.float64) - values)
            assert np.all(ke <= kb) and np.all(ve <= vb)
            errs.append((ke, ve))
        relative.append([np.linalg.norm(np.concatenate([e[i].ravel() for e in errs])) /
                         np.linalg.norm(np.concatenate([p[i].astype(np.float64).ravel()
                                                        for p in pages])) for i in (0, 1)])
    assert np.all(np.diff(np.array(relative), axis=0) > 0)


def test_open_and_malformed_pages_are_refused():
    keys, values = random_page(2, 64)
    for tier in QUANTISED:
        for filled in (1, 31):
            with pytest.raises(ValueError, match=f"{filled} of 32 positions"):
                quant.quantise_page(keys[:filled], values[:filled], tier)
        with pytest.raises(ValueError, match="positions"):
            quant.quantise_page(np.concatenate([keys, keys]), np.concatenate([values, values]),
                                tier)
        page = quant.quantise_page(keys, values, tier)
        with pytest.raises(ValueError, match="bytes"):
            quant.dequantise_page(page[:-1], tier, 2, 64)


def fast_code_model(x, zero, scale, bits):
    """The device's code with the quotient taken as (x - zero) * (1 / scale)
    and the IEEE quotient only inside a 2^-13 band around a half-integer
    (quant_core.hpp code_of_fast), restated in NumPy float32."""
    levels = np.float32((1 << bits) - 1)
    x = np.asarray(x, np.float32)
    zero = np.asarray(zero, np.float32)
    scale = np.asarray(scale, np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        inv = np.where(scale != 0, np.float32(1) / scale, np.float32(0)).astype(np.float32)
        d = (x - zero).astype(np.float32)
        q = (d * inv).astype(np.float32)
        band = (np.abs((q - np.floor(q)) - np.float32(0.5)) < np.float32(2.0 ** -13)) & (scale != 0)
        q = np.where(band, d / scale, q).astype(np.float32)
    q = np.minimum(np.maximum(np.rint(q), np.float32(0)), levels)
    return q.astype(np.uint8)


def test_the_fast_code_path_is_the_division_to_the_bit():
    """Codes through (x - zero) * (1 / scale), with the IEEE quotient only
    near a half-integer, equal code_of's rintf((x - zero) / scale) for every
    element of every group the quantiser forms: random groups at every tier,
    groups whose elements sit exactly on and one fp16 ulp either side of
    every half-level (ties), and groups with subnormal and zero scales."""
    rng = np.random.default_rng(7)
    for bits in (8, 4, 2):
        levels = (1 << bits) - 1
        cases = []
        for _ in range(400):
            g = fp16_exact(rng.normal(rng.normal(0, 4), np.exp(rng.uniform(-12, 6)), 64))
            cases.append(g.astype(np.float16))
        # Scales with odd mantissas (1 / s inexact) and a zero point on the
        # scale's grid, so that every half-level zero + (k + 1/2) s is an
        # fp16 value: exact ties of the IEEE quotient.
        for mant, exp in [(m, e) for m in range(3, 32, 2) for e in range(-20, 4, 3)]:
            s = np.float16(mant * 2.0 ** exp)
            lo = np.float16(int(rng.integers(-8, 8)) * np.float64(s))
            k = np.arange(levels, dtype=np.float64)
            mid = (lo.astype(np.float64) + (k + 0.5) * np.float64(s)).astype(np.float16)
            up = (mid.view(np.uint16) + 1).view(np.float16)
            down = (mid.view(np.uint16) - 1).view(np.float16)
            hi = np.float16(lo.astype(np.float64) + levels * np.float64(s))
            g = np.concatenate([[lo, hi], mid, up, down]).astype(np.float16)
            g = g[np.isfinite(g)]
            cases.append(np.clip(g, min(lo, hi), max(lo, hi)).astype(np.float16))
        cases.append(np.full(64, np.float16(1.5)))
        cases.append(np.array([0, 2.0 ** -24, 2.0 ** -23, 3 * 2.0 ** -24], np.float16))
        for g in cases:
            lo, hi = g.min(), g.max()
            s = quant.scale_of(lo, hi, bits)
            want = quant.code_of(g, lo, s, bits)
            got = fast_code_model(g, lo, s, bits)
            np.testing.assert_array_equal(got, want, err_msg=f"bits {bits} scale {s}")


def fast_scale_model(lo, hi, bits):
    """The device's scale without a double division (quant_core.hpp
    scale_bits_fast), restated: the fp32 estimate rounded to fp16, then that
    or the next fp16 up, whichever is the least s with s * levels >= hi - lo
    (products and the range exact in float64)."""
    levels = float((1 << bits) - 1)
    rng_ = float(np.float64(hi) - np.float64(lo))
    if rng_ == 0.0:
        return np.float16(0)
    est = np.float32(np.float32(rng_) * (np.float32(1.0) / np.float32(levels)))
    c = np.float16(est).view(np.uint16)
    if float(c.view(np.float16)) * levels < rng_:
        return (c + np.uint16(1)).view(np.float16)
    below = (c - np.uint16(1)).view(np.float16)
    if c > 0 and float(below) * levels >= rng_:
        return below
    return c.view(np.float16)


def test_the_fast_scale_is_scale_of_to_the_bit():
    """scale_bits_fast equals scale_of (the reference's fp64 nearest-then-up)
    over random groups at every tier, ranges that are exact multiples of an
    fp16 value times the levels (the nearest is exact), ranges one 2^-24
    either side of those, subnormal ranges and binade edges."""
    rng = np.random.default_rng(11)
    for bits in (8, 4, 2):
        levels = (1 << bits) - 1
        pairs = []
        for _ in range(3000):
            lo = np.float16(rng.normal(0, 8))
            hi = np.float16(lo + abs(rng.normal(0, 1)) * np.exp(rng.uniform(-14, 3)))
            pairs.append((lo, hi))
        for raw in list(range(1, 64)) + list(range(0x3000, 0x3040)) + list(range(0x7000, 0x7010)):
            s = np.uint16(raw).view(np.float16)
            for lo in (np.float16(0), np.float16(-1.5), np.float16(2.0 ** -14)):
                for nudge in (-2.0 ** -24, 0.0, 2.0 ** -24):
                    with np.errstate(over="ignore"):  # a top past fp16's range is skipped
                        hi = np.float16(float(lo) + levels * float(s) + nudge)
                    if np.isfinite(hi) and hi >= lo:
                        pairs.append((lo, hi))
        for lo, hi in pairs:
            want = quant.scale_of(lo, hi, bits)
            got = fast_scale_model(lo, hi, bits)
            assert got.view(np.uint16) == want.view(np.uint16), (bits, lo, hi, got, want)
