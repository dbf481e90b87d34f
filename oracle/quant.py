"""The quantised page: layout, quantiser and dequantiser, restated in NumPy.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Follows the reference:
  - layout:        src/core_kernels/quant.cu:358-392, quant.h:15-59
  - scale_of:      src/core_kernels/quant.cu:44-56 (fp64 range / levels, nearest
                   fp16, one ulp up if short of the exact value)
  - code_of:       src/core_kernels/quant.cu:60-70 (fp32 IEEE subtract and
                   divide, rintf half-even, clamp; 0 for a zero scale)
  - keys:          src/core_kernels/quant.cu:76-126 (per (head, channel) over P)
  - values:        src/core_kernels/quant.cu:141-187 (per (token, head) over hd)
  - dequantise:    src/core_kernels/quant.cu:243-266 (fmaf, then fp16 RN)
  - read_page:     src/microinfer/quantisation.py:22-46
  - bound:         src/microinfer/quantisation.py:49-62
  - FP16 page:     src/core_kernels/kv_pages.cu:62-66 (P rows of keys, then P
                   rows of values, kv_heads*head_dim fp16 each)

PINNED by (tests/test_oracle_quant.py):
  - layout: the reference's known answers (tests/test_quant.py:105-136:
    offsets in documented order, 1280 B metadata and effective bits
    8.625/4.625/2.625 at 2x128; page bytes of README.md:77-82) and the 32K
    byte totals of experiments/logs/benchmark.jsonl:48-51;
  - scale_of: the float64 reference of tests/test_quant.py:66-82 (scales and
    zeros asserted equal there, :155-158), and a brute-force search over all
    finite fp16 values for the smallest one >= the exact scale;
  - codes: on-level inputs whose codes are the inputs themselves, packed by
    hand (tests/test_quant.py:181-217); agreement with the float64 reference
    away from rounding ties (:159-163); the special cases of :241-303
    (outlier isolation, asymmetric [100, 101], subnormal scale rounded up,
    constant group with scale 0);
  - dequantise: exactness of the float64 emulation of fmaf (every term a
    multiple of 2^-24 below 2^18) checked against an fp32 FMA computed with
    math.fma on sampled elements, and the half-step round-trip bound.
"""

from __future__ import annotations

import numpy as np

FP16, INT8, INT4, INT2 = 0, 1, 2, 3
TIER_NAMES = ("FP16", "INT8", "INT4", "INT2")
#: The code width of each quantised tier (quant.h:65-91).
BITS = {INT8: 8, INT4: 4, INT2: 2}
#: The tier a page table gives a page no query reads (device_ops.h:96).
UNREAD = 0xFF


def bits_of(tier: int) -> int:
    if tier not in BITS:
        raise ValueError("FP16 is not a quantised tier: its page has no codes and no metadata")
    return BITS[tier]


def fp16_page_bytes(page_tokens: int, kv_width: int) -> int:
    """kv_pages.cu:62-66: P rows of keys then P rows of values, fp16."""
    return 2 * page_tokens * kv_width * 2


def layout(tier: int, kv_heads: int, head_dim: int, page_tokens: int = 32) -> dict:
    """quant.cu:358-392. Regions back to back: key codes, value codes, key
    scales (W fp16), key zeros (W), value scales (P*kv), value zeros (P*kv)."""
    bits = bits_of(tier)
    for n, what in ((page_tokens, "page_tokens"), (kv_heads, "kv_heads"), (head_dim, "head_dim")):
        if n <= 0:
            raise ValueError(f"{what} must be positive, got {n}")
    if head_dim * bits % 8 != 0:
        raise ValueError(f"head_dim {head_dim} at {bits} bits leaves a value group "
                         f"sharing a byte with the next")
    width = kv_heads * head_dim
    codes = page_tokens * width * bits // 8
    key_meta = width * 2
    value_meta = page_tokens * kv_heads * 2
    out = {"bits": bits, "key_codes": 0, "value_codes": codes, "key_scales": 2 * codes}
    out["key_zeros"] = out["key_scales"] + key_meta
    out["value_scales"] = out["key_zeros"] + key_meta
    out["value_zeros"] = out["value_scales"] + value_meta
    out["page_bytes"] = out["value_zeros"] + value_meta
    out["metadata_bytes"] = out["page_bytes"] - 2 * codes
    out["effective_bits"] = 8.0 * out["page_bytes"] / (2 * page_tokens * width)
    return out


def page_bytes(tier: int, kv_heads: int, head_dim: int, page_tokens: int = 32) -> int:
    if tier == FP16:
        return fp16_page_bytes(page_tokens, kv_heads * head_dim)
    return layout(tier, kv_heads, head_dim, page_tokens)["page_bytes"]


def scale_of(lo: np.ndarray, hi: np.ndarray, bits: int) -> np.ndarray:
    """quant.cu:44-56: (hi - lo) / (2^bits - 1) in fp64, rounded to the
    nearest fp16, then bumped one fp16 ulp up if that fell short."""
    levels = (1 << bits) - 1
    exact = (np.asarray(hi, np.float64) - np.asarray(lo, np.float64)) / levels
    nearest = exact.astype(np.float16)
    short = nearest.astype(np.float64) < exact
    bumped = (nearest.view(np.uint16) + np.uint16(1)).view(np.float16)
    return np.where(short, bumped, nearest).astype(np.float16)


def code_of(x: np.ndarray, zero: np.ndarray, scale: np.ndarray, bits: int) -> np.ndarray:
    """quant.cu:60-70: rintf((x - zero) / scale) in fp32, clamped to the
    levels; 0 where the scale is 0."""
    levels = np.float32((1 << bits) - 1)
    x = np.asarray(x, np.float32)
    zero = np.asarray(zero, np.float32)
    scale = np.asarray(scale, np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.rint((x - zero) / scale)
    q = np.minimum(np.maximum(q, np.float32(0)), levels)
    return np.where(scale == 0, np.float32(0), q).astype(np.uint8)


def pack(codes: np.ndarray, bits: int) -> np.ndarray:
    """8/bits consecutive codes to a byte, the first in the lowest bits
    (quant.h:37-40)."""
    per_byte = 8 // bits
    grouped = codes.astype(np.uint8).reshape(-1, per_byte)
    shifts = (np.arange(per_byte, dtype=np.uint8) * bits)
    return np.bitwise_or.reduce(grouped << shifts, axis=1).astype(np.uint8)


def unpack(raw: np.ndarray, bits: int) -> np.ndarray:
    per_byte = 8 // bits
    shifts = np.arange(per_byte, dtype=np.uint8) * bits
    return ((raw[:, None] >> shifts) & ((1 << bits) - 1)).reshape(-1).astype(np.uint8)


def quantise_page(keys: np.ndarray, values: np.ndarray, tier: int, page_tokens: int = 32,
                  filled: int | None = None) -> np.ndarray:
    """One page's keys and values, each (P, kv_heads, head_dim) fp16, to the
    tier's bytes (quant.cu:76-187, :403-417). Fewer than P positions is the
    open page, which is refused (quant.cu:342-354)."""
    keys = np.asarray(keys, np.float16)
    values = np.asarray(values, np.float16)
    if keys.ndim != 3 or values.shape != keys.shape:
        raise ValueError(f"keys and values must share a (positions, kv_heads, head_dim) shape, "
                         f"got {keys.shape} and {values.shape}")
    filled = keys.shape[0] if filled is None else filled
    lay = layout(tier, keys.shape[1], keys.shape[2], page_tokens)
    if filled < page_tokens:
        raise ValueError(f"the page holds {filled} of {page_tokens} positions and is still being "
                         f"filled: the open page stays at FP16")
    if filled > page_tokens:
        raise ValueError(f"{filled} positions do not fit a page of {page_tokens}")
    bits = lay["bits"]
    P, kv, hd = keys.shape
    k32 = keys.astype(np.float32)
    v32 = values.astype(np.float32)
    # Keys: per (head, channel) over the page's positions.
    k_lo, k_hi = k32.min(axis=0), k32.max(axis=0)                 # (kv, hd)
    k_scale = scale_of(k_lo, k_hi, bits)
    k_codes = code_of(k32, k_lo[None], k_scale.astype(np.float32)[None], bits)
    # Values: per (token, head) over head_dim.
    v_lo, v_hi = v32.min(axis=2), v32.max(axis=2)                 # (P, kv)
    v_scale = scale_of(v_lo, v_hi, bits)
    v_codes = code_of(v32, v_lo[..., None], v_scale.astype(np.float32)[..., None], bits)
    page = np.zeros(lay["page_bytes"], np.uint8)
    page[lay["key_codes"]:lay["value_codes"]] = pack(k_codes.reshape(-1), bits)
    page[lay["value_codes"]:lay["key_scales"]] = pack(v_codes.reshape(-1), bits)
    page[lay["key_scales"]:lay["key_zeros"]] = k_scale.reshape(-1).view(np.uint8)
    page[lay["key_zeros"]:lay["value_scales"]] = k_lo.astype(np.float16).reshape(-1).view(np.uint8)
    page[lay["value_scales"]:lay["value_zeros"]] = v_scale.reshape(-1).view(np.uint8)
    page[lay["value_zeros"]:lay["page_bytes"]] = v_lo.astype(np.float16).reshape(-1).view(np.uint8)
    return page


def read_page(page: np.ndarray, tier: int, kv_heads: int, head_dim: int,
              page_tokens: int = 32) -> dict:
    """quantisation.py:22-46: codes unpacked to (P, kv, hd), fp16 metadata
    widened to float64, key ones (kv, hd) and value ones (P, kv)."""
    lay = layout(tier, kv_heads, head_dim, page_tokens)
    bits = lay["bits"]
    P = page_tokens

    def codes(offset):
        n = P * kv_heads * head_dim * bits // 8
        return unpack(page[offset:offset + n], bits).reshape(P, kv_heads, head_dim)

    def halves(offset, shape):
        n = int(np.prod(shape))
        return page[offset:offset + 2 * n].view(np.float16).astype(np.float64).reshape(shape)

    return {"bits": bits,
            "key_codes": codes(lay["key_codes"]),
            "value_codes": codes(lay["value_codes"]),
            "key_scales": halves(lay["key_scales"], (kv_heads, head_dim)),
            "key_zeros": halves(lay["key_zeros"], (kv_heads, head_dim)),
            "value_scales": halves(lay["value_scales"], (P, kv_heads)),
            "value_zeros": halves(lay["value_zeros"], (P, kv_heads))}


def dequant_values(codes, scale, zero) -> np.ndarray:
    """__float2half_rn(fmaf(q, scale, zero)) (quant.cu:261-263,
    attention.cu:192-201). Every term is a multiple of 2^-24 and below 2^18
    in magnitude, so float64 holds q*scale + zero exactly; rounding that to
    fp32 is fmaf's one rounding, and then to fp16 is __float2half_rn's."""
    exact = np.asarray(codes, np.float64) * np.asarray(scale, np.float64) \
        + np.asarray(zero, np.float64)
    return exact.astype(np.float32).astype(np.float16)


def dequantise_page(page: np.ndarray, tier: int, kv_heads: int, head_dim: int,
                    page_tokens: int = 32) -> tuple[np.ndarray, np.ndarray]:
    """quant.cu:438-450: (keys, values), each (P, kv, hd) fp16."""
    lay = layout(tier, kv_heads, head_dim, page_tokens)
    page = np.asarray(page, np.uint8)
    if page.ndim != 1 or page.shape[0] != lay["page_bytes"]:
        raise ValueError(f"a page at this tier and shape is {lay['page_bytes']} bytes, "
                         f"got shape {page.shape}")
    parts = read_page(page, tier, kv_heads, head_dim, page_tokens)
    k = dequant_values(parts["key_codes"], parts["key_scales"][None], parts["key_zeros"][None])
    v = dequant_values(parts["value_codes"], parts["value_scales"][..., None],
                       parts["value_zeros"][..., None])
    return k, v


def fp16_page(keys: np.ndarray, values: np.ndarray) -> np.ndarray:
    """An FP16 page's bytes (kv_pages.cu:62-66)."""
    return np.concatenate([np.asarray(keys, np.float16).reshape(-1),
                           np.asarray(values, np.float16).reshape(-1)]).view(np.uint8)


def read_fp16_page(page: np.ndarray, page_tokens: int, kv_heads: int, head_dim: int):
    halves = np.asarray(page, np.uint8).view(np.float16).reshape(2, page_tokens, kv_heads, head_dim)
    return halves[0], halves[1]


def round_trip_bound(x: np.ndarray, got: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """quantisation.py:49-62: half a step of the stored scale, half an fp16
    ulp of the larger of input and output, and an fp32 ulp of the element."""
    larger = np.maximum(np.abs(x), np.abs(got)).astype(np.float64)
    out_ulp = np.spacing(larger.astype(np.float16)).astype(np.float64)
    return scales / 2 + out_ulp / 2 + 2.0**-23 * larger


def reference64(x: np.ndarray, bits: int, axis: int):
    """The reference test's float64 quantiser (tests/test_quant.py:66-82):
    scale, zero-point, codes and the unrounded code value."""
    top = (1 << bits) - 1
    x = np.asarray(x, np.float64)
    lo, hi = x.min(axis, keepdims=True), x.max(axis, keepdims=True)
    exact_scale = (hi - lo) / top
    nearest = exact_scale.astype(np.float16)
    scale = np.where(nearest.astype(np.float64) < exact_scale,
                     np.nextafter(nearest, np.float16(np.inf)), nearest).astype(np.float64)
    with np.errstate(divide="ignore", invalid="ignore"):
        exact = np.where(scale > 0, (x - lo) / scale, 0.0)
    codes = np.clip(np.rint(exact), 0, top)
    return scale, lo, codes, exact
