"""A quantised page read on the host, and what its round trip may lose.

The host-side reader of the reference's src/microinfer/quantisation.py:22-62,
reading a page through the offsets the library reports, so it cannot drift
from the kernels. Measurement, not inference: NumPy on the host.
"""

from __future__ import annotations

import numpy as np

from . import _microinfer

P = _microinfer.device.page_tokens


def read_page(page: np.ndarray, tier, heads: int, head_dim: int, page_tokens: int = P) -> dict:
    """A quantised page's regions: the code width, the codes unpacked to
    (P, heads, head_dim), and the fp16 scales and zero-points in float64,
    key ones (heads, head_dim) and value ones (P, heads)."""
    layout = _microinfer.quantised_page_layout(tier, heads, head_dim, page_tokens)
    bits = layout["bits"]
    per_byte = 8 // bits

    def codes(offset):
        raw = page[offset:offset + page_tokens * heads * head_dim // per_byte]
        shifts = np.arange(per_byte, dtype=np.uint8) * bits
        unpacked = (raw[:, None] >> shifts) & ((1 << bits) - 1)
        return unpacked.reshape(page_tokens, heads, head_dim).astype(np.int64)

    def halves(offset, shape):
        n = int(np.prod(shape))
        return page[offset:offset + 2 * n].view(np.float16).astype(np.float64).reshape(shape)

    return {"bits": bits,
            "key_codes": codes(layout["key_codes"]),
            "value_codes": codes(layout["value_codes"]),
            "key_scales": halves(layout["key_scales"], (heads, head_dim)),
            "key_zeros": halves(layout["key_zeros"], (heads, head_dim)),
            "value_scales": halves(layout["value_scales"], (page_tokens, heads)),
            "value_zeros": halves(layout["value_zeros"], (page_tokens, heads))}


def round_trip_bound(x: np.ndarray, got: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """Half a step of the stored scale, half an fp16 ulp of the larger of
    input and output, and an fp32 ulp of the element."""
    larger = np.maximum(np.abs(x), np.abs(got)).astype(np.float64)
    out_ulp = np.spacing(larger.astype(np.float16)).astype(np.float64)
    return scales / 2 + out_ulp / 2 + 2.0**-23 * larger
