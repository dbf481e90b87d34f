"""Seeded synthetic KV of the benchmark configurations.

Data synthesis only: no arithmetic under test lives here. The shapes are the
Qwen2.5 model cards' (src/microinfer/models.py:18-50 of the reference) and
Llama-3.2-1B's; the recipes are the benchmark's: keys and values N(0, 1)
rounded to fp16, with round(2% of the W = kv_heads*head_dim key channels),
chosen without replacement, scaled x10 as outliers; tiers from seeded
lognormal importance, the lowest-ranked pages to the lowest tiers.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

FP16, INT8, INT4, INT2 = 0, 1, 2, 3


@dataclass(frozen=True)
class Shape:
    name: str
    layers: int
    heads: int
    kv_heads: int
    head_dim: int
    hidden: int
    intermediate: int
    rope_theta: float
    rms_eps: float
    vocab: int

    @property
    def kv_width(self) -> int:
        return self.kv_heads * self.head_dim

    @property
    def group(self) -> int:
        return self.heads // self.kv_heads


QWEN_05B = Shape("qwen2.5-0.5b", 24, 14, 2, 64, 896, 4864, 1e6, 1e-6, 151936)
QWEN_15B = Shape("qwen2.5-1.5b", 28, 12, 2, 128, 1536, 8960, 1e6, 1e-6, 151936)
LLAMA_1B = Shape("llama-3.2-1b", 16, 32, 8, 64, 2048, 8192, 5e5, 1e-5, 128256)
SHAPES = {s.name: s for s in (QWEN_05B, QWEN_15B, LLAMA_1B)}

#: Config 3's tier mix, lowest tier first: (tier, fraction of sealed pages).
MIX_CONFIG3 = ((INT2, 0.10), (INT4, 0.40), (INT8, 0.30), (FP16, 0.20))
#: Config 5's decode mix.
MIX_CONFIG5 = ((INT4, 0.30), (INT8, 0.40), (FP16, 0.30))


def outlier_channels(rng: np.random.Generator, width: int, fraction: float = 0.02) -> np.ndarray:
    return rng.choice(width, int(round(fraction * width)), replace=False)


def kv_rows(rng: np.random.Generator, positions: int, shape: Shape,
            outliers: np.ndarray | None = None, scale: float = 10.0):
    """Keys and values (positions, kv_heads, head_dim) fp16, keys with the
    outlier channels scaled."""
    k = rng.standard_normal((positions, shape.kv_width), dtype=np.float32)
    if outliers is not None and len(outliers):
        k[:, outliers] *= np.float32(scale)
    v = rng.standard_normal((positions, shape.kv_width), dtype=np.float32)
    k16 = k.astype(np.float16).reshape(positions, shape.kv_heads, shape.head_dim)
    v16 = v.astype(np.float16).reshape(positions, shape.kv_heads, shape.head_dim)
    return k16, v16


def mix_counts(pages: int, mix) -> list[tuple[int, int]]:
    """Page counts per tier: each fraction rounded, the last tier taking the
    remainder, so the counts sum to `pages`."""
    counts = [int(round(f * pages)) for _, f in mix[:-1]]
    counts.append(pages - sum(counts))
    return [(t, c) for (t, _), c in zip(mix, counts)]


def tiers_by_importance(rng: np.random.Generator, pages: int, mix) -> np.ndarray:
    """Lognormal importance per page, ranked ascending; the lowest-ranked
    pages take the first tier of `mix`, and so on."""
    scores = rng.lognormal(0.0, 1.0, pages)
    order = np.argsort(scores, kind="stable")
    tiers = np.empty(pages, np.int8)
    at = 0
    for tier, count in mix_counts(pages, mix):
        tiers[order[at:at + count]] = tier
        at += count
    return tiers


def model_dict(shape: Shape) -> dict:
    """A shape as DecodeStep takes it."""
    return dict(layers=shape.layers, hidden=shape.hidden, intermediate=shape.intermediate,
                heads=shape.heads, kv_heads=shape.kv_heads, head_dim=shape.head_dim,
                vocab=shape.vocab, rms_eps=shape.rms_eps, rope_theta=shape.rope_theta)


def weight_bytes_per_step(shape: Shape) -> int:
    """fp16 weight bytes a decode step reads: every layer's projections and
    norms, the final norm and the head (the embedding gives one row)."""
    h, i = shape.hidden, shape.intermediate
    q, kv = shape.heads * shape.head_dim, shape.kv_heads * shape.head_dim
    layer = h * (q + 2 * kv) + (q + 2 * kv) + q * h + 3 * h * i + 2 * h
    return 2 * (shape.layers * layer + h + shape.vocab * h + h)


def tier_map(seed: int, layers: int, pages: int, mix) -> list[list[int]]:
    """A tier map, one row of `pages` tiers per layer, from one seeded
    stream."""
    rng = np.random.default_rng(seed)
    return [tiers_by_importance(rng, pages, mix).tolist() for _ in range(layers)]
