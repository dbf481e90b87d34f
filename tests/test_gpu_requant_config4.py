"""Configuration 4 at its full size: the requantisation plan on the
28-layer Qwen2.5-1.5B cache at 32K positions (28 x 1,024 sealed FP16 pages).

One move_pages batch takes 50% of the pages FP16 -> INT4 and 25% FP16 -> INT2
as first downgrades (shadows pinned ahead, spare granules mapped ahead, the
given-up FP16 granules released by the cache's thread); a second batch
restores 10% of the INT4 pages to INT8 from their retained shadows. The plan
is bench.py's (seeded permutation, seed 0), the one the reference's batched
moves are measured on (experiments/logs/benchmark.jsonl:3320).

GPU parity test, at the size where the move path's size-dependent branches
run (a 21,504-move requantise launch, a shadow address table past a thousand
entries, a staging buffer of tens of MB, page references across all of a
range's slots):
  - every page's tier is the plan's (tests/test_batched_moves.py:98-126);
  - every page's bytes, all 28,672 of them, are the oracle's: quantise_page
    of its rows at its tier, or its FP16 rows where it did not move;
  - every moved page holds a shadow equal to its FP16 rows, and no other
    page holds one;
  - each tier's mapped bytes are whole granules over its packed slots
    (paged_kv_cache.cu:437-470), once the spares are dropped and the
    releases drained, and each tier's slots are packed from 0;
  - one layer's decode over the moved cache meets the oracle's 1e-3 bar.
"""

import numpy as np
import pytest

from conftest import announce, assert_attention_close, assert_mass_close, fp16_exact
from oracle import attention as att
from oracle import quant

pytestmark = pytest.mark.gpu

P = 32
CONTEXT = 32768


def plan(layers: int, pages: int, seed: int = 0):
    """bench.py's configuration-4 plan: the downgrades (layer, page, tier)
    and the restores."""
    keys = [(l, p) for l in range(layers) for p in range(pages)]
    order = np.random.default_rng(seed).permutation(len(keys))
    n4, n2 = len(keys) // 2, len(keys) // 4
    n8 = int(round(0.1 * n4))
    down = [(*keys[i], 2) for i in order[:n4]] + [(*keys[i], 3) for i in order[n4:n4 + n2]]
    up = [(*keys[i], 1) for i in order[:n8]]
    return down, up


def test_config4_requant_plan_at_full_size_is_the_oracle():
    from microinfer import _microinfer as m
    from microinfer import workloads as w
    d = m.device
    shape = w.QWEN_15B
    L, kv, hd, heads = shape.layers, shape.kv_heads, shape.head_dim, shape.heads
    pages = CONTEXT // P
    sizes = [quant.page_bytes(t, kv, hd, P) for t in range(4)]
    alloc = m.PagedKVCache(sizes, [L * pages + 2 * L + 8] * 4)
    cache = d.KVPages(alloc, L, P, kv, hd, m.Tier.FP16, d.Halves.Both, [], True)
    rng = np.random.default_rng(0)
    outliers = w.outlier_channels(rng, shape.kv_width)
    rows = []
    announce("config4: store", L, "layers of", CONTEXT)
    cache.reserve(CONTEXT)
    for layer in range(L):
        k, v = w.kv_rows(rng, CONTEXT, shape, outliers)
        # All rows but the last, then the last: the open page keeps the own
        # page's first 31 rows for the decode at the end.
        for a, b in ((0, CONTEXT - 1), (CONTEXT - 1, CONTEXT)):
            cache.store(layer, m.upload_fp16(k[a:b].astype(np.float32)),
                        m.upload_fp16(v[a:b].astype(np.float32)), a, b - a)
        rows.append((k, v))
    m.synchronize()
    assert (cache.page_tiers()[:, :pages] == 0).all()

    down, up = plan(L, pages)
    assert (len(down), len(up)) == (21504, 1434)
    g = alloc.granule_bytes
    cache.pin_shadows(len(down))
    for tier in (2, 3):
        n = sum(1 for _, _, t in down if t == tier)
        alloc.keep_spare_granules(tier, -(-n * sizes[tier] // g))
    announce("config4: downgrade batch", len(down))
    cache.move_pages(np.asarray(down, np.int32))
    batch = cache.last_batch
    assert batch["moves"] == len(down) and batch["shadows_taken"] == len(down)
    for tier in (2, 3):
        alloc.keep_spare_granules(tier, 0)
    alloc.drain_releases()
    announce("config4: restore batch", len(up))
    cache.move_pages(np.asarray(up, np.int32))
    batch = cache.last_batch
    assert batch["moves"] == len(up) and batch["shadows_taken"] == 0
    alloc.drain_releases()
    m.synchronize()

    want = np.zeros((L, pages), np.int8)
    for layer, page, tier in down + up:
        want[layer, page] = tier
    np.testing.assert_array_equal(cache.page_tiers()[:, :pages], want)
    np.testing.assert_array_equal(cache.shadowed()[:, :pages], want != 0)
    assert np.bincount(want.ravel(), minlength=4).tolist() == [7168, 1434, 12902, 7168]

    announce("config4: page bytes and shadows")
    bad = []
    for layer in range(L):
        k, v = rows[layer]
        for page in range(pages):
            kp, vp = k[page * P:(page + 1) * P], v[page * P:(page + 1) * P]
            tier = int(want[layer, page])
            fp16 = quant.fp16_page(kp, vp)
            expect = fp16 if tier == 0 else quant.quantise_page(kp, vp, tier, P)
            if not np.array_equal(alloc.read(layer, page), expect):
                bad.append(("page", layer, page, tier))
            elif tier and not np.array_equal(cache.shadow(layer, page), fp16):
                bad.append(("shadow", layer, page, tier))
    assert not bad, f"{len(bad)} pages differ from the oracle, first {bad[:5]}"

    for tier in range(4):
        keys = alloc.pages(tier)
        assert alloc.spare_granules(tier) == 0
        assert alloc.mapped_bytes(tier) == -(-len(keys) * sizes[tier] // g) * g, tier
        for slot in (0, len(keys) // 2, len(keys) - 1):
            assert alloc.locate(*keys[slot]) == (tier, slot)

    layer = L - 1
    k, v = rows[layer]
    q = fp16_exact(rng.standard_normal((1, heads, hd)))
    out, mass = d.empty(heads * hd), d.empty_f32(heads * pages)
    announce("config4: decode of layer", layer)
    cache.attention(layer, m.upload_fp16(q.reshape(-1)), None, None, out, 1, CONTEXT, heads, kv,
                    hd, m.upload_fp16(k[-1:].astype(np.float32)),
                    m.upload_fp16(v[-1:].astype(np.float32)), mass,
                    d.empty_f32(d.attention_partials(hd)))
    own = pages - 1
    sealed = [alloc.read(layer, i) for i in range(own)]
    got = out.to_numpy().reshape(1, heads, hd)
    expect, expect_mass, bound = att.causal_decode(q, sealed, [int(t) for t in want[layer, :own]],
                                                   k[own * P:], v[own * P:], kv, hd, P,
                                                   with_bound=True)
    assert_attention_close(got, expect, "config4 decode", bound)
    assert_mass_close(mass.to_numpy().reshape(heads, pages), expect_mass, "config4 mass")
