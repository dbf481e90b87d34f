"""The controller's plans applied to a device cache, and the cache a model's
layers attend through (reference: engine.py:1750-1802 Engine._apply,
model.py:273-286 PagedCache.attend).

GPU parity tests: after a plan, every page holds, to the bit, the oracle's
quantise_page of its FP16 rows at the tier the plan leaves it; an upgrade
plan restores the FP16 bytes; the scores a PagedCache folds are, to the bit,
the oracle's fold of the step's masses, on the steps the cadence names."""

import numpy as np
import pytest

from conftest import announce
from oracle import ewma, quant
from test_gpu_kv_pages import LAYERS, mi, normal, page_sizes, pages_for, put, store_in_runs

pytestmark = pytest.mark.gpu

P, KV, HD = 32, 2, 128
ERRORS = {"FP16": 0.0, "INT8": 2.2e-5, "INT4": 6.4e-3, "INT2": 0.161}
SECONDS = {(a, b): 1e-4 for a in ERRORS for b in ERRORS if a != b}


def expected_page(k, v, page, tier):
    kp = k[page * P:(page + 1) * P].astype(np.float16)
    vp = v[page * P:(page + 1) * P].astype(np.float16)
    return quant.fp16_page(kp, vp) if tier == 0 else quant.quantise_page(kp, vp, tier, P)


def check_pages(alloc, cache, k, v, tiers, what):
    np.testing.assert_array_equal(cache.page_tiers(), tiers, err_msg=what)
    for layer in range(tiers.shape[0]):
        for page in range(len(k) // P):
            np.testing.assert_array_equal(alloc.read(layer, page),
                                          expected_page(k, v, page, int(tiers[layer, page])),
                                          err_msg=f"{what}: layer {layer} page {page}")


def test_a_plan_applied_in_batches_leaves_each_page_the_oracle_s_bytes():
    from microinfer import controller, engine, monitor
    rng = np.random.default_rng(41)
    seq = P * 14 + 9
    k, v = normal(rng, seq, KV, HD), normal(rng, seq, KV, HD)
    sizes = page_sizes(P, KV, HD)
    page_bytes = dict(zip(controller.TIERS, sizes))
    caches = []
    for _ in range(2):
        alloc, cache = pages_for(P, KV, HD, 0, always_seal=True)
        for layer in range(LAYERS):
            store_in_runs(cache, layer, k, v, [seq])
        caches.append((alloc, cache))
    tiers = caches[0][1].page_tiers()
    scores = rng.lognormal(size=tiers.shape)
    scores[0, 3] = np.nan
    scores[1, 2] = 1e-9
    plan = controller.target_plan_arrays(12 * (sizes[0] - sizes[2]), monitor.YELLOW, scores,
                                         tiers, page_bytes, ERRORS, move_seconds=SECONDS,
                                         positions=seq, page_tokens=P, recency_floor=64)
    assert len(plan) > 12 and len(set(zip(plan.layers, plan.pages))) < len(plan)
    want = tiers.copy()
    for layer, page, lower in zip(plan.layers, plan.pages, plan.lower):
        want[layer, page] = lower
    # All at once, as at RED.
    announce("apply_plan", len(plan), "moves")
    alloc, cache = caches[0]
    done = engine.apply_plan(cache, plan, sizes)
    assert done.cursor == len(plan) and done.skipped == 0 and not done.stopped
    check_pages(alloc, cache, k, v, want, "apply_plan")
    # In batches of at most three new pages' bytes, each page once a batch.
    alloc, cache = caches[1]
    i, batches = 0, 0
    while i < len(plan):
        b = engine.next_batch(plan, i, cache.page_tiers(), cache.shadowed(), sizes,
                              3 * sizes[1], 1.0, 1e-4)
        announce("next_batch", i, b.end, len(b.moves))
        assert b.end > i and b.skipped == 0
        keys = [(layer, page) for layer, page, _ in b.moves]
        assert len(set(keys)) == len(keys)
        if b.moves:
            cache.move_pages(b.moves)
            assert cache.last_batch["moves"] == len(b.moves)
        i, batches = b.end, batches + 1
    assert batches > 4
    check_pages(alloc, cache, k, v, want, "next_batch")
    # Applying the plan again skips every move and moves nothing.
    again = engine.apply_plan(cache, plan, sizes)
    assert again.skipped == len(plan)
    check_pages(alloc, cache, k, v, want, "again")

    # Upgrades at GREEN restore from the shadows, the plan backwards.
    headroom = (monitor.DEFAULT.yellow_below_bytes + controller.DEFAULT_UPGRADE_SPIKE_BYTES
                + 10 ** 9)
    shadowed = cache.shadowed()
    assert np.all(shadowed[want > 0])
    up = controller.upgrade_plan_arrays(headroom, monitor.DEFAULT, scores, want, shadowed,
                                        page_bytes, ERRORS, move_seconds=SECONDS,
                                        last_downgrade_seconds=None)
    assert len(up) == len(plan)
    announce("upgrade", len(up), "moves")
    done = engine.apply_plan(cache, up, sizes, budget_seconds=1.0)
    assert done.cursor == len(up) and not done.stopped
    check_pages(alloc, cache, k, v, tiers, "upgrade")


def test_the_paged_cache_folds_scores_on_its_cadence_to_the_bit():
    from microinfer import engine
    m = mi()
    d = m.device
    heads = 12
    rng = np.random.default_rng(43)
    seq0 = P * 6 + 1
    total = seq0 + 11
    k, v = normal(rng, total, KV, HD), normal(rng, total, KV, HD)
    tmap = [[(i * 5) % 4 for i in range(total // P + 1)] for _ in range(LAYERS)]
    alloc, cache = pages_for(P, KV, HD, 0, tier_map=tmap, always_seal=True)
    max_pages = total // P + 1
    scores = d.ImportanceScores(LAYERS, max_pages)
    paged = engine.PagedCache(cache, heads, KV, HD, scores=scores, score_every=4)
    for layer in range(LAYERS):
        store_in_runs(cache, layer, k[:seq0], v[:seq0], [seq0])
    steps, folded = [], 0
    part = d.empty_f32(d.attention_partials(HD))
    for t in range(seq0, total):
        seq = t + 1
        pages = -(-seq // P)
        cache.reserve(seq)
        for layer in range(LAYERS):
            cache.store(layer, put(k[t:t + 1]), put(v[t:t + 1]), t, 1)
            q = put(normal(rng, 1, heads, HD))
            own_k, own_v = put(k[t:t + 1]), put(v[t:t + 1])
            before = scores.download()
            out = d.empty(heads * HD)
            paged.attend(layer, q, None, out, 1, seq, own_k, own_v, part)
            # The same step without the cache's scoring: the same output bits,
            # and the masses the fold takes.
            alone, mass = d.empty(heads * HD), d.empty_f32(heads * pages)
            cache.attention(layer, q, None, None, alone, 1, seq, heads, KV, HD, own_k, own_v,
                            mass, part)
            np.testing.assert_array_equal(out.to_numpy(), alone.to_numpy())
            announce("paged step", seq, "layer", layer)
            if seq % 4 == 0:
                steps.append((layer, mass.to_numpy().reshape(heads, pages).astype(np.float32)))
                folded += 1
            else:
                np.testing.assert_array_equal(scores.download(), before)
    assert folded == 3 * LAYERS          # positions 196, 200 and 204
    np.testing.assert_array_equal(scores.download(), ewma.host_ewma(steps, LAYERS, max_pages))
    with pytest.raises(ValueError, match="R >= 1"):
        engine.PagedCache(cache, heads, KV, HD, score_every=0)
