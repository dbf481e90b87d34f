"""The reference's host callers, replayed against this build's `_microinfer`:
the device calls of Engine._apply (src/microinfer/engine.py:1750-1802) with
fixed move lists in place of the precision controller's plans, and of
PagedCache.attend (src/microinfer/model.py:273-286).

The reference's own host code is the drop-in caller: nothing here is a
planner. Each replay restates the device calls those functions make (the
batch loop, its free-memory margin and its retry at half size; not the
engine's time budget) and checks what the device then holds.

GPU parity tests: after each plan every page holds, to the bit, the oracle's
quantise_page of its FP16 rows at the tier the plan leaves it (an upgrade,
its FP16 shadow); the scores attend folds are, to the bit, the oracle's fold
of the step's masses, on the steps the cadence names."""

import numpy as np
import pytest

from conftest import announce, assert_attention_close, assert_mass_close
from oracle import attention as att
from oracle import ewma, quant
from test_gpu_kv_pages import LAYERS, mi, normal, page_sizes, pages_for, put, store_in_runs

pytestmark = pytest.mark.gpu

P, KV, HD, HEADS = 32, 2, 128, 12


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


def apply_like_the_engine(pages, plan, page_bytes, bytes_cap=None):
    """A restatement (not the reference's own code) of the device calls
    Engine._apply makes (engine.py:1750-1802) over a plan of (layer, page,
    from, to) steps, without its time budget: each batch takes the plan's
    moves from the cursor whose page is where the step expects
    (page_tiers()), each page once, while its new pages fit the device's free
    memory less the engine's batch margin (two granules a tier,
    engine.py:1804-1809) and the cap; move_pages(batch); on OutOfMemory the
    same batch again at half its bytes, and a single move that cannot
    allocate ends the plan. Returns (moves applied, batches, skipped,
    stopped, retries)."""
    m = mi()
    i, applied, batches, skipped, stopped, retries = 0, 0, 0, 0, None, 0
    cap = bytes_cap
    margin = 2 * 4 * m.granule_bytes()
    while i < len(plan):
        free = m.device_memory_info()["free"] - margin
        limit = free if cap is None else min(free, cap)
        held = pages.page_tiers()
        shadowed = pages.shadowed()
        assert shadowed.shape == held.shape
        moves, seen, new_bytes, j = [], set(), 0, i
        while j < len(plan):
            layer, page, expect, target = plan[j]
            if int(held[layer, page]) != expect or (layer, page) in seen:
                if (layer, page) in seen:
                    break                    # a page moves once a batch
                skipped += 1
                j += 1
                continue
            if moves and new_bytes + page_bytes[target] > limit:
                break
            moves.append((layer, page, target))
            seen.add((layer, page))
            new_bytes += page_bytes[target]
            j += 1
        if moves:
            try:
                pages.move_pages(moves)
            except m.OutOfMemory:
                if len(moves) == 1:
                    stopped = "stopped"
                    break
                cap = new_bytes // 2
                retries += 1
                continue
            last = pages.last_batch
            assert last["moves"] == len(moves) and last["seconds"] > 0
            applied += len(moves)
        batches += 1
        i = j
    return applied, batches, skipped, stopped, retries


def test_plans_applied_as_the_engine_applies_them():
    """Downgrades in batches capped at a few pages' bytes (a page moved twice
    across batches, a stale step skipped), one batch that fails to allocate
    and is retried at half size, then the upgrades back from the shadows:
    every page's bytes are the oracle's at every end."""
    m = mi()
    rng = np.random.default_rng(41)
    seq = P * 14 + 9
    k, v = normal(rng, seq, KV, HD), normal(rng, seq, KV, HD)
    sizes = page_sizes(P, KV, HD)
    alloc, cache = pages_for(P, KV, HD, 0, always_seal=True)
    for layer in range(LAYERS):
        store_in_runs(cache, layer, k, v, [seq])
    tiers = cache.page_tiers().copy()
    assert (tiers == 0).all() and tiers.shape == (LAYERS, seq // P)
    # A fixed plan: FP16 -> INT8/INT4 first, some pages later INT4 -> INT2,
    # and one stale step (its page is not where the step expects).
    plan, want = [], tiers.copy()
    for page in range(0, 13):
        for layer in range(LAYERS):
            target = 1 if (page + layer) % 3 == 0 else 2
            plan.append((layer, page, 0, target))
            want[layer, page] = target
    for page in range(1, 13, 4):
        plan.append((0, page, int(want[0, page]), 3))
        want[0, page] = 3
    plan.append((1, 13, 2, 3))               # stale: page 13 is at FP16
    announce("engine downgrades", len(plan))
    # The first batch needs the INT8 and INT4 ranges' first granules: the
    # first map fails, and the batch is tried again at half its bytes.
    m.fail_next_granules(1)
    applied, batches, skipped, stopped, retries = apply_like_the_engine(cache, plan, sizes,
                                                                        bytes_cap=3 * sizes[1])
    m.fail_next_granules(0)
    assert stopped is None and skipped == 1 and batches > 4 and retries == 1
    assert applied == len(plan) - 1
    check_pages(alloc, cache, k, v, want, "downgrades")
    # More moves, uncapped: one batch.
    again = [(1, page, int(want[1, page]), 3) for page in (0, 3, 6, 9)]
    for _, page, _, _ in again:
        want[1, page] = 3
    applied, batches, _, stopped, _ = apply_like_the_engine(cache, again, sizes)
    assert stopped is None and applied == len(again) and batches == 1
    check_pages(alloc, cache, k, v, want, "one batch")
    # Upgrades at GREEN: every moved page back to FP16 from its shadow.
    shadowed = cache.shadowed()
    assert np.all(shadowed[want > 0]) and not np.any(shadowed[want == 0])
    up = [(layer, page, int(want[layer, page]), 0) for layer in range(LAYERS)
          for page in range(seq // P) if want[layer, page] > 0]
    announce("engine upgrades", len(up))
    applied, _, skipped, stopped, _ = apply_like_the_engine(cache, up, sizes)
    assert stopped is None and skipped == 0 and applied == len(up)
    check_pages(alloc, cache, k, v, tiers, "upgrades")


def test_paged_cache_attend_folds_scores_on_its_cadence():
    """model.py:273-286: a step is scored when it is one query and the
    positions it attends are a multiple of R = 4; a scored step's attention
    writes the mass, and ImportanceScores.fold takes it, for the step's
    pages. Every output is the oracle's; the scores are the oracle's fold of
    the masses the kernel wrote, to the bit; unscored steps change none."""
    m = mi()
    d = m.device
    rng = np.random.default_rng(43)
    seq0, score_every = P * 6 + 1, 4
    total = seq0 + 11
    k, v = normal(rng, total, KV, HD), normal(rng, total, KV, HD)
    tmap = [[(i * 5) % 4 for i in range(total // P + 1)] for _ in range(LAYERS)]
    alloc, cache = pages_for(P, KV, HD, 0, tier_map=tmap, always_seal=True)
    max_pages = total // P + 1
    scores = d.ImportanceScores(LAYERS, max_pages)
    mass = d.empty_f32(HEADS * max_pages)
    part = d.empty_f32(d.attention_partials(HD))
    for layer in range(LAYERS):
        store_in_runs(cache, layer, k[:seq0], v[:seq0], [seq0])
    folded = []
    for t in range(seq0, total):
        seq_k = t + 1
        cache.reserve(seq_k)
        for layer in range(LAYERS):
            cache.store(layer, put(k[t:t + 1]), put(v[t:t + 1]), t, 1)
        for layer in range(LAYERS):
            q = normal(rng, 1, HEADS, HD)
            out = d.empty(HEADS * HD)
            before = scores.download()
            scored = seq_k % score_every == 0
            announce("attend", seq_k, layer, scored)
            # The reference's calls, in its order.
            cache.attention(layer, put(q), None, None, out, 1, seq_k, HEADS, KV, HD,
                            put(k[t:t + 1]), put(v[t:t + 1]), mass if scored else None, part)
            if scored:
                scores.fold(layer, mass, HEADS, -(-seq_k // d.page_tokens))
            own = (seq_k - 1) // P
            sealed = [alloc.read(layer, p) for p in range(own)]
            stiers = [int(alloc.locate(layer, p)[0]) for p in range(own)]
            want, want_mass, bound = att.causal_decode(q, sealed, stiers, k[own * P:seq_k],
                                                       v[own * P:seq_k], KV, HD, P,
                                                       with_bound=True)
            assert_attention_close(out.to_numpy().reshape(1, HEADS, HD), want, f"step {t}", bound)
            if scored:
                pages = -(-seq_k // P)
                got_mass = mass.to_numpy()[:HEADS * pages].reshape(HEADS, pages)
                assert_mass_close(got_mass, want_mass, f"step {t} mass")
                folded.append((layer, got_mass.astype(np.float32)))
            else:
                np.testing.assert_array_equal(scores.download(), before)
    assert len(folded) == 3 * LAYERS          # positions 196, 200 and 204
    np.testing.assert_array_equal(scores.download(), ewma.host_ewma(folded, LAYERS, max_pages))
