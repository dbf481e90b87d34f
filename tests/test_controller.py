"""The precision controller's plans and the batching of their moves: host
logic, no device (reference: src/microinfer/controller.py, engine.py:322-357,
tests/test_controller.py).

Pinned by brute force: a greedy that literally takes the cheapest next move
of any page, one at a time, from a heap, must give the vectorised plan move
for move (tests/test_controller.py:390-443 is the reference's version of
this check); and by the behaviours the reference's tests state."""

import heapq
import math

import numpy as np
import pytest

from microinfer import controller, monitor
from microinfer.controller import TIERS

MIB = 1 << 20
#: Qwen2.5-0.5B page bytes and rounded round-trip errors, the reference's
#: fixture constants (tests/test_controller.py:24-29).
PAGE_BYTES = {"FP16": 16384, "INT8": 8960, "INT4": 4864, "INT2": 2816}
ERRORS = {"FP16": 0.0, "INT8": 2.2e-5, "INT4": 6.4e-3, "INT2": 0.161}
SECONDS = {(a, b): 1e-4 for a in PAGE_BYTES for b in PAGE_BYTES if a != b}
THRESHOLDS = monitor.Thresholds(red_below_bytes=512 * MIB, yellow_below_bytes=1024 * MIB,
                                persist_polls=3)
P = 32


def arrays(layers, pages, tier=0, score=np.nan):
    return np.full((layers, pages), score), np.full((layers, pages), tier, dtype=np.int8)


def make(target, scores, tiers, floor=0, positions=None, level=monitor.YELLOW, budget=0.02,
         options=controller.DEFAULT_OPTIONS):
    positions = tiers.shape[1] * P + floor if positions is None else positions
    return controller.target_plan_arrays(target, level, scores, tiers, PAGE_BYTES, ERRORS,
                                         move_seconds=SECONDS, positions=positions,
                                         page_tokens=P, recency_floor=floor,
                                         budget_seconds=budget, options=options)


def greedy(target, scores, tiers, floor=0, positions=None, options=controller.DEFAULT_OPTIONS):
    """One move at a time: the cheapest next downgrade of any candidate page,
    a page's cost never below its previous step's, ties by (score, page,
    layer, step)."""
    positions = tiers.shape[1] * P + floor if positions is None else positions
    eligible = controller.candidates(tiers, positions, P, floor)
    if options.protect_first_page:
        eligible[:, 0] = False
    known = scores[eligible & ~np.isnan(scores)]
    neutral = known.mean() if known.size else 1.0
    score = options.weighed(np.where(np.isnan(scores), neutral, scores))
    nbytes = [PAGE_BYTES[t] for t in TIERS]
    err = [ERRORS[t] for t in TIERS]
    lowest = TIERS.index(options.lowest_tier)

    def step_cost(layer, page, s, before):
        if options.importance_only:
            alone = score[layer, page]
        else:
            alone = score[layer, page] * (err[s + 1] - err[s]) / (nbytes[s] - nbytes[s + 1])
        return max(before, alone)

    heap = []
    for layer, page in zip(*np.nonzero(eligible)):
        s = int(tiers[layer, page])
        if s < lowest:
            c = step_cost(layer, page, s, -math.inf)
            heapq.heappush(heap, (c, score[layer, page], page, layer, s))
    moves, got = [], 0
    while heap and got < target:
        c, sc, page, layer, s = heapq.heappop(heap)
        moves.append((layer, page, s, c))
        got += nbytes[s] - nbytes[s + 1]
        if s + 1 < lowest:
            heapq.heappush(heap, (step_cost(layer, page, s + 1, c), sc, page, layer, s + 1))
    return moves, got


def as_moves(plan):
    return [(int(l), int(p), int(s), float(c))
            for l, p, s, c in zip(plan.layers, plan.pages, plan.current, plan.costs)]


@pytest.mark.parametrize("seed", range(12))
def test_the_plan_is_the_greedy_move_for_move(seed):
    rng = np.random.default_rng(seed)
    layers, pages = int(rng.integers(1, 5)), int(rng.integers(1, 40))
    tiers = rng.choice([0, 0, 0, 1, 2, 3, controller.EVICTED, -1],
                       size=(layers, pages)).astype(np.int8)
    scores = rng.lognormal(size=(layers, pages))
    scores[rng.random((layers, pages)) < 0.2] = np.nan
    scores[rng.random((layers, pages)) < 0.1] = 0.0
    if seed % 3 == 0:
        scores[:] = 0.5                                     # ties everywhere
    floor = [0, 64, 128][seed % 3]
    positions = pages * P + [0, 10, 200][seed % 3]
    options = [controller.DEFAULT_OPTIONS, controller.PlanOptions(lowest_tier="INT4"),
               controller.PlanOptions(importance_only=True),
               controller.PlanOptions(protect_first_page=True,
                                      layer_weights=tuple(rng.uniform(0.5, 2, layers)))][seed % 4]
    for target in (1, 7000, 50000, 10 ** 9):
        plan = make(target, scores, tiers, floor, positions, options=options)
        want, got = greedy(target, scores, tiers, floor, positions, options)
        assert as_moves(plan) == want, (seed, target)
        assert np.all(tiers[plan.layers, plan.pages] >= 0)
        assert plan.reclaimed_bytes == got
        assert plan.short == (got < target)


def test_the_plan_meets_the_target_and_overshoots_by_less_than_one_move():
    rng = np.random.default_rng(1)
    scores, tiers = arrays(2, 30)
    scores[:] = rng.lognormal(size=scores.shape)
    for target in (1, 20000, 123457):
        plan = make(target, scores, tiers)
        assert plan.reclaimed_bytes >= target
        assert plan.reclaimed_bytes - plan.saved[-1] < target
    # Through plan(): the target is YELLOW's line plus the margin less the headroom.
    keys = {(l, p): "FP16" for l in range(2) for p in range(30)}
    s = {k: 1.0 for k in keys}
    headroom = THRESHOLDS.yellow_below_bytes - 100000
    plan = controller.plan(headroom, THRESHOLDS, s, keys, PAGE_BYTES, ERRORS, move_seconds=SECONDS,
                           positions=30 * P + 128, page_tokens=P, margin_bytes=4096)
    assert plan.target_bytes == 104096 and plan.reclaimed_bytes >= 104096
    green = controller.plan(THRESHOLDS.yellow_below_bytes, THRESHOLDS, s, keys, PAGE_BYTES,
                            ERRORS, move_seconds=SECONDS, positions=30 * P + 128, page_tokens=P)
    assert len(green) == 0 and green.level == monitor.GREEN


def test_a_move_is_one_tier_down_and_equal_scores_go_breadth_first():
    scores, tiers = arrays(1, 10, score=1.0)
    plan = make(10 * 7424, scores, tiers)
    assert list(plan.lower - plan.current) == [1] * 10
    assert list(plan.current) == [0] * 10          # every page to INT8 before any deeper
    assert list(plan.pages) == list(range(10))     # oldest first among equals
    deeper = make(10 * 7424 + 1, scores, tiers)
    assert deeper.current[-1] == 1                 # then one to INT4


def test_a_near_zero_score_goes_deep_first_and_int2_only_when_outweighed():
    scores, tiers = arrays(1, 6, score=1.0)
    scores[0, 3] = 1e-9
    plan = make(3 * 7000, scores, tiers)
    assert [(int(p), int(s)) for p, s in zip(plan.pages[:3], plan.current[:3])] == \
        [(3, 0), (3, 1), (3, 2)]
    # Equal scores: INT2 comes after every page reached INT4.
    scores, tiers = arrays(1, 6, score=1.0)
    plan = make(6 * (16384 - 4864) + 1, scores, tiers)
    assert int(plan.current[-1]) == 2 and sum(plan.current == 2) == 1


def test_unscored_pages_go_oldest_first_and_no_deeper_than_an_average_one():
    scores, tiers = arrays(2, 8)
    plan = make(5 * 7424, scores, tiers)
    assert [(int(l), int(p)) for l, p in zip(plan.layers, plan.pages)] == \
        [(0, 0), (1, 0), (0, 1), (1, 1), (0, 2)]
    # A page without a score takes the mean of the scored ones.
    scores, tiers = arrays(1, 3)
    scores[0, :2] = [0.5, 1.5]
    plan = make(10 ** 9, scores, tiers)
    assert np.all(plan.scores[plan.pages == 2] == 1.0)


def test_no_plan_names_a_page_within_the_recency_floor():
    scores, tiers = arrays(2, 10, score=1.0)
    for floor, positions in ((128, 10 * P), (0, 10 * P - 5), (64, 9 * P + 7)):
        plan = make(10 ** 9, scores, tiers, floor, positions)
        last_free = (positions - floor) // P     # pages whose end precedes the floor
        assert np.all(plan.pages < last_free)
        assert plan.recency_floor == floor and plan.short
    assert len(make(10 ** 9, scores, tiers, 128, 100)) == 0


def test_batches_fit_the_budget_at_yellow_and_red_is_one():
    scores, tiers = arrays(1, 40, score=1.0)
    plan = make(40 * 7424, scores, tiers, budget=0.00035)
    assert plan.batch_bounds[0] == (0, 3) and len(plan.batch_bounds) == 14
    assert sum(b - a for a, b in plan.batch_bounds) == len(plan)
    red = make(40 * 7424, scores, tiers, level=monitor.RED, budget=0.00035)
    assert red.batch_bounds == ((0, len(red)),)
    assert controller.batch_bounds(np.array([0.5, 0.1]), monitor.YELLOW, 0.2) == ((0, 1), (1, 2))


def test_what_the_controller_refuses():
    scores, tiers = arrays(1, 4, score=1.0)
    with pytest.raises(ValueError, match="floor"):
        make(10, scores, tiers, floor=-1)
    with pytest.raises(ValueError, match="positions"):
        make(10, scores, tiers, positions=-1)
    bad = scores.copy()
    bad[0, 1] = -0.5
    with pytest.raises(ValueError, match="mass"):
        make(10, bad, tiers)
    with pytest.raises(ValueError, match="tier"):
        controller.PlanOptions(lowest_tier="FP16")
    with pytest.raises(ValueError, match="weight"):
        controller.PlanOptions(layer_weights=(1.0, -2.0))
    with pytest.raises(ValueError, match="tier"):
        controller.plan(THRESHOLDS.red_below_bytes, THRESHOLDS, {(0, 0): 1.0}, {(0, 0): "FP8"},
                        PAGE_BYTES, ERRORS, move_seconds=SECONDS, positions=200, page_tokens=P)
    with pytest.raises(ValueError, match="no score"):
        controller.plan(THRESHOLDS.red_below_bytes, THRESHOLDS, {}, {(0, 0): "FP16"},
                        PAGE_BYTES, ERRORS, move_seconds=SECONDS, positions=200, page_tokens=P)
    with pytest.raises(ValueError, match="nest"):
        monitor.Thresholds(red_below_bytes=10, yellow_below_bytes=5, persist_polls=1)


def upgrades(headroom, scores, tiers, shadowed, last=None, now=100.0, **kw):
    return controller.upgrade_plan_arrays(headroom, THRESHOLDS, scores, tiers, shadowed,
                                          PAGE_BYTES, ERRORS, move_seconds=SECONDS,
                                          last_downgrade_seconds=last, now_seconds=now, **kw)


def upgrade_greedy(available, scores, tiers, shadowed):
    """One upgrade at a time: the largest next gain of any page, a page's
    gain never above its previous step's, ties (score, page, layer, step)
    all descending; stop at the first that does not fit."""
    up = (tiers > 0) & shadowed
    known = scores[up & ~np.isnan(scores)]
    score = np.where(np.isnan(scores), known.mean() if known.size else 1.0, scores)
    nbytes = [PAGE_BYTES[t] for t in TIERS]
    err = [ERRORS[t] for t in TIERS]

    def gain(l, p, k, before):
        return min(before, score[l, p] * (err[k] - err[k - 1]) / (nbytes[k - 1] - nbytes[k]))

    heap = []
    for l, p in zip(*np.nonzero(up)):
        k = int(tiers[l, p])
        heapq.heappush(heap, (-gain(l, p, k, math.inf), -score[l, p], -p, -l, -k))
    moves, left = [], available
    while heap:
        g, sc, p, l, k = heapq.heappop(heap)
        l, p, k = -l, -p, -k
        need = nbytes[k - 1] - nbytes[k]
        if need > left:
            break
        left -= need
        moves.append((l, p, k))
        if k - 1 > 0:
            heapq.heappush(heap, (-gain(l, p, k - 1, -g), sc, -p, -l, -(k - 1)))
    return moves


@pytest.mark.parametrize("seed", range(8))
def test_the_upgrade_plan_is_the_greedy_move_for_move(seed):
    rng = np.random.default_rng(100 + seed)
    layers, pages = int(rng.integers(1, 4)), int(rng.integers(1, 30))
    tiers = rng.choice([0, 1, 2, 3], size=(layers, pages)).astype(np.int8)
    scores = rng.lognormal(size=(layers, pages))
    scores[rng.random((layers, pages)) < 0.2] = np.nan
    shadowed = rng.random((layers, pages)) < 0.8
    for extra in (1, 30000, 10 ** 8):
        headroom = THRESHOLDS.yellow_below_bytes + controller.DEFAULT_UPGRADE_SPIKE_BYTES + extra
        plan = upgrades(headroom, scores, tiers, shadowed)
        want = upgrade_greedy(extra, scores, tiers, shadowed)
        assert [(int(l), int(p), int(k)) for l, p, k in
                zip(plan.layers, plan.pages, plan.current)] == want
        assert plan.taken_bytes <= extra


def test_upgrades_wait_for_green_the_cooldown_the_line_and_a_shadow():
    scores, tiers = arrays(1, 4, tier=2, score=1.0)
    shadowed = np.ones((1, 4), bool)
    line = THRESHOLDS.yellow_below_bytes + controller.DEFAULT_UPGRADE_SPIKE_BYTES
    assert "GREEN" in upgrades(THRESHOLDS.red_below_bytes, scores, tiers, shadowed).held_by
    assert "cooldown" in upgrades(line + 10 ** 9, scores, tiers, shadowed, last=97.0).held_by
    assert len(upgrades(line + 10 ** 9, scores, tiers, shadowed, last=94.0)) == 8
    assert "headroom" in upgrades(line, scores, tiers, shadowed).held_by
    with pytest.raises(ValueError, match="clock"):
        upgrades(line + 10 ** 9, scores, tiers, shadowed, last=101.0)
    shadowed[0, 1] = False
    plan = upgrades(line + 10 ** 9, scores, tiers, shadowed)
    assert 1 not in plan.pages and len(plan) == 6


def test_upgrades_undo_a_plan_backwards():
    rng = np.random.default_rng(7)
    scores, tiers = arrays(2, 12)
    scores[:] = rng.lognormal(size=scores.shape)
    plan = make(60000, scores, tiers)
    after = tiers.copy()
    for l, p, t in zip(plan.layers, plan.pages, plan.lower):
        after[l, p] = t
    shadowed = after > 0
    line = THRESHOLDS.yellow_below_bytes + controller.DEFAULT_UPGRADE_SPIKE_BYTES
    up = upgrades(line + 10 ** 9, scores, after, shadowed)
    assert [(int(l), int(p), int(c)) for l, p, c in zip(up.layers, up.pages, up.higher)] == \
        [(int(l), int(p), int(c)) for l, p, c in zip(plan.layers, plan.pages, plan.current)][::-1]


def test_share_bytes_given_back_and_eviction():
    tiers = np.zeros((1, 10), np.int8)
    tiers[0, :3] = 2
    held = 3 * 4864 + 5 * 16384          # candidates: pages 0..7 (floor 64 -> 8 full pages)
    got = controller.share_target_bytes(0.5, tiers, PAGE_BYTES, positions=10 * P,
                                        page_tokens=P, recency_floor=64)
    assert got == math.ceil(held - 0.5 * 16384 * 8)
    after = tiers.copy()
    after[0, 5] = 3
    after[0, 0] = controller.EVICTED
    assert controller.bytes_given_back(tiers, after, PAGE_BYTES) == (16384 - 2816) + 4864
    scores, t2 = arrays(1, 6, score=1.0)
    plan = make(10 ** 9, scores, t2)
    ev = controller.eviction_plan(3 * 16384, plan, t2, PAGE_BYTES)
    assert len(ev) == 3 and ev.reclaimed_bytes == 3 * 16384 and not ev.short
    assert list(ev.pages) == [0, 1, 2]    # all left at INT2: the first taken there first


class _Plan:
    def __init__(self, moves):
        self.layers = np.array([m[0] for m in moves])
        self.pages = np.array([m[1] for m in moves])
        self.current = np.array([m[2] for m in moves])
        self.target = self.current + 1

    def __len__(self):
        return len(self.layers)


def test_next_batch_collapses_chains_skips_stale_moves_and_keeps_to_its_caps():
    from microinfer import engine
    from microinfer._microinfer import Tier
    sizes = [PAGE_BYTES[t] for t in TIERS]
    held = np.zeros((2, 4), np.int8)
    held[1, 3] = 2
    shadowed = np.zeros((2, 4), bool)
    shadowed[0, 1] = True
    # (0,0) FP16 -> INT8 -> INT4 collapses to one move; (1,3) is at INT4
    # already, so its FP16 -> INT8 move is skipped; (0,1) has a shadow.
    plan = _Plan([(0, 0, 0), (1, 3, 0), (0, 1, 0), (0, 0, 1), (0, 2, 0)])
    b = engine.next_batch(plan, 0, held, shadowed, sizes, 10 ** 9, 1.0, 1e-3)
    assert b.moves == [(0, 0, Tier.INT4), (0, 1, Tier.INT8), (0, 2, Tier.INT8)]
    assert (b.end, b.skipped, b.bytes) == (5, 1, sizes[2] + 2 * sizes[1])
    # Seconds: a move and a shadow pin for FP16 without a shadow.
    b = engine.next_batch(plan, 0, held, shadowed, sizes, 10 ** 9, 2e-3, 1e-3)
    assert b.moves == [(0, 0, Tier.INT8)] and b.end == 2
    # Bytes: the first move is always taken; the stale move after it is
    # passed over before the cap stops the batch.
    b = engine.next_batch(plan, 0, held, shadowed, sizes, 1, 1.0, 1e-3)
    assert b.moves == [(0, 0, Tier.INT8)] and (b.end, b.skipped) == (2, 1)
    # A chain ending where the page is moves nothing.
    back = _Plan([(0, 0, 0)])
    back.target = np.array([0])
    assert engine.next_batch(back, 0, held, shadowed, sizes, 10 ** 9, 1.0, 1e-3).moves == []
    assert engine.move_seconds({"moves": 4, "seconds": 0.02, "shadows_taken": 0}) == 0.005
    assert engine.move_seconds({"moves": 40, "seconds": 0.0105, "shadows_taken": 100}) == \
        pytest.approx((0.0105 - 5e-4 - 100 * 2e-5) / 40)
