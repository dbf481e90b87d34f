"""The precision controller's plans: which pages move to which tier, so that
the cache gives back a byte target at the least cost in attention error
(reference: src/microinfer/controller.py; host logic, no device code).

A downgrade takes a page one tier down and saves bytes(current) -
bytes(lower) at a marginal cost of score x (error(lower) - error(current)) /
bytes saved, where `score` is the page's importance (its EWMA of attention
mass) and `error` a tier's logged round-trip error. The plan takes, again
and again, the cheapest next downgrade of any page, until the bytes meet the
target; a page's later downgrades cost no less than its earlier ones (each
costs at least the running maximum of its page), so the greedy is a sort of
every (page, step) by cost. Ties go to the lower score, then the older page,
then the lower layer, then the earlier step. A page without a score (NaN)
takes the mean score of the scored candidates (1.0 when none is).

The recency floor: a page whose last position is among the last W (128)
positions, the partly filled page and the open pages with it, is never a
candidate; nor is an evicted page (tier index 4).

Upgrades (GREEN only, after a cooldown since the last downgrade, within the
headroom above YELLOW's line less one P90 spike) run the other way: the
largest score x error removed / bytes taken first, a page's later upgrades
gaining no more than its earlier ones, ties to the higher score, then the
newer page, then the higher layer, then the page's first step; and they stop
at the first one that does not fit. Only pages holding an FP16 shadow can be
upgraded. Plans fall into batches whose estimated seconds fit a per-step
budget, except at RED, where a plan is one batch.

Tier maps are (layers, pages) int arrays of indices into TIERS (4 for an
evicted page, -1 for a page the cache does not hold); scores the same shape,
float, NaN where not yet scored.
"""

from __future__ import annotations

import functools
import math
import time
from collections.abc import Collection
from dataclasses import dataclass
from fractions import Fraction

import numpy as np

from .monitor import GREEN, RED, MIB, Level, Thresholds

TIERS = ("FP16", "INT8", "INT4", "INT2")
#: A tier map's index of an evicted page: one past the lowest tier, no bytes.
EVICTED = len(TIERS)
DEFAULT_MARGIN_BYTES = 64 * MIB
DEFAULT_BUDGET_SECONDS = 0.020
DEFAULT_RECENCY_FLOOR = 128
DEFAULT_UPGRADE_COOLDOWN_SECONDS = 5.0
DEFAULT_UPGRADE_SPIKE_BYTES = 512 * MIB


@dataclass(frozen=True)
class Downgrade:
    layer: int
    page: int
    current_tier: str
    target_tier: str
    bytes_saved: int
    cost: float
    score: float
    seconds: float


@dataclass(frozen=True)
class PlanOptions:
    """The planner's policy knobs (reference: controller.py:107-160):
    the lowest tier a plan may reach; importance_only (cost = the page's
    score alone, so pages go down in score order, all the way); protect the
    first page of every layer; a weight a layer multiplying its scores."""

    lowest_tier: str = "INT2"
    importance_only: bool = False
    protect_first_page: bool = False
    layer_weights: tuple | None = None

    def __post_init__(self):
        if self.lowest_tier not in TIERS[1:]:
            raise ValueError(f"the lowest tier is a quantised tier, one of {TIERS[1:]}; got "
                             f"{self.lowest_tier!r}")
        if self.layer_weights is not None:
            weights = tuple(float(w) for w in self.layer_weights)
            if not weights or any(not (math.isfinite(w) and w > 0) for w in weights):
                raise ValueError(f"a layer weight is positive and finite, one a layer; got "
                                 f"{self.layer_weights!r}")
            object.__setattr__(self, "layer_weights", weights)

    def weighed(self, scores: np.ndarray) -> np.ndarray:
        if self.layer_weights is None:
            return scores
        if len(self.layer_weights) != scores.shape[0]:
            raise ValueError(f"{len(self.layer_weights)} layer weights for a cache of "
                             f"{scores.shape[0]} layers")
        return scores * np.asarray(self.layer_weights)[:, None]


DEFAULT_OPTIONS = PlanOptions()


def batch_bounds(seconds: np.ndarray, level: Level,
                 budget_seconds: float) -> tuple[tuple[int, int], ...]:
    """[start, end) of each batch: at RED one batch of everything; else each
    batch as full as the budget lets it be, a move longer than the budget a
    batch of its own."""
    n = len(seconds)
    if n == 0:
        return ()
    if level == RED:
        return ((0, n),)
    bounds = []
    start, spent = 0, 0.0
    for i, s in enumerate(np.asarray(seconds, np.float64).tolist()):
        if i > start and spent + s > budget_seconds:
            bounds.append((start, i))
            start, spent = i, 0.0
        spent += s
    bounds.append((start, n))
    return tuple(bounds)


@dataclass(frozen=True, eq=False)
class Plan:
    """The downgrades in the order chosen (arrays, tiers as TIERS indices),
    and how they batch. `short`: every candidate went as low as it may and
    the target was still not met."""

    level: Level
    target_bytes: int
    short: bool
    recency_floor: int
    layers: np.ndarray
    pages: np.ndarray
    current: np.ndarray
    lower: np.ndarray
    saved: np.ndarray
    costs: np.ndarray
    scores: np.ndarray
    seconds: np.ndarray
    budget_seconds: float
    options: PlanOptions = DEFAULT_OPTIONS

    def __len__(self) -> int:
        return len(self.layers)

    @property
    def target(self) -> np.ndarray:
        return self.lower

    @property
    def reclaimed_bytes(self) -> int:
        return int(self.saved.sum())

    @functools.cached_property
    def batch_bounds(self) -> tuple[tuple[int, int], ...]:
        return batch_bounds(self.seconds, self.level, self.budget_seconds)

    def downgrade(self, i: int) -> Downgrade:
        return Downgrade(int(self.layers[i]), int(self.pages[i]), TIERS[self.current[i]],
                         TIERS[self.lower[i]], int(self.saved[i]), float(self.costs[i]),
                         float(self.scores[i]), float(self.seconds[i]))

    @functools.cached_property
    def downgrades(self) -> tuple[Downgrade, ...]:
        return tuple(self.downgrade(i) for i in range(len(self)))

    @functools.cached_property
    def batches(self) -> tuple[tuple[Downgrade, ...], ...]:
        return tuple(self.downgrades[a:b] for a, b in self.batch_bounds)


def _no_moves(level, recency_floor, budget_seconds, options) -> Plan:
    i, f = np.zeros(0, np.int64), np.zeros(0)
    return Plan(level, 0, False, recency_floor, i, i, i, i, i, f, f, f, budget_seconds, options)


def _check_plan_inputs(scores, tiers, positions, page_tokens, recency_floor) -> None:
    if recency_floor < 0:
        raise ValueError(f"the recency floor is a count of positions, >= 0; got {recency_floor}")
    if page_tokens <= 0 or positions < 0:
        raise ValueError(f"a cache holds positions >= 0 on pages of > 0; got {positions} "
                         f"positions on pages of {page_tokens}")
    if scores is not None and np.any(np.asarray(scores)[np.asarray(tiers) >= 0] < 0):
        raise ValueError("a score is a mass, >= 0")


def full_pages(tiers: np.ndarray, positions: int, page_tokens: int,
               recency_floor: int) -> np.ndarray:
    """Held or evicted pages whose last position precedes the floor's first."""
    tiers = np.asarray(tiers)
    last_end = (np.arange(tiers.shape[1]) + 1) * page_tokens
    return (tiers >= 0) & (last_end <= positions - recency_floor)[None, :]


def candidates(tiers: np.ndarray, positions: int, page_tokens: int,
               recency_floor: int) -> np.ndarray:
    """The pages a plan may downgrade: full pages before the floor, not evicted."""
    return full_pages(tiers, positions, page_tokens, recency_floor) & (np.asarray(tiers) != EVICTED)


def place_bytes(page_bytes: dict) -> np.ndarray:
    """Bytes held by a tier-map index: each tier's page bytes, then 0 (evicted)."""
    return np.array([page_bytes[t] for t in TIERS] + [0], dtype=np.int64)


def _neutral_score(scores: np.ndarray, among: np.ndarray) -> float:
    known = scores[among & ~np.isnan(scores)]
    return float(known.mean()) if known.size else 1.0


def _tier_tables(page_bytes: dict, errors: dict):
    return (np.array([page_bytes[t] for t in TIERS], dtype=np.int64),
            np.array([errors[t] for t in TIERS], dtype=np.float64))


def target_plan_arrays(target_bytes: int, level: Level, scores: np.ndarray, tiers: np.ndarray,
                       page_bytes: dict, errors: dict, *, move_seconds: dict, positions: int,
                       page_tokens: int, recency_floor: int = DEFAULT_RECENCY_FLOOR,
                       budget_seconds: float = DEFAULT_BUDGET_SECONDS,
                       options: PlanOptions = DEFAULT_OPTIONS) -> Plan:
    """The greedy plan reclaiming `target_bytes` (reference: controller.py:326-387)."""
    scores = np.asarray(scores, np.float64)
    tiers = np.asarray(tiers)
    _check_plan_inputs(scores, tiers, positions, page_tokens, recency_floor)
    if target_bytes <= 0:
        return _no_moves(level, recency_floor, budget_seconds, options)
    eligible = candidates(tiers, positions, page_tokens, recency_floor)
    if options.protect_first_page:
        eligible[:, 0] = False
    score = options.weighed(np.where(np.isnan(scores), _neutral_score(scores, eligible), scores))
    nbytes, err = _tier_tables(page_bytes, errors)
    n_steps = len(TIERS) - 1          # step s: tier s -> s + 1
    saved_by = nbytes[:-1] - nbytes[1:]
    seconds_by = np.array([move_seconds[(TIERS[s], TIERS[s + 1])] for s in range(n_steps)])
    lowest = TIERS.index(options.lowest_tier)
    # The cost each step would carry alone, then each page's running maximum
    # over the steps still open to it, in order.
    open_step = np.stack([(tiers <= s) & (s < lowest) for s in range(n_steps)], axis=-1)
    if options.importance_only:
        alone = np.repeat(score[..., None], n_steps, axis=-1)
    else:
        alone = score[..., None] * (err[1:] - err[:-1]) / saved_by
    cost = np.full(open_step.shape, -np.inf)
    running = np.full(tiers.shape, -np.inf)
    for s in range(n_steps):
        running = np.where(open_step[..., s], np.maximum(running, alone[..., s]), running)
        cost[..., s] = running
    layer, page, step = np.nonzero(open_step & eligible[..., None])
    move_cost, move_score, move_saved = cost[layer, page, step], score[layer, page], saved_by[step]
    # No more than ceil(target / least saving) + 1 moves can be needed: sort
    # only the cheapest that many (every move tied with the last kept).
    need = -(-int(target_bytes) // int(saved_by.min())) + 1
    if need < len(move_cost):
        cut = np.partition(move_cost, need - 1)[need - 1]
        kept = np.flatnonzero(move_cost <= cut)
    else:
        kept = np.arange(len(move_cost))
    order = kept[np.lexsort((step[kept], layer[kept], page[kept], move_score[kept],
                             move_cost[kept]))]
    total = np.cumsum(move_saved[order])
    short = len(order) == 0 or total[-1] < target_bytes
    order = order[:int(np.searchsorted(total, target_bytes)) + 1]
    taken = step[order].astype(np.int64)
    return Plan(level=level, target_bytes=int(target_bytes), short=bool(short),
                recency_floor=recency_floor, layers=layer[order].astype(np.int64),
                pages=page[order].astype(np.int64), current=taken, lower=taken + 1,
                saved=saved_by[taken], costs=move_cost[order], scores=move_score[order],
                seconds=seconds_by[taken], budget_seconds=budget_seconds, options=options)


def plan_arrays(headroom_bytes: int, thresholds: Thresholds, scores: np.ndarray,
                tiers: np.ndarray, page_bytes: dict, errors: dict, *, move_seconds: dict,
                positions: int, page_tokens: int, recency_floor: int = DEFAULT_RECENCY_FLOOR,
                margin_bytes: int = DEFAULT_MARGIN_BYTES,
                budget_seconds: float = DEFAULT_BUDGET_SECONDS,
                options: PlanOptions = DEFAULT_OPTIONS) -> Plan:
    """The plan for a headroom (reference: controller.py:252-279): none at
    GREEN, else the bytes back to YELLOW's line plus the margin."""
    level = thresholds.classify(headroom_bytes)
    if level == GREEN:
        _check_plan_inputs(np.asarray(scores, np.float64), np.asarray(tiers), positions,
                           page_tokens, recency_floor)
        return _no_moves(level, recency_floor, budget_seconds, options)
    target = max(0, thresholds.yellow_below_bytes + margin_bytes - headroom_bytes)
    return target_plan_arrays(target, level, scores, tiers, page_bytes, errors,
                              move_seconds=move_seconds, positions=positions,
                              page_tokens=page_tokens, recency_floor=recency_floor,
                              budget_seconds=budget_seconds, options=options)


def _check_pages(scores: dict, tiers: dict) -> None:
    for key, tier in tiers.items():
        if tier not in TIERS:
            raise ValueError(f"page {key} is at {tier!r}; a tier is one of {TIERS}")
        if key not in scores:
            raise ValueError(f"page {key} has no score; give NaN for one not yet scored")
        if scores[key] < 0:
            raise ValueError(f"page {key}'s score is {scores[key]}; a score is a mass, >= 0")


def _arrays_of(scores: dict, tiers: dict, extra: Collection | None = None):
    """Dict maps by (layer, page) to arrays; open pages (page < 0) dropped."""
    keys = [key for key in tiers if key[1] >= 0]
    layers = 1 + max((l for l, _ in keys), default=-1)
    pages = 1 + max((p for _, p in keys), default=-1)
    tier = np.full((layers, pages), -1, dtype=np.int8)
    score = np.full((layers, pages), np.nan)
    flag = np.zeros((layers, pages), bool)
    extra = set(extra or ())
    for key in keys:
        tier[key] = TIERS.index(tiers[key])
        score[key] = scores[key]
        flag[key] = key in extra
    return score, tier, flag


def plan(headroom_bytes: int, thresholds: Thresholds, scores: dict, tiers: dict,
         page_bytes: dict, errors: dict, *, move_seconds: dict, positions: int,
         page_tokens: int, recency_floor: int = DEFAULT_RECENCY_FLOOR,
         margin_bytes: int = DEFAULT_MARGIN_BYTES,
         budget_seconds: float = DEFAULT_BUDGET_SECONDS,
         options: PlanOptions = DEFAULT_OPTIONS) -> Plan:
    """plan_arrays on dicts keyed by (layer, page), tiers by name."""
    _check_pages(scores, tiers)
    score, tier, _ = _arrays_of(scores, tiers)
    return plan_arrays(headroom_bytes, thresholds, score, tier, page_bytes, errors,
                       move_seconds=move_seconds, positions=positions, page_tokens=page_tokens,
                       recency_floor=recency_floor, margin_bytes=margin_bytes,
                       budget_seconds=budget_seconds, options=options)


def share_target_bytes(share: float, tiers: np.ndarray, page_bytes: dict, *, positions: int,
                       page_tokens: int, recency_floor: int = DEFAULT_RECENCY_FLOOR) -> int:
    """The bytes a controlled plan reclaims for `share` of the candidates'
    FP16 bytes (reference: controller.py:281-298), in exact fractions."""
    if not 0 <= share <= 1:
        raise ValueError(f"a share is a fraction of the bytes, in [0, 1]; got {share}")
    tiers = np.asarray(tiers)
    _check_plan_inputs(None, tiers, positions, page_tokens, recency_floor)
    eligible = candidates(tiers, positions, page_tokens, recency_floor)
    held = int(place_bytes(page_bytes)[tiers[eligible]].sum())
    keep = (1 - Fraction(str(share))) * page_bytes["FP16"] * int(eligible.sum())
    return max(0, math.ceil(held - keep))


def bytes_given_back(before: np.ndarray, after: np.ndarray, page_bytes: dict) -> int:
    """Bytes the pages held in both maps gave back between them."""
    before, after = np.asarray(before), np.asarray(after)
    both = (before >= 0) & (after >= 0)
    at = place_bytes(page_bytes)
    return int(at[before[both]].sum() - at[after[both]].sum())


@dataclass(frozen=True, eq=False)
class EvictionPlan:
    target_bytes: int
    short: bool
    recency_floor: int
    options: PlanOptions
    layers: np.ndarray
    pages: np.ndarray
    freed: np.ndarray

    @property
    def reclaimed_bytes(self) -> int:
        return int(self.freed.sum())

    def __len__(self) -> int:
        return len(self.layers)


def eviction_plan(target_bytes: int, plan: Plan, tiers: np.ndarray,
                  page_bytes: dict) -> EvictionPlan:
    """The pages `plan` moves, evicted instead until `target_bytes` are
    freed (reference: controller.py:412-432): pages the plan leaves lowest
    first; among equals, the one whose last downgrade came first; each frees
    what it holds now."""
    tiers = np.asarray(tiers)
    key = plan.layers * tiers.shape[1] + plan.pages
    last_of = {}
    for i, k in enumerate(key.tolist()):
        last_of[k] = i                   # the page's last downgrade in the plan
    last = np.array(sorted(last_of.values()), dtype=np.int64)
    order = last[np.lexsort((last, -plan.lower[last]))] if len(last) else last
    layers, pages = plan.layers[order], plan.pages[order]
    freed = place_bytes(page_bytes)[tiers[layers, pages]]
    total = np.cumsum(freed)
    count = int(np.searchsorted(total, target_bytes)) + 1 if target_bytes > 0 else 0
    short = bool(target_bytes > 0 and (len(order) == 0 or total[-1] < target_bytes))
    return EvictionPlan(target_bytes, short, plan.recency_floor, plan.options, layers[:count],
                        pages[:count], freed[:count])


@dataclass(frozen=True)
class Upgrade:
    layer: int
    page: int
    current_tier: str
    target_tier: str
    bytes_taken: int
    gain: float
    score: float
    seconds: float


@dataclass(frozen=True, eq=False)
class UpgradePlan:
    """The upgrades in the order chosen, or none with `held_by` saying why."""

    level: Level
    available_bytes: int
    held_by: str
    layers: np.ndarray
    pages: np.ndarray
    current: np.ndarray
    higher: np.ndarray
    taken: np.ndarray
    gains: np.ndarray
    scores: np.ndarray
    seconds: np.ndarray
    budget_seconds: float
    options: PlanOptions = DEFAULT_OPTIONS

    def __len__(self) -> int:
        return len(self.layers)

    @property
    def target(self) -> np.ndarray:
        return self.higher

    @property
    def taken_bytes(self) -> int:
        return int(self.taken.sum())

    @functools.cached_property
    def batch_bounds(self) -> tuple[tuple[int, int], ...]:
        return batch_bounds(self.seconds, self.level, self.budget_seconds)

    def upgrade(self, i: int) -> Upgrade:
        return Upgrade(int(self.layers[i]), int(self.pages[i]), TIERS[self.current[i]],
                       TIERS[self.higher[i]], int(self.taken[i]), float(self.gains[i]),
                       float(self.scores[i]), float(self.seconds[i]))

    @functools.cached_property
    def upgrades(self) -> tuple[Upgrade, ...]:
        return tuple(self.upgrade(i) for i in range(len(self)))

    @functools.cached_property
    def batches(self) -> tuple[tuple[Upgrade, ...], ...]:
        return tuple(self.upgrades[a:b] for a, b in self.batch_bounds)


def upgrade_plan_arrays(headroom_bytes: int, thresholds: Thresholds, scores: np.ndarray,
                        tiers: np.ndarray, shadowed: np.ndarray, page_bytes: dict, errors: dict,
                        *, move_seconds: dict, last_downgrade_seconds: float | None,
                        now_seconds: float | None = None,
                        cooldown_seconds: float = DEFAULT_UPGRADE_COOLDOWN_SECONDS,
                        spike_bytes: int = DEFAULT_UPGRADE_SPIKE_BYTES,
                        budget_seconds: float = DEFAULT_BUDGET_SECONDS,
                        options: PlanOptions = DEFAULT_OPTIONS) -> UpgradePlan:
    """The upgrades for a headroom (reference: controller.py:612-690)."""
    now = time.monotonic() if now_seconds is None else now_seconds
    if last_downgrade_seconds is not None and last_downgrade_seconds > now:
        raise ValueError(f"the last downgrade, at {last_downgrade_seconds} s, is after now, "
                         f"{now} s: both times must come from one clock, time.monotonic()")
    level = thresholds.classify(headroom_bytes)
    available = headroom_bytes - thresholds.yellow_below_bytes - spike_bytes

    def held(reason: str) -> UpgradePlan:
        i, f = np.zeros(0, np.int64), np.zeros(0)
        return UpgradePlan(level, max(0, available), reason, i, i, i, i, i, f, f, f,
                           budget_seconds, options)

    if level != GREEN:
        return held(f"the level is {level.value}; upgrades are made at GREEN only")
    if last_downgrade_seconds is not None and now - last_downgrade_seconds < cooldown_seconds:
        return held(f"cooldown: {now - last_downgrade_seconds:.2f} s since the last "
                    f"downgrade, {cooldown_seconds} s needed")
    if available <= 0:
        return held(f"headroom: {headroom_bytes} bytes leave none above T_high + "
                    f"{spike_bytes} bytes")
    scores = np.asarray(scores, np.float64)
    tiers = np.asarray(tiers)
    upgradable = (tiers > 0) & np.asarray(shadowed, bool)
    score = options.weighed(np.where(np.isnan(scores), _neutral_score(scores, upgradable),
                                     scores))
    nbytes, err = _tier_tables(page_bytes, errors)
    # Step k (k = 1..3) takes a page from tier k up to k - 1.
    ks = np.arange(1, len(TIERS))
    taken_by = nbytes[:-1] - nbytes[1:]
    removed_by = err[1:] - err[:-1]
    seconds_by = np.array([move_seconds[(TIERS[k], TIERS[k - 1])] for k in ks])
    possible = ks[None, None, :] <= tiers[..., None]
    own = score[..., None] * removed_by / taken_by
    # A page's upgrades run from its tier upward; each is ordered no sooner
    # than the ones before it: the running minimum of its gains from the top.
    rank = np.full(possible.shape, np.inf)
    running = np.full(tiers.shape, np.inf)
    for j in range(len(ks) - 1, -1, -1):
        running = np.where(possible[..., j], np.minimum(running, own[..., j]), running)
        rank[..., j] = running
    layer, page, j = np.nonzero(possible & upgradable[..., None])
    move_rank, move_score, move_taken = rank[layer, page, j], score[layer, page], taken_by[j]
    need = int(available // int(taken_by.min())) + 1
    if need < len(move_rank):
        cut = -np.partition(-move_rank, need - 1)[need - 1]
        kept = np.flatnonzero(move_rank >= cut)
    else:
        kept = np.arange(len(move_rank))
    order = kept[np.lexsort((-j[kept], -layer[kept], -page[kept], -move_score[kept],
                             -move_rank[kept]))]
    order = order[:int(np.searchsorted(np.cumsum(move_taken[order]), available, side="right"))]
    leaving = (j[order] + 1).astype(np.int64)
    return UpgradePlan(level=level, available_bytes=int(available), held_by="",
                       layers=layer[order].astype(np.int64), pages=page[order].astype(np.int64),
                       current=leaving, higher=leaving - 1, taken=move_taken[order],
                       gains=own[layer, page, j][order], scores=move_score[order],
                       seconds=seconds_by[leaving - 1], budget_seconds=budget_seconds,
                       options=options)


def upgrade_plan(headroom_bytes: int, thresholds: Thresholds, scores: dict, tiers: dict,
                 page_bytes: dict, errors: dict, *, move_seconds: dict,
                 shadowed: Collection, last_downgrade_seconds: float | None,
                 now_seconds: float | None = None,
                 cooldown_seconds: float = DEFAULT_UPGRADE_COOLDOWN_SECONDS,
                 spike_bytes: int = DEFAULT_UPGRADE_SPIKE_BYTES,
                 budget_seconds: float = DEFAULT_BUDGET_SECONDS,
                 options: PlanOptions = DEFAULT_OPTIONS) -> UpgradePlan:
    """upgrade_plan_arrays on dicts keyed by (layer, page), tiers by name."""
    _check_pages(scores, tiers)
    score, tier, shadow = _arrays_of(scores, tiers, shadowed)
    return upgrade_plan_arrays(headroom_bytes, thresholds, score, tier, shadow, page_bytes,
                               errors, move_seconds=move_seconds,
                               last_downgrade_seconds=last_downgrade_seconds,
                               now_seconds=now_seconds, cooldown_seconds=cooldown_seconds,
                               spike_bytes=spike_bytes, budget_seconds=budget_seconds,
                               options=options)
