"""The host callers on either side of the decode path: the cache a model's
layers attend through, with the importance scores folded on a cadence
(reference: src/microinfer/model.py:273-286 PagedCache.attend), and the
application of a precision plan in batches of page moves (reference:
src/microinfer/engine.py:322-371 next_batch / move_seconds, :1750-1802
Engine._apply).
"""

from __future__ import annotations

import math
import time
from dataclasses import dataclass, field

import numpy as np

from . import _microinfer as mi
from . import controller
from .monitor import RED

#: Pinning a page's FP16 shadow: page-locking host memory, ~8 µs for a
#: 1.5B page, taken high (reference: engine.py:292-295).
SHADOW_PIN_SECONDS = 2e-5
#: A batch's fixed part (synchronisations, the address tables), taken high.
BATCH_FIXED_SECONDS = 5e-4
#: The room a paced step keeps past its batches' estimate.
MOVE_MARGIN_SECONDS = 2e-3
#: The least a move is taken to cost when a budget sizes a batch.
MIN_MOVE_SECONDS = 1e-6
#: Moves a batch needs before its per-move time is measured past its fixed part.
PACED_BATCH_MOVES = 32
FP16 = controller.TIERS.index("FP16")


@dataclass(frozen=True)
class MoveBatch:
    """The moves of one batch ((layer, page, Tier) triples, each page once at
    the tier its moves end at), the plan index after the last move taken,
    the moves skipped, and the bytes the batch's new pages take."""

    moves: list
    end: int
    skipped: int
    bytes: int


def next_batch(plan, first: int, held: np.ndarray, shadowed: np.ndarray, page_bytes: list,
               bytes_cap: float, seconds_cap: float, move_seconds: float) -> MoveBatch:
    """The next batch of `plan` from its move `first` (reference:
    engine.py:322-357). A page moved in several steps is moved once, straight
    to where its steps end (the quantised tier is always quantised from
    FP16). A move whose page is not where the plan expects (after the
    batch's earlier moves, else in `held`) is skipped. Moves are taken while
    the new pages' bytes fit `bytes_cap` and the time fits `seconds_cap`:
    `move_seconds` a page, plus SHADOW_PIN_SECONDS for a page leaving FP16
    without a shadow yet; at least one move is taken. A page whose steps end
    where it is moves nothing."""
    ends: dict = {}
    skipped = 0
    new_bytes = 0
    seconds = 0.0
    k = first
    while k < len(plan):
        key = (int(plan.layers[k]), int(plan.pages[k]))
        at = ends[key] if key in ends else int(held[key])
        if at != int(plan.current[k]):
            skipped += 1
            k += 1
            continue
        target = int(plan.target[k])
        grows = page_bytes[target] - (page_bytes[ends[key]] if key in ends else 0)
        takes = 0.0
        if key not in ends:
            takes = move_seconds
            if at == FP16 and not shadowed[key]:
                takes += SHADOW_PIN_SECONDS
        if ends and (new_bytes + grows > bytes_cap or seconds + takes > seconds_cap):
            break
        ends[key] = target
        new_bytes += grows
        seconds += takes
        k += 1
    moves = [(layer, page, mi.Tier(t)) for (layer, page), t in ends.items()
             if t != int(held[layer, page])]
    return MoveBatch(moves, k, skipped, new_bytes)


def move_seconds(batch: dict) -> float:
    """A move's time in a finished batch, for pacing the next: past the fixed
    part and the shadow pinning when the batch is large enough to tell them
    apart, else its whole time a move."""
    if batch["moves"] < PACED_BATCH_MOVES:
        return batch["seconds"] / max(batch["moves"], 1)
    rest = batch["seconds"] - BATCH_FIXED_SECONDS - batch["shadows_taken"] * SHADOW_PIN_SECONDS
    return max(rest, 0.0) / batch["moves"]


@dataclass
class Applied:
    """What apply_plan did: the plan index reached, the moves skipped, and
    each batch's (start, end, seconds)."""

    cursor: int
    skipped: int = 0
    batches: list = field(default_factory=list)
    stopped: str = ""


def apply_plan(pages, plan, page_bytes: list, *, first: int = 0, budget_seconds: float | None = None,
               started: float | None = None, batch_margin_bytes: int | None = None,
               recent_moves: list | None = None) -> Applied:
    """Applies `plan` from move `first` in batches on the device (reference:
    engine.py:1750-1802). A RED plan (or no budget) goes at once; any other
    takes no more than `budget_seconds` from `started`, each batch sized to
    what is left of it. A batch also fits the device's free memory less a
    margin, its new pages being allocated before any old one is freed; one
    that cannot allocate is tried again at half its bytes, and a single move
    that cannot stops the application. `recent_moves` (seconds a move, of
    earlier batches) paces the next; it is appended to."""
    started = time.perf_counter() if started is None else started
    recent = recent_moves if recent_moves is not None else []
    margin = (2 * len(controller.TIERS) * mi.granule_bytes() if batch_margin_bytes is None
              else batch_margin_bytes)
    paced = plan.level != RED and budget_seconds is not None
    done = Applied(cursor=first)
    i, bytes_cap = first, None
    while i < len(plan):
        per = max(2 * max(recent, default=0.0), MIN_MOVE_SECONDS)
        seconds = math.inf
        if paced:
            seconds = (budget_seconds - (time.perf_counter() - started) - BATCH_FIXED_SECONDS
                       - MOVE_MARGIN_SECONDS)
            if seconds < per and i > first:
                break
        free = mi.device_memory_info()["free"] - margin
        batch = next_batch(plan, i, pages.page_tiers(), pages.shadowed(), page_bytes,
                           free if bytes_cap is None else min(free, bytes_cap), seconds, per)
        t0 = time.perf_counter()
        if batch.moves:
            try:
                pages.move_pages(batch.moves)
            except mi.OutOfMemory as exc:
                if len(batch.moves) == 1:
                    done.stopped = f"stopped: {exc}"
                    break
                bytes_cap = batch.bytes // 2
                continue
            last = pages.last_batch
            if last is not None:
                recent.append(move_seconds(last))
        done.batches.append((i, batch.end, time.perf_counter() - t0))
        done.skipped += batch.skipped
        i = batch.end
    done.cursor = i
    return done


class PagedCache:
    """The cache a model's layers attend through (reference: model.py
    PagedCache): the KV pages, and, if kept, the importance scores, into
    which a step's per-page attention mass is folded when the step is a
    single query and the positions it attends are a multiple of
    `score_every` (reference: model.py:273-286; engine.py's R = 4)."""

    def __init__(self, pages, heads: int, kv_heads: int, head_dim: int,
                 scores=None, score_every: int = 4, rope=None):
        if score_every <= 0:
            raise ValueError(f"scores are folded every R >= 1 positions; got {score_every}")
        self.pages = pages
        self.heads, self.kv_heads, self.head_dim = heads, kv_heads, head_dim
        self.scores, self.score_every, self.rope = scores, score_every, rope
        self._mass = None
        self._mass_pages = 0

    def _mass_for(self, pages: int):
        if self._mass is None or self._mass_pages < pages:
            self._mass_pages = max(pages, 2 * self._mass_pages)
            self._mass = mi.device.empty_f32(self.heads * self._mass_pages)
        return self._mass

    def attend(self, layer: int, q, k_bias, out, seq_q: int, seq_k: int, keys=None, values=None,
               partials=None) -> None:
        scored = self.scores is not None and seq_q == 1 and seq_k % self.score_every == 0
        pages = -(-seq_k // self.pages.page_tokens)
        self.pages.attention(layer, q, k_bias, self.rope, out, seq_q, seq_k, self.heads,
                             self.kv_heads, self.head_dim, keys, values,
                             self._mass_for(pages) if scored else None, partials,
                             scores=self.scores if scored else None)
