"""The tail-swap page allocator, as a pure-Python model.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Follows the reference's src/core_kernels/paged_kv_cache.cu:
  - allocate:       :145-185 (page at the tail of its tier; granules mapped
                    as the tail crosses into them; generation +1)
  - free:           :202-225 (the tier's tail page moves into the freed slot)
  - free_pages:     :227-359 (per tier: the first `kept` slots stay; each freed
                    slot below `kept` is a hole, each kept slot at or above it
                    a mover; movers fill holes in ascending order)
  - replace(_pages):  :361-416 (free the old pages, then rename each staged
                    page to its key, keeping its tier, slot and bytes)
  - fit_granules:   :437-470 (ceil(slots * page_bytes / granule) granules,
                    plus spares up to the reserved range)
  - reserve:        :100 (capacity * page_bytes rounded up to granules)

Contents are modelled too: each slot holds the bytes last written to its
page, so a model replay says what read() must return after any sequence of
operations.

PINNED by (tests/test_oracle_slots.py): brute force on tiny inputs against a
dictionary model with no slots at all (a page's bytes survive any sequence of
frees and replaces); the invariants that slots are packed with no holes and
that the table and the slot lists agree; the granule count against the closed
form; free_pages against the same frees made one at a time as far as the set
of survivors and their bytes go (slot order differs by design); the reference
footprint totals of experiments/logs/benchmark.jsonl:48-51.
"""

from __future__ import annotations


def ceil_div(a: int, b: int) -> int:
    return -(-a // b)


class Slots:
    def __init__(self, page_bytes, capacity_pages, granule: int):
        self.page_bytes = list(page_bytes)
        self.capacity = list(capacity_pages)
        self.granule = granule
        self.reserved = [ceil_div(p * c, granule) * granule
                         for p, c in zip(self.page_bytes, self.capacity)]
        self.slots = [[] for _ in page_bytes]
        self.data = [[] for _ in page_bytes]
        self.table = {}
        self.granules = [0] * len(page_bytes)
        self.spares = [0] * len(page_bytes)
        self.generation = 0

    # -- granules ------------------------------------------------------------
    def _fit(self, t: int, map_spares: bool) -> None:
        needed = ceil_div(len(self.slots[t]) * self.page_bytes[t], self.granule)
        kept = min(needed + self.spares[t], self.reserved[t] // self.granule)
        if self.granules[t] < needed:
            self.granules[t] = needed
        if map_spares and self.granules[t] < kept:
            self.granules[t] = kept
        if self.granules[t] > kept:
            self.granules[t] = kept

    def mapped_bytes(self, t: int) -> int:
        return self.granules[t] * self.granule

    def keep_spare_granules(self, t: int, n: int) -> None:
        self.spares[t] = n
        self._fit(t, True)

    # -- pages ---------------------------------------------------------------
    def locate(self, key):
        if key not in self.table:
            raise KeyError(key)
        return self.table[key]

    def allocate(self, key, t: int, data=None) -> None:
        if key in self.table:
            raise ValueError(f"{key} is already allocated")
        if len(self.slots[t]) == self.capacity[t]:
            raise ValueError(f"tier {t} is full")
        self.slots[t].append(key)
        self.data[t].append(data)
        self._fit(t, True)
        self.table[key] = (t, len(self.slots[t]) - 1)
        self.generation += 1

    def write(self, key, data) -> None:
        t, s = self.locate(key)
        self.data[t][s] = data

    def read(self, key):
        t, s = self.locate(key)
        return self.data[t][s]

    def free(self, key) -> None:
        t, slot = self.locate(key)
        tail = len(self.slots[t]) - 1
        if slot != tail:
            moved = self.slots[t][tail]
            self.slots[t][slot] = moved
            self.data[t][slot] = self.data[t][tail]
            self.table[moved] = (t, slot)
        self.slots[t].pop()
        self.data[t].pop()
        del self.table[key]
        self.generation += 1
        self._fit(t, False)

    def free_pages(self, keys) -> None:
        freeing = set()
        for key in keys:
            self.locate(key)
            if key in freeing:
                raise ValueError(f"{key} is named twice in one free")
            freeing.add(key)
        if not keys:
            return
        touched = []
        for t in range(len(self.slots)):
            going = [k in freeing for k in self.slots[t]]
            if not any(going):
                continue
            touched.append(t)
            kept = len(going) - sum(going)
            holes = [s for s in range(len(going)) if s < kept and going[s]]
            movers = [s for s in range(len(going)) if s >= kept and not going[s]]
            for hole, mover in zip(holes, movers):
                moved = self.slots[t][mover]
                self.slots[t][hole] = moved
                self.data[t][hole] = self.data[t][mover]
                self.table[moved] = (t, hole)
            del self.slots[t][kept:]
            del self.data[t][kept:]
        for key in keys:
            del self.table[key]
        self.generation += 1
        for t in touched:
            self._fit(t, False)

    def replace_pages(self, pairs) -> None:
        staged = set()
        for key, stage in pairs:
            if key == stage:
                raise ValueError("a page cannot replace itself")
            self.locate(stage)
            if stage in staged:
                raise ValueError(f"{stage} is named twice in one replace")
            staged.add(stage)
        for key, _ in pairs:
            if key in staged:
                raise ValueError(f"{key} is both replaced and staged")
        self.free_pages([k for k, _ in pairs])
        for key, stage in pairs:
            t, s = self.table.pop(stage)
            self.table[key] = (t, s)
            self.slots[t][s] = key
        self.generation += 1

    def replace(self, key, stage) -> None:
        if key == stage:
            raise ValueError("a page cannot replace itself")
        self.locate(stage)
        self.free(key)
        t, s = self.table.pop(stage)
        self.table[key] = (t, s)
        self.slots[t][s] = key
        self.generation += 1

    def check_packed(self) -> None:
        """Slots are packed from 0 with no holes, and the table agrees."""
        count = 0
        for t, keys in enumerate(self.slots):
            for s, key in enumerate(keys):
                assert self.table[key] == (t, s), (key, t, s)
                count += 1
            needed = ceil_div(len(keys) * self.page_bytes[t], self.granule)
            assert self.granules[t] >= needed
        assert count == len(self.table)


def cache_ranges(layers: int, context: int, page_tokens: int, page_bytes, tier_map_rows=None,
                 tier: int = 0, seals: bool = True, open_pages: int = 2):
    """src/microinfer/engine.py:133-160 (paged_cache_ranges): the bytes each
    tier's range needs for `context` positions."""
    ranges = [0] * 4
    if not seals:
        ranges[0] = layers * ceil_div(context, page_tokens) * page_bytes[0]
        return ranges
    rows = tier_map_rows or [[] for _ in range(layers)]
    for row in rows:
        for i in range(context // page_tokens):
            born = row[i] if i < len(row) else tier
            ranges[born] += page_bytes[born]
    if context > 0:
        ranges[0] += layers * open_pages * page_bytes[0]
    return ranges


def cache_bytes(ranges, granule: int) -> int:
    """engine.py:163-174 (paged_cache_bytes): each range in whole granules."""
    return sum(ceil_div(n, granule) * granule for n in ranges)
