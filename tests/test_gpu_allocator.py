"""The VMM page allocator on the device against the oracle's slot model:
slot order, page contents, mapped granules, rollback. GPU parity tests."""

import numpy as np
import pytest

from conftest import announce
from oracle import slots

pytestmark = pytest.mark.gpu


def mi():
    from microinfer import _microinfer
    return _microinfer


def test_random_operations_match_the_slot_model():
    m = mi()
    granule = m.granule_bytes()
    announce("granule", granule)
    assert granule > 0
    # Page sizes as fractions of the granule, as the reference's tests use
    # (tests/test_paged_kv_cache.py:1-87), and capacity for several granules.
    page_bytes = [granule // 3 // 16 * 16, granule // 5 // 16 * 16, granule // 7 // 16 * 16, 4096]
    cap = [40, 40, 40, 40]
    alloc = m.PagedKVCache(page_bytes, cap)
    model = slots.Slots(page_bytes, cap, granule)
    rng = np.random.default_rng(0)
    held = {}
    for step in range(300):
        op = rng.integers(0, 7)
        keys = list(held)
        if op == 6:
            # Releases drained: a run the tail cut is settled (replaced by a
            # shorter one holding the same bytes), which the checks below read.
            alloc.drain_releases()
            continue
        if op <= 2 or not keys:
            key = (int(rng.integers(0, 3)), int(rng.integers(-20, 30)))
            tier = int(rng.integers(0, 4))
            if key in held or len(model.slots[tier]) == cap[tier]:
                continue
            data = rng.integers(0, 256, page_bytes[tier], dtype=np.uint8)
            alloc.allocate(key[0], key[1], tier)
            alloc.write(key[0], key[1], data)
            model.allocate(key, tier, data=data)
            held[key] = data
        elif op == 3:
            key = keys[rng.integers(0, len(keys))]
            alloc.free(*key)
            model.free(key)
            del held[key]
        elif op == 4:
            n = int(rng.integers(1, min(8, len(keys)) + 1))
            chosen = [keys[i] for i in rng.choice(len(keys), n, replace=False)]
            alloc.free_pages(chosen)
            model.free_pages(chosen)
            for key in chosen:
                del held[key]
        else:
            n = int(rng.integers(1, min(4, len(keys)) + 1))
            chosen = [keys[i] for i in rng.choice(len(keys), n, replace=False)]
            pairs = []
            for i, key in enumerate(chosen):
                stage = (key[0], -100 - i)
                tier = int(rng.integers(0, 4))
                if len(model.slots[tier]) == cap[tier]:
                    continue
                data = rng.integers(0, 256, page_bytes[tier], dtype=np.uint8)
                alloc.allocate(stage[0], stage[1], tier)
                alloc.write(stage[0], stage[1], data)
                model.allocate(stage, tier, data=data)
                pairs.append((key, stage))
                held[key] = data
            if pairs:
                alloc.replace_pages(pairs)
                model.replace_pages(pairs)
        if step % 25 == 0 or step == 299:
            announce("allocator step", step)
            for t in range(4):
                assert alloc.pages(t) == model.slots[t], (step, t)
                assert alloc.mapped_bytes(t) == model.mapped_bytes(t), (step, t)
            for key, data in held.items():
                np.testing.assert_array_equal(alloc.read(*key), data)


def test_a_failed_granule_rolls_back_and_full_is_refused():
    m = mi()
    granule = m.granule_bytes()
    alloc = m.PagedKVCache([granule, granule, granule, granule], [3, 0, 0, 1])
    alloc.allocate(0, 0, 0)
    mapped = alloc.mapped_bytes(0)
    m.fail_next_granules(1)
    with pytest.raises(m.OutOfMemory):
        alloc.allocate(0, 1, 0)
    m.fail_next_granules(0)
    assert (0, 1) not in alloc and alloc.mapped_bytes(0) == mapped
    alloc.allocate(0, 1, 0)
    alloc.allocate(0, 2, 0)
    with pytest.raises(ValueError, match="full"):
        alloc.allocate(0, 3, 0)
    with pytest.raises(KeyError):
        alloc.free(5, 5)
    with pytest.raises(ValueError, match="already"):
        alloc.allocate(0, 1, 0)


def test_spare_granules_are_kept_mapped_beyond_the_tail():
    m = mi()
    granule = m.granule_bytes()
    alloc = m.PagedKVCache([granule // 2] * 4, [16, 16, 16, 16])
    alloc.allocate(0, 0, 2)
    assert alloc.mapped_bytes(2) == granule
    alloc.keep_spare_granules(2, 2)
    assert alloc.spare_granules(2) == 2 and alloc.mapped_bytes(2) == 3 * granule
    for i in range(1, 5):
        alloc.allocate(0, i, 2)
    assert alloc.mapped_bytes(2) == 5 * granule
    for i in range(5):
        alloc.free(0, i)
    assert alloc.mapped_bytes(2) == 2 * granule


def test_given_up_granules_are_mapped_again_once_released():
    """Granules a range gives up go back to the driver on the cache's release
    thread; mapping the same addresses again waits for them, and the pages
    written there read back whole."""
    m = mi()
    granule = m.granule_bytes()
    page = granule // 4
    alloc = m.PagedKVCache([page] * 4, [64, 64, 64, 64])
    rng = np.random.default_rng(7)
    for round_ in range(3):
        data = {}
        for i in range(32):
            alloc.allocate(round_, i, 1)
            data[i] = rng.integers(0, 256, page, dtype=np.uint8)
            alloc.write(round_, i, data[i])
        assert alloc.mapped_bytes(1) == 8 * granule
        for i in range(32):
            assert np.array_equal(alloc.read(round_, i), data[i])
        alloc.free_pages([(round_, i) for i in range(32)])
        assert alloc.mapped_bytes(1) == 0
    alloc.drain_releases()
    assert alloc.mapped_bytes(1) == 0


def test_footprint_at_32k_is_the_reference_measurement():
    """experiments/logs/benchmark.jsonl:48-51: a 28-layer Qwen2.5-1.5B cache
    reserved for 32K positions maps exactly the reference's measured bytes at
    every tier (whole 2 MiB granules per tier range, two FP16 open pages a
    layer once the cache seals)."""
    import json
    from conftest import GOLDEN
    from oracle import quant
    m = mi()
    d = m.device
    f = json.loads((GOLDEN / "known_answers.json").read_text())["footprint_32k_1_5b"]
    assert m.granule_bytes() == f["granule"]
    sizes = [quant.page_bytes(t, 2, 128) for t in range(4)]
    for tier, name in enumerate(("FP16", "INT8", "INT4", "INT2")):
        announce("footprint", name)
        cap = [0, 0, 0, 0]
        cap[tier] = f["layers"] * 1024
        cap[0] += f["layers"] * 2
        alloc = m.PagedKVCache(sizes, cap)
        cache = d.KVPages(alloc, f["layers"], 32, 2, 128, tier)
        cache.reserve(f["context"])
        assert sum(alloc.mapped_bytes(t) for t in range(4)) == f["bytes"][name]
        del cache, alloc
