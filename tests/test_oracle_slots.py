"""The oracle's allocator model, pinned by brute force against a slot-free
dictionary model and by its invariants. CPU only."""

import numpy as np

from oracle import slots


def test_contents_survive_any_sequence_like_a_plain_dictionary():
    rng = np.random.default_rng(0)
    for trial in range(30):
        s = slots.Slots([100, 60, 40, 30], [50, 50, 50, 50], 256)
        plain = {}
        serial = 0
        for _ in range(200):
            op = rng.integers(0, 5)
            keys = list(plain)
            if op <= 1 or not keys:
                key = (int(rng.integers(0, 3)), int(rng.integers(0, 30)))
                if key in plain:
                    continue
                tier = int(rng.integers(0, 4))
                serial += 1
                s.allocate(key, tier, data=serial)
                plain[key] = (tier, serial)
            elif op == 2:
                key = keys[rng.integers(0, len(keys))]
                s.free(key)
                del plain[key]
            elif op == 3:
                n = int(rng.integers(1, min(6, len(keys)) + 1))
                chosen = [keys[i] for i in rng.choice(len(keys), n, replace=False)]
                s.free_pages(chosen)
                for key in chosen:
                    del plain[key]
            else:
                # replace: stage a new page, then rename it over an old one
                key = keys[rng.integers(0, len(keys))]
                stage = (key[0], -16 - int(rng.integers(0, 4)))
                if stage in plain:
                    continue
                tier = int(rng.integers(0, 4))
                serial += 1
                s.allocate(stage, tier, data=serial)
                s.replace_pages([(key, stage)])
                plain[key] = (tier, serial)
            s.check_packed()
            for key, (tier, data) in plain.items():
                assert s.locate(key)[0] == tier
                assert s.read(key) == data
            for t in range(4):
                need = -(-len(s.slots[t]) * s.page_bytes[t] // 256)
                assert s.granules[t] == need


def test_free_moves_the_tail_into_the_hole():
    s = slots.Slots([10] * 4, [8] * 4, 16)
    for i in range(5):
        s.allocate((0, i), 0, data=i)
    s.free((0, 1))
    assert s.slots[0] == [(0, 0), (0, 4), (0, 2), (0, 3)]
    s.free_pages([(0, 0), (0, 3)])
    # kept = 2: slot 0 is a hole, slot 2 ((0, 2)) a mover; (0, 3) in slot 3 goes.
    assert s.slots[0] == [(0, 2), (0, 4)]


def test_spare_granules_are_kept_and_capped_by_the_reservation():
    s = slots.Slots([100, 10, 10, 10], [10, 1, 1, 1], 256)
    s.allocate((0, 0), 0)
    assert s.granules[0] == 1
    s.keep_spare_granules(0, 2)
    assert s.granules[0] == 3
    s.keep_spare_granules(0, 10)
    assert s.granules[0] == s.reserved[0] // 256
    s.free((0, 0))
    assert s.granules[0] == s.reserved[0] // 256
