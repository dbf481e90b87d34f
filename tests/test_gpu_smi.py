"""The amdsmi reader (the reference's NVML reader, nvml.py, on AMD's SMI) and
what it is for: granules the allocator gives back show in the device's free
memory as amdsmi reports it (the ADR-0007 contract,
tests/test_paged_kv_cache.py:146-192 of the reference), and shadows pinned
ahead are what a batch of first downgrades uses.

GPU tests: they read the device HIP runs on, found by its PCI bus id."""

import numpy as np
import pytest

from conftest import announce

pytestmark = pytest.mark.gpu


def mi():
    from microinfer import _microinfer
    return _microinfer


def smi():
    from microinfer import smi as reader
    return reader


def test_the_reader_names_the_device_and_its_memory():
    m, s = mi(), smi()
    announce("smi memory")
    mem = s.memory()
    free, total = m.device_memory_info()["free"], m.device_memory_info()["total"]
    assert 0 < mem.free <= mem.total and mem.used == mem.total - mem.free
    # HIP and amdsmi count the same VRAM: totals within 2%.
    assert abs(mem.total - total) <= 0.02 * total, (mem.total, total)
    assert abs(mem.free - free) <= 0.05 * total, (mem.free, free)
    assert s.device_name()
    announce("smi memory source", s.memory_source(), mem)
    assert s.memory_source() in ("amdsmi", "hip")
    assert s.headroom() == pytest.approx(mem.free, rel=0.05)
    split = s.split()
    assert split.others_bytes is None or split.others_bytes >= 0


def test_granules_given_back_show_in_amdsmi_free_memory():
    """Pages a granule / 64 each; 64 granules' worth held, then the lowest
    pages freed one at a time (each a tail swap: memory comes back only
    because the tail retracts). Once the releases have drained, amdsmi's free
    memory has risen by at least the granules emptied; allocating the pages
    again takes it back. The median of three rounds, against other work on
    the device. And 65 pages reach a second granule; freeing any one empties
    it, freeing another empties nothing."""
    m, s = mi(), smi()
    g = m.granule_bytes()
    page = g // 64
    emptied = 48
    held = (emptied + 3) * 64
    alloc = m.PagedKVCache([page] * 4, [held] * 4)
    for i in range(held):
        alloc.allocate(0, i, m.Tier.FP16)
    gains = []
    for round_ in range(3):
        announce("granule release round", round_)
        alloc.drain_releases()
        m.synchronize()
        before = s.memory().free
        for i in range(emptied * 64):
            alloc.free(0, i)
        alloc.drain_releases()
        m.synchronize()
        after = s.memory().free
        gains.append(after - before)
        assert alloc.mapped_bytes(m.Tier.FP16) == 3 * g
        for i in range(emptied * 64):
            alloc.allocate(0, i, m.Tier.FP16)
    gained = sorted(gains)[1]
    assert gained >= emptied * g, f"freeing {emptied} granules returned {gained / 2**20:.1f} MiB"

    small = m.PagedKVCache([g // 64] * 4, [128] * 4)
    for i in range(65):
        small.allocate(0, i, m.Tier.FP16)
    assert small.mapped_bytes(m.Tier.FP16) == 2 * g
    small.free(0, 0)
    assert small.mapped_bytes(m.Tier.FP16) == g
    small.free(0, 1)
    assert small.mapped_bytes(m.Tier.FP16) == g


def test_shadows_pinned_ahead_are_the_ones_a_batch_uses():
    """pin_shadows(n) pins room for n shadows at once; a batch of n first
    downgrades afterwards pins nothing more (shadow_bytes unchanged) and its
    shadows hold each page's FP16 bytes."""
    from oracle import quant
    m = mi()
    d = m.device
    P, kv, hd, layers = 32, 2, 128, 2
    sizes = [quant.page_bytes(t, kv, hd, P) for t in range(4)]
    alloc = m.PagedKVCache(sizes, [256] * 4)
    cache = d.KVPages(alloc, layers, P, kv, hd, m.Tier.FP16, d.Halves.Both, [], True)
    rng = np.random.default_rng(4)
    seq = P * 40
    k = rng.standard_normal((seq, kv, hd)).astype(np.float16).astype(np.float32)
    v = rng.standard_normal((seq, kv, hd)).astype(np.float16).astype(np.float32)
    cache.reserve(seq)
    for layer in range(layers):
        cache.store(layer, m.upload_fp16(k), m.upload_fp16(v), 0, seq)
    assert cache.shadow_count == 0 and cache.shadow_bytes == 0
    moves = [(layer, p, (2, 3)[p % 2]) for layer in range(layers) for p in range(0, 36, 3)]
    cache.pin_shadows(len(moves))
    pinned = cache.shadow_bytes
    assert pinned >= len(moves) * sizes[0]
    announce("pinned-ahead batch", len(moves))
    cache.move_pages(moves)
    assert cache.shadow_bytes == pinned
    assert cache.shadow_count == len(moves)
    for layer, p, t in moves:
        kp = k[p * P:(p + 1) * P].astype(np.float16)
        vp = v[p * P:(p + 1) * P].astype(np.float16)
        np.testing.assert_array_equal(cache.shadow(layer, p), quant.fp16_page(kp, vp))
        np.testing.assert_array_equal(alloc.read(layer, p), quant.quantise_page(kp, vp, t, P))
