"""The cache manager on the device: sealing, causal mixed-tier attention with
per-page mass and the fused EWMA, downgrades, upgrades and batched moves,
against the oracle.

GPU parity tests. Bytes, tiers and shadows are compared to the bit; attention
outputs and masses to the 1e-3 bar; the fused scores to the bit against the
oracle's fold of the kernel's own masses."""

import numpy as np
import pytest

from conftest import (announce, assert_attention_close, assert_mass_close, each, fp16_exact)
from oracle import attention as att
from oracle import ewma, quant

pytestmark = pytest.mark.gpu

LAYERS = 2


def mi():
    from microinfer import _microinfer
    return _microinfer


def page_sizes(P, kv, hd):
    return [quant.page_bytes(t, kv, hd, P) for t in range(4)]


def pages_for(P, kv, hd, tier=0, tier_map=None, always_seal=False, capacity=4096):
    m = mi()
    cap = [capacity] * 4
    cap[0] += LAYERS * 2 + 8
    alloc = m.PagedKVCache(page_sizes(P, kv, hd), cap)
    cache = m.device.KVPages(alloc, LAYERS, P, kv, hd, tier, m.device.Halves.Both,
                             tier_map or [], always_seal)
    return alloc, cache


def put(x):
    return mi().upload_fp16(np.ascontiguousarray(x, np.float32).reshape(-1))


def normal(rng, *shape):
    return fp16_exact(rng.standard_normal(shape))


def store_in_runs(cache, layer, k, v, runs):
    start = 0
    for n in runs:
        cache.reserve(start + n)
        cache.store(layer, put(k[start:start + n]), put(v[start:start + n]), start, n)
        start += n
    return start - runs[-1]


def sealed_pages(alloc, layer, n):
    pages, tiers = [], []
    for i in range(n):
        pages.append(alloc.read(layer, i))
        tiers.append(int(alloc.locate(layer, i)[0]))
    return pages, tiers


def test_sealed_pages_are_quantise_page_s_bytes_however_rows_arrive():
    """A full page holds, byte for byte, the oracle's quantise_page of its
    rows at its birth tier, whether its positions came in one store, one at a
    time, or in runs that begin and end mid-page (P = 16, 32, 48)."""
    def check(P, tier, runs_name):
        kv, hd = 2, 64
        rng = np.random.default_rng(P + tier)
        seq = 3 * P + 5
        k, v = normal(rng, seq, kv, hd), normal(rng, seq, kv, hd)
        runs = {"one": [seq], "single": [1] * seq, "ragged": [P // 2 + 1, P + 3, seq - (3 * P // 2 + 4)]}[runs_name]
        announce("seal", P, tier, runs_name)
        alloc, cache = pages_for(P, kv, hd, tier)
        store_in_runs(cache, 1, k, v, runs)
        for i in range(seq // P):
            kp = k[i * P:(i + 1) * P].astype(np.float16)
            vp = v[i * P:(i + 1) * P].astype(np.float16)
            want = quant.fp16_page(kp, vp) if tier == 0 else quant.quantise_page(kp, vp, tier, P)
            np.testing.assert_array_equal(alloc.read(1, i), want)

    each([(P, t, r) for P in (16, 32, 48) for t in (1, 2, 3)
          for r in ("one", "single", "ragged")], check)
    # An FP16 cache that seals (always_seal) copies its rows.
    for P in (16, 32):
        kv, hd = 2, 64
        rng = np.random.default_rng(3)
        k, v = normal(rng, 2 * P, kv, hd), normal(rng, 2 * P, kv, hd)
        alloc, cache = pages_for(P, kv, hd, 0, always_seal=True)
        store_in_runs(cache, 0, k, v, [P - 3, P + 3])
        for i in range(2):
            want = quant.fp16_page(k[i * P:(i + 1) * P].astype(np.float16),
                                   v[i * P:(i + 1) * P].astype(np.float16))
            np.testing.assert_array_equal(alloc.read(0, i), want)


def decode_case(P, kv, hd, heads, tier_map, seq, seed, bias=False, theta=1e6):
    m = mi()
    rng = np.random.default_rng(seed)
    k, v = normal(rng, seq, kv, hd), normal(rng, seq, kv, hd)
    k[:, :, rng.choice(hd, 2, replace=False)] *= 10
    k = fp16_exact(k)
    alloc, cache = pages_for(P, kv, hd, 0, tier_map=tier_map, always_seal=True)
    store_in_runs(cache, 0, k, v, [seq - 1, 1])
    q = normal(rng, 1, heads, hd)
    b = fp16_exact(3 * rng.standard_normal((kv, hd))) if bias else None
    return m, alloc, cache, k, v, q, b


def oracle_decode(alloc, P, kv, hd, k, v, q, bias=None, theta=1e6):
    seq = len(k)
    own = (seq - 1) // P
    pages, tiers = sealed_pages(alloc, 0, own)
    return att.causal_decode(q, pages, tiers, k[own * P:], v[own * P:], kv, hd, P,
                             k_bias=bias, theta=theta, with_bound=True)


def run_decode(m, cache, k, v, q, heads, kv, hd, bias=None, theta=1e6, mass=True, partials=True,
               scores=None):
    d = m.device
    seq = len(k)
    P = cache.page_tokens
    pages = -(-seq // P)
    rope = None
    if bias is not None:
        rope = d.RopeTable(hd, theta)
        rope.cover(seq)
    out = d.empty(heads * hd)
    mbuf = d.empty_f32(heads * pages) if mass else None
    part = d.empty_f32(d.attention_partials(hd)) if partials else None
    cache.attention(0, put(q), put(bias) if bias is not None else None, rope, out, 1, seq, heads,
                    kv, hd, put(k[-1:]), put(v[-1:]), mbuf, part, scores=scores)
    got = out.to_numpy().reshape(1, heads, hd)
    return got, (mbuf.to_numpy().reshape(heads, pages) if mass else None)


def test_decode_over_mixed_tiers_is_the_oracle():
    """One decode query over a cache whose pages were born at every tier,
    own page FP16 from the open page and the row it brought: output and
    per-page masses against the float64 causal view."""
    def check(P, shape, seq, bias):
        heads, kv, hd = shape
        cycle = [1, 0, 3, 2]
        tmap = [[cycle[i % 4] for i in range(seq // P + 1)] for _ in range(LAYERS)]
        announce("decode mixed", P, shape, seq, bias)
        m, alloc, cache, k, v, q, b = decode_case(P, kv, hd, heads, tmap, seq, seed=seq, bias=bias)
        for partials in (True, False):
            got, mass = run_decode(m, cache, k, v, q, heads, kv, hd, b, partials=partials)
            want, want_mass, bound = oracle_decode(alloc, P, kv, hd, k, v, q, b)
            assert_attention_close(got, want, f"P={P} {shape} seq={seq} partials={partials}",
                                   bound)
            assert_mass_close(mass, want_mass, "mass")
            np.testing.assert_allclose(mass.sum(1), 1.0, atol=1e-5)

    cases = [(32, (12, 2, 128), 32 * 9 + 7, False), (32, (14, 2, 64), 32 * 40 + 1, True),
             (32, (14, 2, 64), 32 * 40 + 1, False), (32, (12, 2, 128), 32 * 2 + 1, False),
             (16, (14, 2, 64), 16 * 20 + 5, False), (48, (12, 2, 128), 48 * 7 + 20, False),
             (32, (32, 8, 64), 32 * 33, False), (32, (12, 2, 128), 32 * 300 + 31, False),
             (32, (12, 2, 128), 32 * 9 + 7, True), (32, (12, 2, 128), 32 * 300 + 31, True),
             (32, (32, 8, 64), 32 * 33, True), (32, (14, 2, 64), 20, False),
             (32, (14, 2, 64), 20, True),
             (32, (12, 2, 128), 32 * 2 + 1, True), (32, (12, 2, 128), 32, True)]
    each(cases, check)


def test_decode_over_a_cache_that_does_not_seal_is_the_oracle():
    """An FP16 cache that never seals (config 2's layout: every page FP16 in
    the page table, the last one partly filled): one decode query with its
    masses, against float64 over the same keys and values."""
    m = mi()
    d = m.device
    for heads, kv, hd, seq in ((14, 2, 64, 8192 - 5), (12, 2, 128, 32 * 37 + 1), (14, 2, 64, 20)):
        announce("paged fp16 decode", heads, kv, hd, seq)
        rng = np.random.default_rng(seq)
        k, v = normal(rng, seq, kv, hd), normal(rng, seq, kv, hd)
        alloc, cache = pages_for(32, kv, hd, 0)
        assert not cache.seals
        store_in_runs(cache, 0, k, v, [seq - 1, 1])
        q = normal(rng, 1, heads, hd)
        pages = -(-seq // 32)
        out, mass = d.empty(heads * hd), d.empty_f32(heads * pages)
        cache.attention(0, put(q), None, None, out, 1, seq, heads, kv, hd, None, None, mass,
                        d.empty_f32(d.attention_partials(hd)))
        want, w = att.attention64(q, k, v)
        assert_attention_close(out.to_numpy().reshape(1, heads, hd), want, "paged",
                               att.attention_bound(q, k, v, w))
        assert_mass_close(mass.to_numpy().reshape(heads, pages), att.page_mass(w[:, 0], 32),
                          "paged mass")


def test_the_row_launch_is_rmsnorm_rope_and_store_to_the_bit():
    """rope_store (config 2's row work as one launch) against the three
    calls it replaces on a twin cache: the normed row, the rotated q and k
    and every page byte agree to the bit, at the 0.5B and 1.5B head shapes,
    mid-page, at a page's last row and its first; a position past the
    reserved ones rotates but stores nothing. The three calls are held to
    the float64 references by the pointwise and decode tests."""
    m = mi()
    d = m.device
    for heads, kv, hd, hidden, positions in ((14, 2, 64, 896, (100, 127, 128)),
                                             (12, 2, 128, 1536, (33, 63))):
        rng = np.random.default_rng(hd)
        rope = d.RopeTable(hd, 1e6)
        rope.cover(4096)
        seq = 160
        k, v = normal(rng, seq, kv, hd), normal(rng, seq, kv, hd)
        (alloc_a, a), (alloc_b, b) = pages_for(32, kv, hd, 0), pages_for(32, kv, hd, 0)
        for cache in (a, b):
            store_in_runs(cache, 1, k, v, [seq])
        norm_w = put(rng.uniform(0.5, 1.5, hidden))
        for pos in positions + (seq,):
            announce("row launch", heads, kv, hd, pos)
            x = d.upload_f32(rng.standard_normal(hidden).astype(np.float32))
            raw = put(normal(rng, heads + kv, hd))
            vals = put(normal(rng, kv, hd))
            at = d.DeviceIndex([pos])
            rows = (heads + kv) * hd
            # The three calls.
            n_a, qk_a = d.empty(hidden), d.empty(rows)
            d.rmsnorm_f32(x, norm_w, n_a, 1, hidden, 1e-6)
            d.rope_from_table(raw, at, rope, qk_a, 1, heads + kv, hd)
            if pos < seq:
                a.store(1, d.view(qk_a, heads * hd, kv * hd), vals, pos, 1)
            # The one launch.
            n_b, qk_b = d.empty(hidden), d.empty(rows)
            b.rope_store(1, raw, qk_b, heads, at, rope, vals, norm=(x, norm_w, n_b, 1e-6))
            np.testing.assert_array_equal(n_b.to_numpy(), n_a.to_numpy())
            np.testing.assert_array_equal(qk_b.to_numpy(), qk_a.to_numpy())
            for page in range(seq // 32):
                np.testing.assert_array_equal(alloc_b.read(1, page), alloc_a.read(1, page))
        # Without the norm: the rows alone, and layer 0 left as it was.
        before = alloc_b.read(0, 1)
        raw = put(normal(rng, heads + kv, hd))
        qk_a, qk_b = d.empty((heads + kv) * hd), d.empty((heads + kv) * hd)
        at = d.DeviceIndex([40])
        d.rope_from_table(raw, at, rope, qk_a, 1, heads + kv, hd)
        b.rope_store(1, raw, qk_b, heads, at, rope, put(normal(rng, kv, hd)))
        np.testing.assert_array_equal(qk_b.to_numpy(), qk_a.to_numpy())
        np.testing.assert_array_equal(alloc_b.read(0, 1), before)
    # A cache that seals refuses it.
    _, sealing = pages_for(32, 2, 64, 1)
    rope = d.RopeTable(64, 1e6)
    rope.cover(64)
    with pytest.raises(Exception, match="seals"):
        sealing.rope_store(0, put(np.zeros(16 * 64)), d.empty(16 * 64), 14, d.DeviceIndex([0]),
                           rope, put(np.zeros(128)))


def test_the_row_attention_is_rope_store_then_attention_to_the_bit():
    """attend_row (config 2's layer as two launches: the pages launch turns
    q and the row's k, stores the row and forms the RMSNorm, then the
    combine) against rope_store then attention with partials on a twin
    cache: the output, the normed row, the turned rows and every page byte
    agree to the bit, at the 0.5B and 1.5B head shapes at position 0 (one
    row to attend), mid-page, at a page's last row and a page's first, at
    the largest group (16 q heads a KV head), and at a Llama shape long
    enough that the
    launch is bounded to the resident workgroups (the current page is then a
    wave's second). The two calls are held to the float64 references by the
    row launch and decode tests."""
    m = mi()
    d = m.device
    for heads, kv, hd, hidden, seq, positions in ((14, 2, 64, 896, 160, (0, 100, 127, 128)),
                                                  (12, 2, 128, 1536, 96, (33, 63, 64)),
                                                  (32, 2, 128, 2048, 96, (40,)),
                                                  (32, 8, 128, 4096, 16448, (16447,))):
        rng = np.random.default_rng(hd + kv)
        rope = d.RopeTable(hd, 1e6)
        rope.cover(seq + 64)
        k, v = normal(rng, seq, kv, hd), normal(rng, seq, kv, hd)
        (alloc_a, a), (alloc_b, b) = pages_for(32, kv, hd, 0), pages_for(32, kv, hd, 0)
        for cache in (a, b):
            store_in_runs(cache, 1, k, v, [seq])
            cache.reserve(seq + 1)
        norm_w = put(rng.uniform(0.5, 1.5, hidden))
        partials = d.empty_f32(d.attention_partials(hd))
        rows = (heads + kv) * hd
        for pos in positions:
            for with_norm in (True, False):
                announce("row attention", heads, kv, hd, pos, with_norm)
                x = d.upload_f32(rng.standard_normal(hidden).astype(np.float32))
                raw = put(normal(rng, heads + kv, hd))
                vals = put(normal(rng, kv, hd))
                n_a, qk_a, out_a = d.empty(hidden), d.empty(rows), d.empty(heads * hd)
                n_b, qk_b, out_b = d.empty(hidden), d.empty(rows), d.empty(heads * hd)
                a.rope_store(1, raw, qk_a, heads, d.DeviceIndex([pos]), rope, vals,
                             norm=(x, norm_w, n_a, 1e-6) if with_norm else None)
                a.attention(1, d.view(qk_a, 0, heads * hd), None, None, out_a, 1, pos + 1, heads,
                            kv, hd, None, None, None, partials)
                b.attend_row(1, raw, qk_b, heads, pos + 1, rope, vals, out_b,
                             norm=(x, norm_w, n_b, 1e-6) if with_norm else None)
                got = out_b.to_numpy()
                assert np.isfinite(got).all()
                np.testing.assert_array_equal(got, out_a.to_numpy())
                np.testing.assert_array_equal(qk_b.to_numpy(), qk_a.to_numpy())
                if with_norm:
                    np.testing.assert_array_equal(n_b.to_numpy(), n_a.to_numpy())
                page = pos // 32
                for near in range(max(0, page - 1), page + 1):
                    np.testing.assert_array_equal(alloc_b.read(1, near), alloc_a.read(1, near))
        # Without qk_out: the same output and page.
        pos = positions[0]
        raw, vals = put(normal(rng, heads + kv, hd)), put(normal(rng, kv, hd))
        out_a, out_b = d.empty(heads * hd), d.empty(heads * hd)
        b.attend_row(1, raw, d.empty(rows), heads, pos + 1, rope, vals, out_a)
        b.attend_row(1, raw, None, heads, pos + 1, rope, vals, out_b)
        np.testing.assert_array_equal(out_b.to_numpy(), out_a.to_numpy())
    # A cache that seals, and a table short of the position, are refused.
    _, sealing = pages_for(32, 2, 64, 1)
    rope = d.RopeTable(64, 1e6)
    rope.cover(64)
    with pytest.raises(Exception, match="seals"):
        sealing.attend_row(0, put(np.zeros(16 * 64)), None, 14, 1, rope, put(np.zeros(128)),
                           d.empty(14 * 64))
    _, plain = pages_for(32, 2, 64, 0)
    plain.reserve(256)
    with pytest.raises(Exception, match="covering"):
        plain.attend_row(0, put(np.zeros(16 * 64)), None, 14, 200, rope, put(np.zeros(128)),
                         d.empty(14 * 64))


def test_asking_for_the_mass_changes_no_output_bit():
    for P in (16, 32):
        for tier in (0, 2):
            announce("mass off", P, tier)
            tmap = [[tier] * 20 for _ in range(LAYERS)]
            m, alloc, cache, k, v, q, _ = decode_case(P, 2, 64, 14, tmap, P * 12 + 3, seed=P)
            on, _ = run_decode(m, cache, k, v, q, 14, 2, 64, mass=True)
            off, _ = run_decode(m, cache, k, v, q, 14, 2, 64, mass=False)
            np.testing.assert_array_equal(on, off)


def test_the_fused_ewma_is_the_oracle_fold_of_the_kernel_s_masses():
    """Decode steps with the scores folded in the same pass: the scores
    equal, to the bit, the oracle's fp32 fold (importance_scores.cu:31-50) of
    the masses the same kernel wrote; and the masses are the float64 ones."""
    m = mi()
    d = m.device
    P, heads, kv, hd = 32, 12, 2, 128
    rng = np.random.default_rng(21)
    seq0 = P * 10 + 4
    total = seq0 + 40
    k, v = normal(rng, total, kv, hd), normal(rng, total, kv, hd)
    tmap = [[(i * 7) % 4 for i in range(total // P + 1)] for _ in range(LAYERS)]
    alloc, cache = pages_for(P, kv, hd, 0, tier_map=tmap, always_seal=True)
    max_pages = total // P + 2
    scores = d.ImportanceScores(LAYERS, max_pages)
    store_in_runs(cache, 0, k[:seq0], v[:seq0], [seq0])
    steps = []
    for t in range(seq0, total):
        cache.reserve(t + 1)
        cache.store(0, put(k[t:t + 1]), put(v[t:t + 1]), t, 1)
        q = normal(rng, 1, heads, hd)
        announce("ewma step", t)
        got, mass = run_decode(m, cache, k[:t + 1], v[:t + 1], q, heads, kv, hd, scores=scores)
        steps.append((0, mass.astype(np.float32)))
        if t % 13 == 0:
            want, want_mass, bound = oracle_decode(alloc, P, kv, hd, k[:t + 1], v[:t + 1], q)
            assert_attention_close(got, want, f"step {t}", bound)
            assert_mass_close(mass, want_mass, f"step {t}")
    np.testing.assert_array_equal(scores.download(), ewma.host_ewma(steps, LAYERS, max_pages))


def test_one_launch_over_several_layers_matches_each_layer_and_the_oracle():
    """attention_layers, beyond the reference (several layers' decode queries
    in one launch, streamed through LDS a page at a time, the waves of a
    range one KV head each: 1, 2, 4 and 8 KV heads, and 3, whose heads a
    range's waves cannot share), against each layer's own split attention
    call and the float64 oracle, at the 1e-3 bar, over mixed tiers, 1.5B /
    0.5B / Llama head shapes; the scores folded over
    two steps equal, to the bit, the oracle's fold of the launch's own masses.
    Also a sub-range of layers, a cache that does not seal, and a range past
    the cache refused."""
    m = mi()
    d = m.device
    P, L = 32, 3
    cases = [((12, 2, 128), 32 * 9 + 7), ((12, 2, 128), 32 * 64), ((12, 2, 128), 33),
             ((14, 2, 64), 32 * 40 + 1), ((32, 8, 64), 32 * 17 + 30),
             ((12, 4, 64), 32 * 11 + 3), ((9, 3, 128), 32 * 6 + 5), ((4, 1, 128), 32 * 5),
             ((12, 2, 128), 20)]  # no page sealed yet: the cache has no page tables
    for (heads, kv, hd), seq in cases:
        announce("layers in one launch", heads, kv, hd, seq)
        rng = np.random.default_rng(seq + hd)
        cap = [4096] * 4
        cap[0] += L * 2 + 8
        alloc = m.PagedKVCache(page_sizes(P, kv, hd), cap)
        tmap = [[(i * 5 + l) % 4 for i in range(seq // P + 1)] for l in range(L)]
        cache = d.KVPages(alloc, L, P, kv, hd, 0, d.Halves.Both, tmap, True)
        k, v = normal(rng, L, seq, kv, hd), normal(rng, L, seq, kv, hd)
        for l in range(L):
            store_in_runs(cache, l, k[l], v[l], [seq - 1, 1])
        pages = -(-seq // P)
        max_pages = pages + 1
        scores = d.ImportanceScores(L, max_pages)
        part = d.empty_f32(d.attention_partials(hd))
        own_k, own_v = put(k[:, -1]), put(v[:, -1])
        own = (seq - 1) // P
        folded = []
        for step in range(2):
            q = normal(rng, L, heads, hd)
            out, mass = d.empty(L * heads * hd), d.empty_f32(L * heads * pages)
            cache.attention_layers(0, L, put(q), out, seq, heads, kv, hd, own_k, own_v, mass,
                                   scores=scores)
            got = out.to_numpy().reshape(L, heads, hd)
            got_mass = mass.to_numpy()[:L * heads * pages].reshape(L, heads, pages)
            oracle = {}
            for l in range(L):
                folded.append((l, got_mass[l].astype(np.float32)))
                sealed, tiers = sealed_pages(alloc, l, own)
                want, want_mass, bound = att.causal_decode(q[l:l + 1], sealed, tiers,
                                                           k[l, own * P:], v[l, own * P:], kv, hd,
                                                           P, with_bound=True)
                oracle[l] = (want, bound)
                assert_attention_close(got[l:l + 1], want, f"layer {l} seq={seq}", bound)
                assert_mass_close(got_mass[l], want_mass, f"layer {l} mass")
                # The layer's own launch meets the same bar.
                o1, m1 = d.empty(heads * hd), d.empty_f32(heads * pages)
                cache.attention(l, put(q[l]), None, None, o1, 1, seq, heads, kv, hd,
                                put(k[l, -1:]), put(v[l, -1:]), m1, part)
                assert_attention_close(o1.to_numpy().reshape(1, heads, hd), want,
                                       f"layer {l} own launch", bound)
                assert_mass_close(m1.to_numpy().reshape(heads, pages), want_mass,
                                  f"layer {l} own launch mass")
            np.testing.assert_array_equal(scores.download(),
                                          ewma.host_ewma(folded, L, max_pages))
        # Layers 1 and 2 alone.
        out2 = d.empty(2 * heads * hd)
        cache.attention_layers(1, 2, put(q[1:]), out2, seq, heads, kv, hd, put(k[1:, -1]),
                               put(v[1:, -1]))
        two = out2.to_numpy().reshape(2, heads, hd)
        for i, l in enumerate((1, 2)):
            assert_attention_close(two[i:i + 1], oracle[l][0], f"layers 1-2: {l}", oracle[l][1])
        with pytest.raises(IndexError):
            cache.attention_layers(2, 2, put(q[1:]), out2, seq, heads, kv, hd, put(k[1:, -1]),
                                   put(v[1:, -1]))
    # A cache that does not seal: every page FP16 in the table, the last partly filled.
    heads, kv, hd, seq = 14, 2, 64, 32 * 20 + 9
    announce("layers in one launch, no seal", seq)
    rng = np.random.default_rng(5)
    cap = [4096] * 4
    cap[0] += L * 2 + 8
    alloc = m.PagedKVCache(page_sizes(P, kv, hd), cap)
    cache = d.KVPages(alloc, L, P, kv, hd, 0, d.Halves.Both, [], False)
    assert not cache.seals
    k, v = normal(rng, L, seq, kv, hd), normal(rng, L, seq, kv, hd)
    for l in range(L):
        store_in_runs(cache, l, k[l], v[l], [seq])
    q = normal(rng, L, heads, hd)
    out = d.empty(L * heads * hd)
    cache.attention_layers(0, L, put(q), out, seq, heads, kv, hd)
    got = out.to_numpy().reshape(L, heads, hd)
    for l in range(L):
        want, w = att.attention64(q[l:l + 1], k[l], v[l])
        assert_attention_close(got[l:l + 1], want, f"no-seal layer {l}",
                               att.attention_bound(q[l:l + 1], k[l], v[l], w))


def test_downgrade_upgrade_and_moves_are_quantise_of_the_shadow():
    """A page at tier T is quantise_page(FP16, T) of its shadow; a page back
    at FP16 is its shadow; a batch leaves every byte, tier and shadow as the
    per-page path does (tests/test_batched_moves.py:98-126)."""
    m = mi()
    P, kv, hd = 32, 2, 128
    rng = np.random.default_rng(5)
    seq = P * 12
    k, v = normal(rng, seq, kv, hd), normal(rng, seq, kv, hd)
    plan = [(0, 1, 2), (0, 3, 3), (1, 0, 1), (1, 5, 2), (0, 7, 3), (1, 11, 2)]
    caches = []
    for batched in (False, True):
        alloc, cache = pages_for(P, kv, hd, 0, always_seal=True)
        for layer in range(LAYERS):
            store_in_runs(cache, layer, k, v, [seq])
        announce("moves", "batched" if batched else "per-page")
        if batched:
            cache.move_pages(plan)
            assert cache.last_batch["moves"] == len(plan)
            assert cache.last_batch["shadows_taken"] == len(plan)
        else:
            for layer, page, tier in plan:
                cache.downgrade(layer, page, tier)
        caches.append((alloc, cache))
    for (alloc, cache), name in zip(caches, ("per-page", "batched")):
        for layer, page, tier in plan:
            shadow = cache.shadow(layer, page)
            kp = k[page * P:(page + 1) * P].astype(np.float16)
            vp = v[page * P:(page + 1) * P].astype(np.float16)
            np.testing.assert_array_equal(shadow, quant.fp16_page(kp, vp))
            assert cache.page_tier(layer, page) == tier
            np.testing.assert_array_equal(alloc.read(layer, page),
                                          quant.quantise_page(kp, vp, tier, P), err_msg=name)
    a0, c0 = caches[0]
    a1, c1 = caches[1]
    np.testing.assert_array_equal(c0.page_tiers(), c1.page_tiers())
    for layer in range(LAYERS):
        for page in range(12):
            np.testing.assert_array_equal(a0.read(layer, page), a1.read(layer, page))
    # Up again, and across: from the shadows, per page and in a batch.
    up = [(0, 1, 0), (0, 3, 1), (1, 5, 3)]
    for layer, page, tier in up:
        c0.upgrade(layer, page, tier) if tier < plan_tier(plan, layer, page) else \
            c0.downgrade(layer, page, tier)
    c1.move_pages(up)
    for alloc, cache in caches:
        for layer, page, tier in up:
            kp = k[page * P:(page + 1) * P].astype(np.float16)
            vp = v[page * P:(page + 1) * P].astype(np.float16)
            want = quant.fp16_page(kp, vp) if tier == 0 else quant.quantise_page(kp, vp, tier, P)
            np.testing.assert_array_equal(alloc.read(layer, page), want)
            assert cache.page_tier(layer, page) == tier


def test_a_refused_large_batch_leaves_no_shadow_and_the_retry_is_exact():
    """A batch of at least 256 moves takes its first downgrades' shadows in
    pieces of 1,024 while it is validated: refused at its last move (a page
    named twice) after a piece has gone out, it leaves no shadow, tier or
    page byte changed; the same batch without that move then leaves every
    page at quantise_page of its rows and every shadow at the page's FP16
    bytes (the places the refused piece wrote are taken again)."""
    m = mi()
    P, kv, hd = 32, 2, 64
    rng = np.random.default_rng(8)
    pages = 560
    k, v = normal(rng, P * pages, kv, hd), normal(rng, P * pages, kv, hd)
    alloc, cache = pages_for(P, kv, hd, 0, always_seal=True)
    for layer in range(LAYERS):
        store_in_runs(cache, layer, k, v, [P * pages])
    plan = [(layer, page, 1 + (layer * pages + page) % 3)
            for layer in range(LAYERS) for page in range(pages - 1)]
    assert len(plan) > 1024
    before = [alloc.read(layer, page) for layer, page, _ in plan[:40]]
    shadows = cache.shadow_count
    announce("refused large batch", len(plan) + 1)
    with pytest.raises(Exception, match="twice"):
        cache.move_pages(plan + [plan[7]])
    assert cache.shadow_count == shadows
    assert (cache.page_tiers()[:, :pages] == 0).all()
    for (layer, page, _), want in zip(plan[:40], before):
        np.testing.assert_array_equal(alloc.read(layer, page), want)
    announce("large batch", len(plan))
    cache.move_pages(plan)
    assert cache.last_batch["shadows_taken"] == len(plan)
    for layer, page, tier in plan[::9] + plan[1020:1030] + plan[-3:]:
        kp = k[page * P:(page + 1) * P].astype(np.float16)
        vp = v[page * P:(page + 1) * P].astype(np.float16)
        assert cache.page_tier(layer, page) == tier
        np.testing.assert_array_equal(cache.shadow(layer, page), quant.fp16_page(kp, vp))
        np.testing.assert_array_equal(alloc.read(layer, page), quant.quantise_page(kp, vp, tier, P))


def plan_tier(plan, layer, page):
    return next(t for l, p, t in plan if l == layer and p == page)


def test_refusals_leave_every_byte_unchanged():
    m = mi()
    P, kv, hd = 32, 2, 64
    rng = np.random.default_rng(6)
    k, v = normal(rng, P * 4, kv, hd), normal(rng, P * 4, kv, hd)
    alloc, cache = pages_for(P, kv, hd, 0, always_seal=True)
    for layer in range(LAYERS):
        store_in_runs(cache, layer, k, v, [P * 4])
    cache.downgrade(0, 1, 2)
    before = [[alloc.read(l, p) for p in range(4)] for l in range(LAYERS)]
    tiers = cache.page_tiers().copy()
    with pytest.raises(ValueError, match="lower"):
        cache.downgrade(0, 1, 1)
    with pytest.raises(ValueError, match="higher"):
        cache.upgrade(0, 2, 1)
    with pytest.raises(ValueError, match="twice"):
        cache.move_pages([(0, 2, 3), (0, 2, 2)])
    with pytest.raises(ValueError, match="already"):
        cache.move_pages([(0, 2, 0)])
    with pytest.raises(ValueError, match="not a page of positions"):
        cache.move_pages([(0, 9, 2)])
    m.fail_next_granules(1)
    with pytest.raises(m.OutOfMemory):
        cache.move_pages([(0, 0, 3), (1, 3, 3), (1, 2, 1)])
    m.fail_next_granules(0)
    np.testing.assert_array_equal(cache.page_tiers(), tiers)
    for l in range(LAYERS):
        for p in range(4):
            np.testing.assert_array_equal(alloc.read(l, p), before[l][p])


def test_an_evicted_page_reads_as_a_masked_one_to_the_bit():
    """tests/test_split_attention.py:295-319: attention over a cache with a
    page evicted is, to the bit, attention over the same cache with it
    masked; its mass is 0."""
    m = mi()
    P, heads, kv, hd = 32, 12, 2, 128
    rng = np.random.default_rng(8)
    seq = P * 20 + 3
    k, v = normal(rng, seq, kv, hd), normal(rng, seq, kv, hd)
    q = normal(rng, 1, heads, hd)
    outs = []
    for how in ("evict", "mask"):
        alloc, cache = pages_for(P, kv, hd, 2)
        store_in_runs(cache, 0, k, v, [seq - 1, 1])
        for page in (3, 4, 11):
            getattr(cache, how)(0, page)
        announce("unread", how)
        got, mass = run_decode(m, cache, k, v, q, heads, kv, hd)
        assert np.all(mass[:, [3, 4, 11]] == 0)
        outs.append(got)
        if how == "mask":
            pages, tiers = sealed_pages(alloc, 0, seq // P)
            for p in (3, 4, 11):
                tiers[p] = quant.UNREAD
            want, want_mass, bound = att.causal_decode(q, pages, tiers, k[(seq // P) * P:],
                                                       v[(seq // P) * P:], kv, hd, P,
                                                       with_bound=True)
            assert_attention_close(got, want, "masked", bound)
            assert_mass_close(mass, want_mass, "masked mass")
    np.testing.assert_array_equal(outs[0], outs[1])


def test_full_size_config3_layer_against_the_oracle():
    """Config 3 (the headline workload) at its full size on one layer: 32K positions of
    Qwen2.5-1.5B shape, tiers 20/30/40/10 by seeded importance, built by
    storing all rows (pages sealed at birth tier in batched launches), then
    one decode with the fused mass and EWMA, against the float64 oracle."""
    from microinfer import workloads as w
    m = mi()
    d = m.device
    shape = w.QWEN_15B
    P, seq = 32, 32768
    rng = np.random.default_rng(0)
    outliers = w.outlier_channels(rng, shape.kv_width)
    k, v = w.kv_rows(rng, seq, shape, outliers)
    tmap = [w.tiers_by_importance(np.random.default_rng(0), seq // P - 1, w.MIX_CONFIG3).tolist()]
    tmap = tmap * LAYERS
    alloc, cache = pages_for(P, shape.kv_heads, shape.head_dim, 0, tier_map=tmap,
                             always_seal=True, capacity=1100 * LAYERS)
    announce("config3 full layer: store")
    store_in_runs(cache, 0, k.astype(np.float32), v.astype(np.float32), [seq - 1, 1])
    counts = np.bincount(cache.page_tiers()[0][:seq // P - 1], minlength=4)
    assert list(counts) == [205, 307, 409, 102]
    # The pages the decode reads are, byte for byte, the oracle's quantise_page
    # of their rows at their birth tiers (sealed by the batched store launches).
    for page in range(seq // P - 1):
        tier = tmap[0][page]
        kp, vp = k[page * P:(page + 1) * P], v[page * P:(page + 1) * P]
        want_page = quant.fp16_page(kp, vp) if tier == 0 else quant.quantise_page(kp, vp, tier, P)
        np.testing.assert_array_equal(alloc.read(0, page), want_page, err_msg=f"page {page}")
    q = fp16_exact(rng.standard_normal((1, shape.heads, shape.head_dim)))
    scores = d.ImportanceScores(LAYERS, seq // P)
    announce("config3 full layer: decode")
    got, mass = run_decode(m, cache, k.astype(np.float32), v.astype(np.float32), q, shape.heads,
                           shape.kv_heads, shape.head_dim, scores=scores)
    want, want_mass, bound = oracle_decode(alloc, P, shape.kv_heads, shape.head_dim, k, v, q)
    assert_attention_close(got, want, "config3", bound)
    assert_mass_close(mass, want_mass, "config3 mass")
    np.testing.assert_array_equal(scores.download()[0],
                                  ewma.host_ewma([(0, mass.astype(np.float32))], 1, seq // P)[0])


def test_the_shadow_store_binding_takes_a_page_once():
    """The standalone shadow store (bindings_device.cpp:652-680; the store a
    KVPages holds): take copies the first page_bytes of a device tensor into
    a new pinned shadow; a second take for the same page is refused ("has a
    shadow already", RuntimeError) and the first shadow kept; contains and
    count follow; shadows pack into pinned allocations of whole pages
    (shadow_store.h:28), a new allocation only when the last is full; a page
    with no shadow is a PageNotFound, a tensor short of a page a ValueError."""
    m = mi()
    d = m.device
    page_bytes = quant.page_bytes(0, 2, 128)
    store = d.ShadowStore(page_bytes)
    rng = np.random.default_rng(96)
    first = normal(rng, page_bytes // 2)
    announce("shadow store")
    store.take(0, 1, put(first))
    with pytest.raises(RuntimeError, match="has a shadow already"):
        store.take(0, 1, put(normal(rng, page_bytes // 2)))
    np.testing.assert_array_equal(store.shadow(0, 1), first.astype(np.float16).view(np.uint8))
    assert store.count == 1 and store.contains(0, 1) and not store.contains(1, 0)
    per_allocation = max(1, d.ShadowStore.allocation_bytes // page_bytes)
    taken = {}
    for page in range(2, per_allocation + 2):
        taken[page] = normal(rng, page_bytes // 2)
        store.take(3, page, put(taken[page]))
    assert store.count == per_allocation + 1
    assert store.bytes == 2 * per_allocation * page_bytes
    for page, rows in taken.items():
        assert store.contains(3, page)
        np.testing.assert_array_equal(store.shadow(3, page), rows.astype(np.float16).view(np.uint8))
    with pytest.raises(m.PageNotFound):
        store.shadow(5, 5)
    with pytest.raises(ValueError):
        store.take(0, 99, put(first[:16]))
    assert store.count == per_allocation + 1 and not store.contains(0, 99)


def test_chained_store_and_decode_steps_across_a_seal_at_llama_shape():
    """Forty-four decode steps at the Llama-3.2-1B shape (32 q / 8 KV heads,
    head_dim 64), each storing its row and then attending, crossing a seal
    (the own page's 32nd row arrives, the page is quantised at its birth tier,
    the next open page takes over) over a 30/40/30 FP16/INT8/INT4 cache:
    every step's output and masses against the float64 causal view of the
    cache as it then is, and the scores folded on every step equal, to the
    bit, the oracle's fold of the kernel's masses."""
    from microinfer import workloads as w
    m = mi()
    d = m.device
    P, shape = 32, w.LLAMA_1B
    heads, kv, hd = shape.heads, shape.kv_heads, shape.head_dim
    rng = np.random.default_rng(17)
    seq0, steps = P * 20 + 10, 44                 # 650 -> 694: seals page 20 at 672
    total = seq0 + steps
    k, v = normal(rng, total, kv, hd), normal(rng, total, kv, hd)
    k[:, :, rng.choice(hd, 2, replace=False)] *= 10
    k = fp16_exact(k)
    tmap = w.tier_map(0, LAYERS, total // P + 1, w.MIX_CONFIG5)
    alloc, cache = pages_for(P, kv, hd, 0, tier_map=tmap, always_seal=True)
    max_pages = total // P + 1
    scores = d.ImportanceScores(LAYERS, max_pages)
    store_in_runs(cache, 0, k[:seq0], v[:seq0], [seq0])
    folded = []
    for t in range(seq0, total):
        cache.reserve(t + 1)
        cache.store(0, put(k[t:t + 1]), put(v[t:t + 1]), t, 1)
        q = normal(rng, 1, heads, hd)
        announce("chained llama step", t)
        got, mass = run_decode(m, cache, k[:t + 1], v[:t + 1], q, heads, kv, hd, scores=scores)
        folded.append((0, mass.astype(np.float32)))
        want, want_mass, bound = oracle_decode(alloc, P, kv, hd, k[:t + 1], v[:t + 1], q)
        assert_attention_close(got, want, f"step {t}", bound)
        assert_mass_close(mass, want_mass, f"step {t} mass")
        np.testing.assert_allclose(mass.sum(1), 1.0, atol=1e-5)
    # The page sealed during the run holds quantise_page of its rows.
    sealed = seq0 // P
    assert total // P > sealed
    tier = int(alloc.locate(0, sealed)[0])
    assert tier == tmap[0][sealed]
    kp = k[sealed * P:(sealed + 1) * P].astype(np.float16)
    vp = v[sealed * P:(sealed + 1) * P].astype(np.float16)
    want_page = quant.fp16_page(kp, vp) if tier == 0 else quant.quantise_page(kp, vp, tier, P)
    np.testing.assert_array_equal(alloc.read(0, sealed), want_page)
    np.testing.assert_array_equal(scores.download(), ewma.host_ewma(folded, LAYERS, max_pages))


@pytest.mark.parametrize("extra", [10, 700])
def test_llama_shape_at_16k_two_kv_heads_a_wave_is_the_oracle(extra):
    """At the Llama-3.2-1B shape and 16K positions (more waves of one KV head
    each than the device holds at once) the decode takes two KV heads a wave
    as one 128-channel unit: output and masses against the float64 causal
    view of a 30/40/30 FP16/INT8/INT4 cache, and the scores the oracle's
    fold of the kernel's masses, to the bit. Past 512 pages (65 and 67
    splits a KV-head pair here, against the 64 workgroups a pair the device
    holds at once) the busy workgroups take balanced runs of pages and the
    splits past them are empty partials."""
    from microinfer import workloads as w
    P, shape = 32, w.LLAMA_1B
    heads, kv, hd = shape.heads, shape.kv_heads, shape.head_dim
    seq = 16384 + extra
    pages = seq // P + 1
    tmap = w.tier_map(1, LAYERS, pages, w.MIX_CONFIG5)
    announce("llama 16K decode", seq)
    m, alloc, cache, k, v, q, _ = decode_case(P, kv, hd, heads, tmap, seq, seed=23)
    scores = m.device.ImportanceScores(LAYERS, pages)
    got, mass = run_decode(m, cache, k, v, q, heads, kv, hd, scores=scores)
    want, want_mass, bound = oracle_decode(alloc, P, kv, hd, k, v, q)
    assert_attention_close(got, want, "llama 16K", bound)
    assert_mass_close(mass, want_mass, "llama 16K mass")
    np.testing.assert_allclose(mass.sum(1), 1.0, atol=1e-5)
    np.testing.assert_array_equal(scores.download(),
                                  ewma.host_ewma([(0, mass.astype(np.float32))], LAYERS, pages))


def test_decode_after_pages_move_reads_them_where_they_now_are():
    """tests/test_kv_pages.py:112-150 and tests/test_quantised_pages.py:
    202-224: the cache's page tables are resolved by a first decode; then
    pages move under it three ways: a batched move (new slots at new tiers),
    an eviction whose free moves a tier's tail page into the hole, and a
    free of someone else's page that moves one of the cache's own pages. The
    slot each moved page left is then taken by another page and filled with
    NaN, so that a stale table cannot read the old bytes back by luck. Every
    decode after each change, the per-layer call and the one-launch form,
    meets the float64 oracle over the cache as it then is."""
    m = mi()
    d = m.device
    P, heads, kv, hd = 32, 12, 2, 128
    rng = np.random.default_rng(31)
    seq = P * 24 + 5
    k, v = normal(rng, seq, kv, hd), normal(rng, seq, kv, hd)
    tmap = [[(1, 0, 2, 0, 3)[i % 5] for i in range(seq // P + 1)] for _ in range(LAYERS)]
    alloc, cache = pages_for(P, kv, hd, 0, tier_map=tmap, always_seal=True)
    cache.reserve(P)
    # Someone else's pages, between the cache's own at every tier.
    for t in range(4):
        alloc.allocate(90 + t, 0, t)
    store_in_runs(cache, 0, k, v, [seq - 1, 1])
    store_in_runs(cache, 1, k, v, [seq - 1, 1])
    q = normal(rng, 1, heads, hd)
    own = (seq - 1) // P
    pages = own + 1

    def oracle_now():
        """The float64 view of layer 0 as the cache now holds it: an evicted
        page unread."""
        tiers_now = cache.page_tiers()[0]
        raw, tiers = [], []
        for p in range(own):
            if tiers_now[p] == 4:
                raw.append(None)
                tiers.append(quant.UNREAD)
            else:
                raw.append(alloc.read(0, p))
                tiers.append(int(alloc.locate(0, p)[0]))
        return att.causal_decode(q, raw, tiers, k[own * P:], v[own * P:], kv, hd, P,
                                 with_bound=True)

    def decode_both(what):
        announce("moved pages decode", what)
        got, mass = run_decode(m, cache, k, v, q, heads, kv, hd)
        want, want_mass, bound = oracle_now()
        assert_attention_close(got, want, what, bound)
        assert_mass_close(mass, want_mass, what + " mass")
        # The one-launch form over both layers reads the same tables.
        q2 = np.concatenate([q, q])
        out = d.empty(2 * heads * hd)
        mass2 = d.empty_f32(2 * heads * pages)
        cache.attention_layers(0, 2, put(q2), out, seq, heads, kv, hd,
                               put(np.concatenate([k[-1:], k[-1:]])),
                               put(np.concatenate([v[-1:], v[-1:]])), mass2)
        both = out.to_numpy().reshape(2, heads, hd)
        assert_attention_close(both[:1], want, what + " one launch", bound)
        return got

    def poison_slot(tier, slot):
        """Another page takes the slot a moved page left and fills it with
        NaN (FP16) or 0xFF bytes."""
        key = (70 + len(poisoned), 0)
        alloc.allocate(*key, tier)
        assert alloc.locate(*key) == (tier, slot), (alloc.locate(*key), tier, slot)
        nbytes = alloc.page_bytes(tier)
        junk = (np.full(nbytes // 2, np.nan, np.float16).view(np.uint8) if tier == 0
                else np.full(nbytes, 0xFF, np.uint8))
        alloc.write(*key, junk)
        poisoned.append(key)

    poisoned = []
    first = decode_both("before")

    # 1. A foreign free: the tier's tail (one of the cache's pages) moves
    # into the freed slot; the slot it left is poisoned.
    for t in range(4):
        tail = alloc.pages(t)[-1]
        assert tail[0] < LAYERS, "the tail should be one of the cache's pages"
        tail_slot = alloc.locate(*tail)[1]
        alloc.free(90 + t, 0)
        assert alloc.locate(*tail)[1] < tail_slot
        poison_slot(t, tail_slot)
    np.testing.assert_array_equal(decode_both("after a foreign free"), first)

    # 2. A batched move: FP16 pages down, an INT8 page up from its shadow
    # after a first downgrade; the slots the old pages held are reused.
    fp16_pages = [p for p in range(own) if tmap[0][p] == 0][:6]
    plan = [(0, fp16_pages[0], 2), (0, fp16_pages[1], 3), (0, fp16_pages[2], 1),
            (1, fp16_pages[3], 2), (0, fp16_pages[4], 3)]
    cache.move_pages(plan)
    for layer, page, tier in plan:
        assert cache.page_tier(layer, page) == tier
    decode_both("after a batched move")
    cache.move_pages([(0, fp16_pages[0], 0), (0, fp16_pages[1], 1)])
    decode_both("after a restore")

    # 3. An eviction whose free swaps the tier's tail into the hole.
    victim = next(p for p in range(own) if tmap[0][p] == 2 and cache.page_tier(0, p) == 2)
    tier = int(alloc.locate(0, victim)[0])
    tail = alloc.pages(tier)[-1]
    tail_slot = alloc.locate(*tail)[1]
    cache.evict(0, victim)
    if tail != (0, victim):
        assert alloc.locate(*tail)[1] < tail_slot
    poison_slot(tier, tail_slot)
    decode_both("after an eviction")


def test_the_halves_diagnostic_rounds_one_half_through_its_tier():
    """A diagnostic Halves cache (kv_pages.h's Halves, the reference's
    ablation of keys against values) stores every page at FP16: the chosen
    half as quantise_page then dequantise_page at the cache's tier gives it,
    the other half as it came, to the bit; rows arriving one by one, in one
    run, or in runs crossing pages; the register path (P = 32, head_dim 64
    and 128) and the LDS path (P = 16)."""
    m = mi()
    d = m.device

    def check(P, hd, tier, halves, runs_name):
        kv = 2
        rng = np.random.default_rng(P * 7 + hd + tier)
        seq = 3 * P + 3
        k, v = normal(rng, seq, kv, hd), normal(rng, seq, kv, hd)
        k[:, :, rng.choice(hd, 2, replace=False)] *= 10
        k = fp16_exact(k)
        runs = {"one": [seq], "single": [1] * seq, "ragged": [P // 2 + 1, P + 3,
                                                              seq - (3 * P // 2 + 4)]}[runs_name]
        sizes = page_sizes(P, kv, hd)
        alloc = m.PagedKVCache(sizes, [64 + LAYERS * 2] * 4)
        cache = d.KVPages(alloc, LAYERS, P, kv, hd, tier, getattr(d.Halves, halves), [], False)
        assert cache.page_bytes == sizes[0]
        announce("halves", P, hd, tier, halves, runs_name)
        store_in_runs(cache, 1, k, v, runs)
        for i in range(seq // P):
            kp = k[i * P:(i + 1) * P].astype(np.float16)
            vp = v[i * P:(i + 1) * P].astype(np.float16)
            kr, vr = quant.dequantise_page(quant.quantise_page(kp, vp, tier, P), tier, kv, hd, P)
            kr = np.asarray(kr, np.float16)
            vr = np.asarray(vr, np.float16)
            want = quant.fp16_page(kr if halves == "Keys" else kp, vr if halves == "Values" else vp)
            np.testing.assert_array_equal(alloc.read(1, i), want)

    each([(P, hd, t, h, r) for P, hd in ((32, 128), (32, 64), (16, 64)) for t in (1, 2, 3)
          for h in ("Keys", "Values") for r in ("one", "single", "ragged")], check)


def test_a_cache_keeps_its_allocator_alive():
    """The allocator's handle destroyed before its cache's (a garbage
    collector finalizes a cycle in any order): the cache still stores,
    attends and moves pages, and the allocator goes with the cache."""
    import weakref
    m = mi()
    P, heads, kv, hd = 32, 12, 2, 128
    rng = np.random.default_rng(12)
    seq = P * 8 + 3
    k, v = normal(rng, seq, kv, hd), normal(rng, seq, kv, hd)
    alloc, cache = pages_for(P, kv, hd, 0, tier_map=[[2, 0] * 5] * LAYERS, always_seal=True)
    store_in_runs(cache, 0, k, v, [seq - 1])
    # Run the allocator handle's own finalizer now.
    for f, info in list(weakref.finalize._registry.items()):
        if info.args == (alloc._h,) and getattr(info.func, "__name__", "") == "mi_cache_destroy":
            f()
    announce("cache outliving its allocator's handle")
    cache.reserve(seq)
    cache.store(0, put(k[-1:]), put(v[-1:]), seq - 1, 1)
    q = normal(rng, 1, heads, hd)
    got, mass = run_decode(m, cache, k, v, q, heads, kv, hd)
    own = (seq - 1) // P
    assert np.isfinite(got).all() and mass.shape == (heads, own + 1)
    np.testing.assert_allclose(mass.sum(1), 1.0, atol=1e-5)
    cache.move_pages([(0, 1, 3)])
    assert cache.page_tier(0, 1) == 3
    del cache


def test_after_a_capture_the_runtime_is_back_on_the_null_stream():
    """A decode captured as a graph on a stream of the caller's, replayed,
    then the graph and the stream destroyed: the cache's later work (frees
    that give granules back, a store, a decode) runs on the null stream, as
    set_stream(None) after the capture names, and meets the oracle."""
    import weakref
    m = mi()
    d = m.device
    P, heads, kv, hd = 32, 12, 2, 128
    rng = np.random.default_rng(13)
    seq = P * 70 + 5
    k, v = normal(rng, seq, kv, hd), normal(rng, seq, kv, hd)
    alloc, cache = pages_for(P, kv, hd, 0, tier_map=[[1, 0, 2] * 24] * LAYERS, always_seal=True)
    store_in_runs(cache, 0, k, v, [seq - 1, 1])
    q = normal(rng, 1, heads, hd)
    qd, kd, vd = put(q), put(k[-1:]), put(v[-1:])
    out = d.empty(heads * hd)
    part = d.empty_f32(d.attention_partials(hd))

    def body():
        cache.attention(0, qd, None, None, out, 1, seq, heads, kv, hd, kd, vd, None, part)

    body()
    m.synchronize()
    stream = m.Stream()
    graph = m.Graph(stream)
    announce("capture, replay, destroy the stream")
    with graph.capture():
        body()
    graph.launch()
    stream.synchronize()
    for obj in (graph, stream):
        for f, info in list(weakref.finalize._registry.items()):
            if info.weakref() is obj:
                f()
    # Frees (whole granules given back), then an eager decode.
    for page in range(0, 60, 3):
        cache.evict(0, page)
    got, mass = run_decode(m, cache, k, v, q, heads, kv, hd)
    m.synchronize()
    own = (seq - 1) // P
    tiers_now = cache.page_tiers()[0]
    raw, tiers = [], []
    for p in range(own):
        if tiers_now[p] == 4:
            raw.append(None)
            tiers.append(quant.UNREAD)
        else:
            raw.append(alloc.read(0, p))
            tiers.append(int(alloc.locate(0, p)[0]))
    want, want_mass, bound = att.causal_decode(q, raw, tiers, k[own * P:], v[own * P:], kv, hd, P,
                                               with_bound=True)
    assert_attention_close(got, want, "after the stream went", bound)
    assert_mass_close(mass, want_mass, "after the stream went")


def test_a_step_folded_once_is_the_fused_step_to_the_bit():
    """attention_kept on every layer then one fold_kept (beyond the
    reference) against attention(..., mass, scores) a layer at a time: the
    same output bits, the same mass bits, the same score bits, over two
    steps (the second folding into the first's scores), mixed tiers, the
    1.5B and Llama head shapes; and a fold with a layer missing is refused."""
    m = mi()
    d = m.device
    P, L = 32, 3
    for (heads, kv, hd), seq in (((12, 2, 128), 32 * 40 + 7), ((32, 8, 64), 32 * 21 + 30)):
        rng = np.random.default_rng(seq)
        cap = [4096] * 4
        cap[0] += L * 2 + 8
        alloc = m.PagedKVCache(page_sizes(P, kv, hd), cap)
        tmap = [[(i * 3 + l) % 4 for i in range(seq // P + 2)] for l in range(L)]
        cache = d.KVPages(alloc, L, P, kv, hd, 0, d.Halves.Both, tmap, True)
        k, v = normal(rng, L, seq + 1, kv, hd), normal(rng, L, seq + 1, kv, hd)
        pages = -(-seq // P)
        fused_scores = d.ImportanceScores(L, pages + 1)
        kept_scores = d.ImportanceScores(L, pages + 1)
        part = d.empty_f32(d.attention_partials(hd))
        for step, s in enumerate((seq - 1, seq)):
            for l in range(L):
                if step == 0:
                    store_in_runs(cache, l, k[l, :s], v[l, :s], [s])
                else:
                    cache.reserve(s)
                    cache.store(l, put(k[l, s - 1:s]), put(v[l, s - 1:s]), s - 1, 1)
            npages = -(-s // P)
            q = normal(rng, L, heads, hd)
            kept_mass = d.empty_f32(L * heads * npages)
            outs = []
            announce("kept step", heads, kv, hd, s)
            for l in range(L):
                out = d.empty(heads * hd)
                cache.attention_kept(l, put(q[l]), None, None, out, s, heads, kv, hd,
                                     put(k[l, s - 1:s]), put(v[l, s - 1:s]))
                outs.append(out)
            cache.fold_kept(kept_scores, kept_mass, s, heads)
            got_mass = kept_mass.to_numpy().reshape(L, heads, npages)
            for l in range(L):
                out, mass = d.empty(heads * hd), d.empty_f32(heads * npages)
                cache.attention(l, put(q[l]), None, None, out, 1, s, heads, kv, hd,
                                put(k[l, s - 1:s]), put(v[l, s - 1:s]), mass, part,
                                scores=fused_scores)
                np.testing.assert_array_equal(outs[l].raw(), out.raw())
                np.testing.assert_array_equal(got_mass[l], mass.to_numpy().reshape(heads, npages))
            np.testing.assert_array_equal(kept_scores.download(), fused_scores.download())
        # A fold with a layer not attended since the last is refused.
        out = d.empty(heads * hd)
        cache.attention_kept(0, put(q[0]), None, None, out, seq, heads, kv, hd,
                             put(k[0, seq - 1:seq]), put(v[0, seq - 1:seq]))
        with pytest.raises(RuntimeError, match="every layer"):
            cache.fold_kept(kept_scores)
