"""Chunk attention on the matrix cores (the prefill tile, attention.cu:449-746
with qpb = 16; kv_pages.h:86-93): a chunk of queries through a cache that
seals, each query reading the pages before its own at their tiers and its own
page at FP16, against the float64 oracle; the same kernel over an FP16 page
table and contiguous rows; split and unsplit launches.

GPU parity tests, held to the reference's attention gate at 1e-3
(conftest.ATTN_MAX_REL) with the oracle's fp32 error bound."""

import numpy as np
import pytest

from conftest import announce, assert_attention_close, each, fp16_exact
from oracle import attention as att
from oracle import quant
from test_gpu_kv_pages import (LAYERS, mi, normal, pages_for, put, sealed_pages,
                               store_in_runs)

pytestmark = pytest.mark.gpu

P = 32
THETA = 1e6
#: (heads, kv_heads, head_dim): Qwen2.5-1.5B, Qwen2.5-0.5B, Llama-3.2-1B.
SHAPES = [(12, 2, 128), (14, 2, 64), (32, 8, 64)]


def mixed_map(seq):
    order = [1, 0, 3, 2]
    return [[order[(layer + i) % 4] for i in range(seq // P + 1)] for layer in range(LAYERS)]


def chunk_case(heads, kv, hd, seq, seq_q, seed, bias, split, unread=()):
    """Stores `seq` positions, the last `seq_q` as one run, seals pages at the
    mixed tiers, then attends the run's queries through the cache."""
    m = mi()
    d = m.device
    rng = np.random.default_rng(seed)
    k, v = normal(rng, seq, kv, hd), normal(rng, seq, kv, hd)
    k[:, :, rng.choice(hd, 2, replace=False)] *= 10
    k = fp16_exact(k)
    alloc, cache = pages_for(P, kv, hd, 0, tier_map=mixed_map(seq), always_seal=True)
    runs = [seq - seq_q, seq_q] if seq > seq_q else [seq]
    start = store_in_runs(cache, 1, k, v, runs)
    assert start == seq - seq_q
    for page in unread:
        cache.mask(1, page)
    q = normal(rng, seq_q, heads, hd)
    b = fp16_exact(3 * rng.standard_normal((kv, hd))) if bias else None
    rope = None
    if bias:
        rope = d.RopeTable(hd, THETA)
        rope.cover(seq)
    out = d.empty(seq_q * heads * hd)
    part = d.empty_f32(d.attention_partials(hd)) if split else None
    announce("prefill chunk", heads, kv, hd, seq, seq_q, "bias" if bias else "", "split" if split
             else "", unread)
    cache.attention(1, put(q), put(b) if bias else None, rope, out, seq_q, seq, heads, kv, hd,
                    put(k[start:]), put(v[start:]), None, part)
    got = out.to_numpy().reshape(seq_q, heads, hd)
    # The oracle: every full page's bytes and tier as the cache holds them.
    own_first = start // P
    pages, tiers = sealed_pages(alloc, 1, (seq - 1) // P)
    for page in unread:
        tiers[page] = quant.UNREAD
    want, bound = att.causal_chunk(q, pages, tiers, k, v, kv, hd, P, b, THETA, with_bound=True)
    assert_attention_close(got, want, f"{heads}x{kv}x{hd} seq {seq} chunk {seq_q}", bound)
    return got, own_first


def test_a_chunk_reads_earlier_pages_at_their_tiers_and_its_own_at_fp16():
    """Chunks that begin mid-page and cross pages, a one-page chunk, a chunk
    that is the whole prompt, a prompt shorter than a page (no page sealed:
    the cache has no page tables); every shape; the key bias on and off."""
    cases = []
    for i, (heads, kv, hd) in enumerate(SHAPES):
        for seq, seq_q in ((P * 9 + 7, 75), (P * 4, P), (P * 3 + 5, P * 3 + 5), (P * 20 + 1, 16),
                           (P * 6 + 31, 130), (20, 20)):
            for bias in (False, True):
                cases.append((heads, kv, hd, seq, seq_q, 100 * i + seq_q, bias))
    each(cases, lambda h, kv, hd, seq, sq, seed, bias: chunk_case(h, kv, hd, seq, sq, seed, bias,
                                                                  False))


def test_split_launches_fold_to_the_unsplit_result():
    """With the attention workspace the keys split into runs of whole pages
    and a combine folds them; both forms meet the oracle. The reference's
    prefill-tile benchmark shape: 16 queries at the end of a long context."""
    def case(heads, kv, hd, seq, seq_q, bias):
        a, _ = chunk_case(heads, kv, hd, seq, seq_q, 7, bias, True)
        b, _ = chunk_case(heads, kv, hd, seq, seq_q, 7, bias, False)
        np.testing.assert_allclose(a, b, rtol=2e-3, atol=1e-4)

    each([(12, 2, 128, P * 64 + 9, 16, True), (32, 8, 64, P * 40 + 17, 48, False),
          (14, 2, 64, P * 30, 1, True)], case)


def test_unread_pages_weigh_nothing():
    """Masked pages before the chunk are skipped by every query."""
    each([(12, 2, 128, P * 12 + 3, 40, (2, 5, 6)), (32, 8, 64, P * 8 + 20, 70, (0, 3))],
         lambda h, kv, hd, seq, sq, unread: chunk_case(h, kv, hd, seq, sq, 5, False, False, unread))


def test_fp16_page_table_and_contiguous_rows():
    """A cache that does not seal (an FP16 page table) and contiguous rows
    (device.attention) take the same kernel: plain causal attention."""
    m = mi()
    d = m.device
    for heads, kv, hd in SHAPES:
        rng = np.random.default_rng(hd + heads)
        seq, seq_q = P * 7 + 11, 90
        k, v = normal(rng, seq, kv, hd), normal(rng, seq, kv, hd)
        q = normal(rng, seq_q, heads, hd)
        want, w = att.attention64(q, k, v)
        bound = att.attention_bound(q, k, v, w)
        alloc, cache = pages_for(P, kv, hd, 0)
        store_in_runs(cache, 0, k, v, [seq])
        for split in (False, True):
            announce("paged fp16", heads, kv, hd, split)
            out = d.empty(q.size)
            part = d.empty_f32(d.attention_partials(hd)) if split else None
            cache.attention(0, put(q), None, None, out, seq_q, seq, heads, kv, hd, None, None,
                            None, part)
            assert_attention_close(out.to_numpy().reshape(q.shape), want, "paged", bound)
            announce("contiguous", heads, kv, hd, split)
            out = d.empty(q.size)
            d.attention(put(q), put(k), put(v), None, None, out, seq_q, seq, heads, kv, hd, part)
            assert_attention_close(out.to_numpy().reshape(q.shape), want, "contiguous", bound)


def test_config5_chunk_at_full_size():
    """Config 5's prefill chunk at its full size: the Llama-3.2-1B shape
    (32 q / 8 KV heads, head_dim 64), a 2,048-query chunk ending at position
    16,384 over a cache of 30/40/30 FP16/INT8/INT4 pages (tiers by seeded
    importance), split across the attention workspace. 256 queries, eight
    runs of 32 spread over the chunk so that each run is one own page's
    queries, are held to the float64 oracle; every output is finite."""
    from microinfer import workloads as w
    m = mi()
    d = m.device
    shape = w.LLAMA_1B
    heads, kv, hd = shape.heads, shape.kv_heads, shape.head_dim
    seq, seq_q = 16384, 2048
    rng = np.random.default_rng(5)
    k, v = w.kv_rows(rng, seq, shape, w.outlier_channels(rng, shape.kv_width))
    k, v = k.astype(np.float32), v.astype(np.float32)
    tmap = w.tier_map(0, LAYERS, seq // P, w.MIX_CONFIG5)
    alloc, cache = pages_for(P, kv, hd, 0, tier_map=tmap, always_seal=True,
                             capacity=seq // P * LAYERS + 8)
    start = store_in_runs(cache, 1, k, v, [seq - seq_q, seq_q])
    assert start == seq - seq_q
    counts = np.bincount([int(alloc.locate(1, p)[0]) for p in range(seq // P)], minlength=4)
    assert list(counts) == [153, 205, 154, 0], counts
    q = normal(rng, seq_q, heads, hd)
    out = d.empty(seq_q * heads * hd)
    part = d.empty_f32(d.attention_partials(hd))
    announce("config5 chunk", seq, seq_q)
    cache.attention(1, put(q), None, None, out, seq_q, seq, heads, kv, hd, put(k[start:]),
                    put(v[start:]), None, part)
    got = out.to_numpy().reshape(seq_q, heads, hd)
    assert np.isfinite(got).all()
    pages, tiers = sealed_pages(alloc, 1, (seq - 1) // P)
    # Own pages sampled across the chunk: its first, last and six between.
    own_pages = np.linspace(start // P, (seq - 1) // P, 8).astype(int)
    checked = 0
    for own in own_pages:
        end = min((own + 1) * P, seq)      # the run's last position + 1
        first = own * P
        rows = slice(first - start, end - start)
        want, bound = att.causal_chunk(q[rows], pages, tiers, k[:end], v[:end], kv, hd, P,
                                       with_bound=True)
        assert_attention_close(got[rows], want, f"config5 own page {own}", bound)
        checked += end - first
    assert checked >= 256
