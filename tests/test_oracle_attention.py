"""The oracle's attention, causal paged view and per-page mass, pinned by
brute force on tiny inputs and by invariants. CPU only."""

import math

import numpy as np

from conftest import fp16_exact
from oracle import attention as att
from oracle import quant


def qkv(seq_q, seq_k, heads, kv_heads, hd, seed=0):
    rng = np.random.default_rng(seed)
    return (fp16_exact(rng.standard_normal((seq_q, heads, hd))),
            fp16_exact(rng.standard_normal((seq_k, kv_heads, hd))),
            fp16_exact(rng.standard_normal((seq_k, kv_heads, hd))))


def test_attention_is_the_double_loop():
    for seq_q, seq_k, heads, kv_heads, hd in ((1, 5, 4, 2, 4), (3, 3, 2, 1, 6), (2, 7, 6, 3, 2)):
        q, k, v = qkv(seq_q, seq_k, heads, kv_heads, hd, seed=seq_k)
        out, _ = att.attention64(q, k, v)
        np.testing.assert_allclose(out, att.attention_bruteforce(q, k, v), rtol=1e-12, atol=1e-12)


def test_weights_are_a_causal_distribution():
    q, k, v = qkv(5, 9, 4, 2, 8, seed=2)
    _, w = att.attention64(q, k, v)
    np.testing.assert_allclose(w.sum(-1), 1.0, rtol=0, atol=1e-12)
    for i in range(5):
        assert np.all(w[:, i, 4 + i + 1:] == 0)


def test_one_key_gives_its_value_and_group_one_is_multi_head():
    q, k, v = qkv(1, 1, 4, 4, 8, seed=3)
    out, _ = att.attention64(q, k, v)
    np.testing.assert_allclose(out, v.astype(np.float64), rtol=0, atol=0)
    q, k, v = qkv(2, 6, 4, 4, 8, seed=4)
    out, _ = att.attention64(q, k, v)
    for h in range(4):
        o1, _ = att.attention64(q[:, h:h + 1], k[:, h:h + 1], v[:, h:h + 1])
        np.testing.assert_allclose(out[:, h:h + 1], o1, rtol=1e-12, atol=1e-14)


def test_key_bias_is_a_hand_rotation():
    """k + RoPE(bias, j) with cos/sin from math, one element at a time."""
    rng = np.random.default_rng(5)
    hd, theta = 8, 1e4
    bias = fp16_exact(rng.standard_normal((2, hd)))
    rot = att.rotated_bias(bias, 6, theta)
    half = hd // 2
    for j in range(6):
        for h in range(2):
            for d in range(half):
                a = j * theta ** (-2.0 * d / hd)
                c, s = math.cos(a), math.sin(a)
                b1, b2 = float(bias[h, d]), float(bias[h, d + half])
                assert abs(rot[j, h, d] - (b1 * c - b2 * s)) < 1e-12
                assert abs(rot[j, h, d + half] - (b2 * c + b1 * s)) < 1e-12


def test_unread_keys_weigh_nothing_and_mass_sums_to_one():
    q, k, v = qkv(1, 40, 4, 2, 8, seed=6)
    unread = np.zeros(40, bool)
    unread[8:16] = True
    out, w = att.attention64(q, k, v, unread=unread)
    assert np.all(w[:, 0, 8:16] == 0)
    keep = ~unread
    out2, _ = att.attention64(q, k[keep], v[keep])
    np.testing.assert_allclose(out, out2, rtol=1e-12, atol=1e-14)
    mass = att.page_mass(w[:, -1, :], 8)
    np.testing.assert_allclose(mass.sum(1), 1.0, atol=1e-12)
    assert np.all(mass[:, 1] == 0)
    np.testing.assert_allclose(mass[:, 0], w[:, 0, :8].sum(1), rtol=1e-12)


def test_causal_decode_reads_sealed_pages_at_their_tiers():
    """The causal view is the sealed pages dequantised as dequantise_page
    returns them, then the own page's rows as they came."""
    rng = np.random.default_rng(7)
    P, kv, hd, heads = 16, 2, 8, 4
    k = fp16_exact(rng.standard_normal((3 * P + 5, kv, hd))).astype(np.float16)
    v = fp16_exact(rng.standard_normal((3 * P + 5, kv, hd))).astype(np.float16)
    tiers = [quant.INT4, quant.FP16, quant.INT8]
    pages = []
    for p, t in enumerate(tiers):
        kp, vp = k[p * P:(p + 1) * P], v[p * P:(p + 1) * P]
        pages.append(quant.fp16_page(kp, vp) if t == quant.FP16
                     else quant.quantise_page(kp, vp, t, P))
    q = fp16_exact(rng.standard_normal((1, heads, hd)))
    out, mass = att.causal_decode(q, pages, tiers, k[3 * P:], v[3 * P:], kv, hd, P)
    kk, vv = [], []
    for p, t in enumerate(tiers):
        if t == quant.FP16:
            kk.append(k[p * P:(p + 1) * P]); vv.append(v[p * P:(p + 1) * P])
        else:
            a, b = quant.dequantise_page(pages[p], t, kv, hd, P)
            kk.append(a); vv.append(b)
    K = np.concatenate(kk + [k[3 * P:]]).astype(np.float64)
    V = np.concatenate(vv + [v[3 * P:]]).astype(np.float64)
    want, w = att.attention64(q, K, V)
    np.testing.assert_allclose(out, want, rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(mass, att.page_mass(w[:, 0], P), rtol=1e-12, atol=1e-15)
    assert mass.shape == (heads, 4)


def test_error_bound_is_the_reference_formula_by_hand():
    """attention_bound (tests/test_attention.py:58-107) on a case worked by
    hand: two visible keys with equal scores (weights 1/2 each), so terms =
    (|v0| + |v1|) / 2 per channel and the largest score term is the bigger
    of sum_d |q_d k_jd| / sqrt(hd); a third key past the query is masked and
    must not count."""
    hd = 4
    q = np.array([[[1.0, -2.0, 0.5, 0.0]]])
    k = np.array([[[1.0, 0.0, 0.0, 0.0]], [[1.0, 0.0, 0.0, 0.0]], [[9.0, 9.0, 9.0, 9.0]]])
    v = np.array([[[1.0, -3.0, 0.0, 2.0]], [[-1.0, 1.0, 4.0, 0.0]], [[100.0] * 4]])
    out, w = att.attention64(q, k, v, positions=np.array([1]))
    assert np.allclose(w[0, 0], [0.5, 0.5, 0.0])
    bound = att.attention_bound(q, k, v, w, positions=np.array([1]))
    terms = (np.abs(v[0, 0]) + np.abs(v[1, 0])) / 2
    score_terms = max(np.abs(q[0, 0] * k[0, 0]).sum(), np.abs(q[0, 0] * k[1, 0]).sum()) / 2.0
    want = (np.sqrt(2) + np.sqrt(hd) * score_terms) * 2.0**-24 * terms
    np.testing.assert_allclose(bound[0, 0], want, rtol=1e-12)


def test_causal_chunk_is_each_query_decoded_alone_and_plain_attention_at_fp16():
    """A chunk's query at position x is causal_decode of that query over the
    pages before its own and its own page's rows up to x; over FP16 pages the
    whole chunk is plain causal attention over the rows. A chunk that begins
    mid-page and crosses two page boundaries, an unread page among them."""
    rng = np.random.default_rng(11)
    P, kv, hd, heads = 16, 2, 8, 4
    seq_k, seq_q = 4 * P + 3, 2 * P + 9            # positions 26 .. 66: own pages 1 .. 4
    k = fp16_exact(rng.standard_normal((seq_k, kv, hd))).astype(np.float16)
    v = fp16_exact(rng.standard_normal((seq_k, kv, hd))).astype(np.float16)
    q = fp16_exact(rng.standard_normal((seq_q, heads, hd)))
    bias = fp16_exact(3 * rng.standard_normal((kv, hd)))
    tiers = [quant.INT2, quant.UNREAD, quant.INT8, quant.INT4]
    pages = []
    for p, t in enumerate(tiers):
        kp, vp = k[p * P:(p + 1) * P], v[p * P:(p + 1) * P]
        pages.append(quant.fp16_page(kp, vp) if t in (quant.FP16, quant.UNREAD)
                     else quant.quantise_page(kp, vp, t, P))
    out, bound = att.causal_chunk(q, pages, tiers, k, v, kv, hd, P, bias, 1e4, with_bound=True)
    assert out.shape == bound.shape == q.shape and np.all(bound > 0)
    for i in range(seq_q):
        x = seq_k - seq_q + i
        own = x // P
        want, _ = att.causal_decode(q[i:i + 1], pages[:own], tiers[:own], k[own * P:x + 1],
                                    v[own * P:x + 1], kv, hd, P, bias, 1e4)
        np.testing.assert_allclose(out[i:i + 1], want, rtol=1e-12, atol=1e-14, err_msg=f"query {i}")
    fp16 = [quant.fp16_page(k[p * P:(p + 1) * P], v[p * P:(p + 1) * P]) for p in range(4)]
    plain = att.causal_chunk(q, fp16, [quant.FP16] * 4, k, v, kv, hd, P)
    want, _ = att.attention64(q, k, v)
    np.testing.assert_allclose(plain, want, rtol=1e-12, atol=1e-14)
