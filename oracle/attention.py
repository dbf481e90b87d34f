"""Attention over the KV cache, and each page's share of it, in float64.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Follows the reference:
  - attention:   tests/test_attention.py:54-107 (float64 causal softmax with
                 bottom-right alignment and HuggingFace repeat_kv GQA order),
                 the kernel it checks being src/core_kernels/attention.cu:449-746
  - key bias:    tests/test_attention.py:338-348 (k + RoPE(k_bias, j), rotate
                 half, complex form), attention.cu:104-116
  - causal view: tests/test_quantised_pages.py:55-105 (pages before a query's
                 own read at the tier the page table records, dequantised as
                 dequantise_page returns them; the own page's rows as they
                 came), attention.cu:302-364
  - unread page: attention.cu:326-360, device_ops.h:91-96 (a page whose tier
                 is 0xFF is masked like a future position and contributes no
                 mass)
  - page mass:   tests/test_attention_mass.py:68-86 and
                 tests/test_split_attention.py:234-249 (each head's softmax
                 summed over each page's keys)

PINNED by (tests/test_oracle_attention.py): brute force against a plain
Python double loop on tiny inputs (explicit mask, explicit group index);
invariants (each head's weights and masses sum to 1; a masked or unread
key gets weight 0; GQA with group 1 equals multi-head; one key gives v);
the key bias pinned against completing the keys by hand with a scalar
cos/sin rotation; mass per page against the weights of the attention call.
"""

from __future__ import annotations

import numpy as np

from . import quant


def expand_kv(heads: int, kv: np.ndarray) -> np.ndarray:
    """Query head h reads KV head h // (heads / kv_heads): contiguous groups
    (attention.cu:85-90)."""
    return np.repeat(kv, heads // kv.shape[1], axis=1)


def rotated_bias(bias: np.ndarray, seq_k: int, theta: float) -> np.ndarray:
    """RoPE of the key bias at every key position, rotate-half pairing:
    (seq_k, kv_heads, head_dim) float64 (tests/test_attention.py:338-348)."""
    half = bias.shape[-1] // 2
    inv_freq = theta ** (-np.arange(half, dtype=np.float64) * 2.0 / bias.shape[-1])
    rot = np.exp(1j * np.arange(seq_k)[:, None] * inv_freq)[:, None, :]
    b = np.asarray(bias, np.float64)
    z = (b[..., :half] + 1j * b[..., half:])[None] * rot
    return np.concatenate([z.real, z.imag], axis=-1)


def attention64(q, k, v, k_bias=None, theta: float = 0.0, unread=None, positions=None):
    """float64 softmax(q k^T / sqrt(d) + mask) v for q (seq_q, heads, hd)
    and k, v (seq_k, kv_heads, hd); queries bottom-right aligned unless
    `positions` names them. `unread`, a bool per key, masks keys as the
    causal layout masks an unread page's. Returns (out, weights) with
    weights (heads, seq_q, seq_k)."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    seq_q, heads, hd = q.shape
    seq_k = k.shape[0]
    if heads % k.shape[1] != 0:
        raise ValueError("the KV head count must divide the query head count")
    if k_bias is not None:
        k = k + rotated_bias(k_bias, seq_k, theta)
    if positions is None:
        positions = np.arange(seq_q) + (seq_k - seq_q)
    kk, vv = expand_kv(heads, k), expand_kv(heads, v)
    # Batched over heads: (h, q, d) @ (h, d, k), float64 throughout.
    scores = np.matmul(q.transpose(1, 0, 2), kk.transpose(1, 2, 0)) / np.sqrt(hd)
    masked = np.arange(seq_k)[None, :] > np.asarray(positions)[:, None]
    if unread is not None:
        masked = masked | np.asarray(unread, bool)[None, :]
    scores[:, masked] = -np.inf
    top = scores.max(axis=-1, keepdims=True)
    p = np.exp(scores - top)
    p /= p.sum(axis=-1, keepdims=True)
    out = np.matmul(p, vv.transpose(1, 0, 2)).transpose(1, 0, 2)
    return out, p


#: fp32's unit roundoff, and the smallest normal fp16: the two constants of
#: the reference's error gate (tests/ulp_gate.py:28-38).
FP32_REL_ULP = 2.0**-24
FP16_MIN_NORMAL = 6.103515625e-05


def attention_bound(q, k, v, weights, k_bias=None, theta: float = 0.0, unread=None,
                    positions=None):
    """Per output element, the absolute error an fp32-accumulating kernel
    may carry (tests/test_attention.py:58-107): the fp32 sum over the
    visible keys, sqrt(n) * u32 * terms with terms = sum_j p_j |v_j|, plus
    the fp32 scores' rounding, sqrt(hd) * u32 * (largest sum_d |q_d k_d| /
    sqrt(hd) over the visible keys), weighing the same terms. `weights` are
    attention64's. Returns (seq_q, heads, hd)."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    seq_q, heads, hd = q.shape
    seq_k = k.shape[0]
    if k_bias is not None:
        k = k + rotated_bias(k_bias, seq_k, theta)
    if positions is None:
        positions = np.arange(seq_q) + (seq_k - seq_q)
    positions = np.asarray(positions)
    kk, vv = expand_kv(heads, k), expand_kv(heads, v)
    terms = np.matmul(weights, np.abs(vv).transpose(1, 0, 2)).transpose(1, 0, 2)
    score_terms = np.matmul(np.abs(q).transpose(1, 0, 2),
                            np.abs(kk).transpose(1, 2, 0)) / np.sqrt(hd)
    masked = np.arange(seq_k)[None, :] > positions[:, None]
    if unread is not None:
        masked = masked | np.asarray(unread, bool)[None, :]
    score_terms[:, masked] = 0.0
    score_terms = score_terms.max(axis=-1).T[..., None]
    visible = (positions + 1)[:, None, None]
    return (np.sqrt(visible) + np.sqrt(hd) * score_terms) * FP32_REL_ULP * terms


def page_mass(weights: np.ndarray, page_tokens: int) -> np.ndarray:
    """(heads, seq_k) softmax weights of one query -> (heads, pages), each
    page's share (tests/test_attention_mass.py:68-86)."""
    heads, seq_k = weights.shape
    pages = -(-seq_k // page_tokens)
    padded = np.zeros((heads, pages * page_tokens))
    padded[:, :seq_k] = weights
    return padded.reshape(heads, pages, page_tokens).sum(axis=2)


def read_sealed(pages, tiers, kv_heads: int, head_dim: int, page_tokens: int):
    """The sealed pages of one layer as attention reads them: each page's
    bytes at the tier recorded for it, dequantised as dequantise_page returns
    them; an unread page (tier 0xFF) as zeros, flagged. Returns (K, V, unread)
    with K, V (n*P, kv, hd) float64 and unread a bool per key."""
    ks, vs, flags = [], [], []
    shape = (page_tokens, kv_heads, head_dim)
    for raw, tier in zip(pages, tiers):
        tier = int(tier)
        if tier == quant.UNREAD:
            k = v = np.zeros(shape)
            flags.append(np.ones(page_tokens, bool))
        else:
            if tier == quant.FP16:
                k, v = quant.read_fp16_page(raw, page_tokens, kv_heads, head_dim)
            else:
                k, v = quant.dequantise_page(raw, tier, kv_heads, head_dim, page_tokens)
            flags.append(np.zeros(page_tokens, bool))
        ks.append(np.asarray(k, np.float64))
        vs.append(np.asarray(v, np.float64))
    if not ks:
        empty = np.zeros((0, kv_heads, head_dim))
        return empty, empty, np.zeros(0, bool)
    return np.concatenate(ks), np.concatenate(vs), np.concatenate(flags)


def causal_decode(q, sealed_pages, tiers, own_k, own_v, kv_heads: int, head_dim: int,
                  page_tokens: int, k_bias=None, theta: float = 0.0, with_bound: bool = False):
    """One decode query over a cache that seals (tests/test_quantised_pages.py:86-105):
    the sealed pages before its own at their tiers, then its own page's rows
    as they came, `own_k`/`own_v` (n_own, kv, hd), the last of them the
    query's own position. Returns (out (1, heads, hd), mass (heads, pages)),
    and attention_bound's error bound third when `with_bound`."""
    K, V, unread = read_sealed(sealed_pages, tiers, kv_heads, head_dim, page_tokens)
    k = np.concatenate([K, np.asarray(own_k, np.float64)])
    v = np.concatenate([V, np.asarray(own_v, np.float64)])
    flags = np.concatenate([unread, np.zeros(len(own_k), bool)])
    out, w = attention64(q, k, v, k_bias, theta, unread=flags)
    mass = page_mass(w[:, -1, :], page_tokens)
    if not with_bound:
        return out, mass
    return out, mass, attention_bound(q, k, v, w, k_bias, theta, unread=flags)


def causal_chunk(q, sealed_pages, tiers, k_rows, v_rows, kv_heads: int, head_dim: int,
                 page_tokens: int, k_bias=None, theta: float = 0.0, with_bound: bool = False):
    """A chunk of queries, the last len(q) positions of the rows, over a cache
    that seals (tests/test_quantised_pages.py:86-104): the query at position
    x reads every page before its own at the tier recorded for it (the
    sealed pages' bytes) and its own page's rows as they came, k_rows and
    v_rows (seq_k, kv, hd) holding every position's rows. Returns out
    (seq_q, heads, hd), and attention_bound's error bound second when
    `with_bound`."""
    q = np.asarray(q, np.float64)
    k_rows = np.asarray(k_rows, np.float64)
    v_rows = np.asarray(v_rows, np.float64)
    seq_q = q.shape[0]
    seq_k = k_rows.shape[0]
    positions = np.arange(seq_k - seq_q, seq_k)
    owns = positions // page_tokens
    K, V, unread = read_sealed(sealed_pages, tiers, kv_heads, head_dim, page_tokens)
    out = np.zeros(q.shape)
    bound = np.zeros(q.shape)
    for own in np.unique(owns):
        rows = owns == own
        first = own * page_tokens
        last = positions[rows].max()
        k = np.concatenate([K[:first], k_rows[first:last + 1]])
        v = np.concatenate([V[:first], v_rows[first:last + 1]])
        flags = np.concatenate([unread[:first], np.zeros(last + 1 - first, bool)])
        o, w = attention64(q[rows], k, v, k_bias, theta, unread=flags, positions=positions[rows])
        out[rows] = o
        if with_bound:
            bound[rows] = attention_bound(q[rows], k, v, w, k_bias, theta, unread=flags,
                                          positions=positions[rows])
    return (out, bound) if with_bound else out


def attention_bruteforce(q, k, v):
    """A plain double loop, for tiny inputs only: the check on attention64."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    seq_q, heads, hd = q.shape
    seq_k, kv_heads, _ = k.shape
    group = heads // kv_heads
    out = np.zeros_like(q)
    for i in range(seq_q):
        pos = i + seq_k - seq_q
        for h in range(heads):
            kh = h // group
            s = [sum(q[i, h, d] * k[j, kh, d] for d in range(hd)) / hd ** 0.5
                 for j in range(pos + 1)]
            top = max(s)
            e = [np.exp(x - top) for x in s]
            tot = sum(e)
            for d in range(hd):
                out[i, h, d] = sum(e[j] * v[j, kh, d] for j in range(pos + 1)) / tot
    return out
