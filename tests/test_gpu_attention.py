"""Attention kernels against the float64 oracle: contiguous layout, GQA,
the key bias, causal masking, split-K.

GPU parity tests (tolerance: conftest.ATTN_MAX_REL, the reference's error gate
held to 1e-3)."""

import numpy as np
import pytest

from conftest import announce, assert_attention_close, each, fp16_exact
from oracle import attention as att
from oracle import pointwise

pytestmark = pytest.mark.gpu

SHAPES = {"qwen2.5-0.5b": (14, 2, 64, 1e6), "qwen2.5-1.5b": (12, 2, 128, 1e6),
          "llama-3.2-1b": (32, 8, 64, 5e5)}


def mi():
    from microinfer import _microinfer
    return _microinfer


def qkv(seq_q, seq_k, heads, kv_heads, hd, seed, scale=1.0):
    rng = np.random.default_rng(seed)
    return (fp16_exact(scale * rng.standard_normal((seq_q, heads, hd))),
            fp16_exact(rng.standard_normal((seq_k, kv_heads, hd))),
            fp16_exact(rng.standard_normal((seq_k, kv_heads, hd))))


def test_contiguous_attention_is_the_float64_reference():
    m = mi()

    def check(name, seq_q, seq_k):
        heads, kv, hd, _ = SHAPES[name]
        announce("attention", name, seq_q, seq_k)
        q, k, v = qkv(seq_q, seq_k, heads, kv, hd, seed=seq_q * 1000 + seq_k, scale=2.0)
        got = m.attention(q, k, v)
        want, w = att.attention64(q, k, v)
        assert_attention_close(got, want, f"{name} {seq_q}x{seq_k}", att.attention_bound(q, k, v, w))

    cases = [(n, sq, sk) for n in SHAPES for sq, sk in
             ((1, 1), (1, 31), (1, 32), (1, 33), (1, 700), (1, 4099), (16, 16), (17, 40),
              (37, 300))]
    each(cases, check)


def test_grouped_query_heads_read_their_own_kv_head():
    """Each KV head's values are a constant of its own: a query head's
    output is the constant of KV head h // group, whatever its scores."""
    m = mi()
    heads, kv, hd = 12, 3, 64
    rng = np.random.default_rng(1)
    q = fp16_exact(rng.standard_normal((1, heads, hd)))
    k = fp16_exact(rng.standard_normal((50, kv, hd)))
    v = np.zeros((50, kv, hd), np.float32)
    for h in range(kv):
        v[:, h, :] = h + 1
    got = m.attention(q, k, v)
    for h in range(heads):
        np.testing.assert_array_equal(got[0, h], np.full(hd, h // (heads // kv) + 1, np.float32))


def test_the_key_bias_completes_each_key():
    """k_bias (kv_heads, hd) completes key j as k + RoPE(k_bias, j)
    (reference attention.cu:104-116), against the whole key in float64."""
    m = mi()
    for name in ("qwen2.5-0.5b", "qwen2.5-1.5b"):
        heads, kv, hd, theta = SHAPES[name]
        for seq_q, seq_k in ((1, 99), (40, 40)):
            announce("key bias", name, seq_q, seq_k)
            rng = np.random.default_rng(seq_k)
            q = fp16_exact(rng.standard_normal((seq_q, heads, hd)))
            k = fp16_exact(0.3 * rng.standard_normal((seq_k, kv, hd)))
            v = fp16_exact(rng.standard_normal((seq_k, kv, hd)))
            bias = fp16_exact(3 * rng.standard_normal((kv, hd)))
            got = m.attention(q, k, v, k_bias=bias, theta=theta)
            want, w = att.attention64(q, k, v, k_bias=bias, theta=theta)
            assert_attention_close(got, want, f"bias {name}",
                                   att.attention_bound(q, k, v, w, k_bias=bias, theta=theta))


def test_attention_is_causal_and_a_nan_key_does_not_leak():
    """tests/test_attention.py:215-242: changing every key and value after
    position i moves no bit of query i's output; a NaN in a masked key does
    not leak; position 0 attends to itself alone."""
    m = mi()
    heads, kv, hd, _ = SHAPES["qwen2.5-0.5b"]
    rng = np.random.default_rng(2)
    for seq in (29, 69):
        q, k, v = qkv(seq, seq, heads, kv, hd, seed=1)
        base = m.attention(q, k, v)
        for i in (0, 1, 16, seq - 2):
            announce("causal", seq, i)
            k2, v2 = k.copy(), v.copy()
            k2[i + 1:] = fp16_exact(1000 * rng.standard_normal(k2[i + 1:].shape))
            v2[i + 1:] = fp16_exact(1000 * rng.standard_normal(v2[i + 1:].shape))
            moved = m.attention(q, k2, v2)
            np.testing.assert_array_equal(moved[:i + 1], base[:i + 1])
            assert not np.array_equal(moved[i + 1:], base[i + 1:])
    q, k, v = qkv(41, 41, heads, kv, hd, seed=5)
    base = m.attention(q, k, v)
    k2 = k.copy()
    k2[-1] = np.nan
    np.testing.assert_array_equal(m.attention(q, k2, v)[:-1], base[:-1])
    q, k, v = qkv(3, 3, heads, kv, hd, seed=6)
    np.testing.assert_array_equal(m.attention(q, k, v)[0], np.repeat(v[0], heads // kv, axis=0))


def test_split_launches_match_the_reference_and_the_unsplit_one():
    """A long decode launch splits its keys into runs (device.attention with
    partials); without partials it does not. Both are the reference."""
    m = mi()
    d = m.device
    heads, kv, hd, _ = SHAPES["qwen2.5-1.5b"]
    seq_k = 5000
    splits, keys = d.attention_split(1, seq_k, heads, kv, 0)
    assert splits > 1, "the case must split"
    q, k, v = qkv(1, seq_k, heads, kv, hd, seed=9)
    want, w = att.attention64(q, k, v)
    bound = att.attention_bound(q, k, v, w)
    outs = []
    for partials in (d.empty_f32(d.attention_partials(hd)), None):
        announce("split", partials is not None)
        out = d.empty(q.size)
        d.attention(m.upload_fp16(q), m.upload_fp16(k), m.upload_fp16(v), None, None, out, 1,
                    seq_k, heads, kv, hd, partials)
        outs.append(out.to_numpy().reshape(q.shape))
        assert_attention_close(outs[-1], want, "split" if partials else "unsplit", bound)


def test_rope_rmsnorm_swiglu_are_the_float64_references():
    m = mi()
    rng = np.random.default_rng(0)
    # RoPE: positions past 2048 and at the end of the window (tests/test_rope.py:30-41).
    for heads, hd in ((14, 64), (2, 128)):
        announce("rope", heads, hd)
        pos = np.array([0, 1, 31, 2047, 2049, 16384, 32767], np.int32)
        x = fp16_exact(rng.standard_normal((len(pos), heads, hd)))
        got = m.rope(x, pos, 1e6)
        want = pointwise.rope(x, pos, 1e6)
        ulp = np.spacing(np.abs(want).astype(np.float16)).astype(np.float64)
        assert np.all(np.abs(got - want) <= 2 * ulp + 1e-6 * np.abs(x).max())
    # Eight values a thread (hidden a multiple of 8) and one a thread (1001).
    for hidden in (896, 2048, 1001):
        announce("rmsnorm", hidden)
        x = fp16_exact(rng.standard_normal((3, hidden)))
        w = fp16_exact(rng.uniform(0.5, 1.5, hidden))
        got = m.rmsnorm(x, w, 1e-6)
        want = pointwise.rmsnorm(x, w, 1e-6)
        ulp = np.spacing(np.abs(want).astype(np.float16)).astype(np.float64)
        assert np.all(np.abs(got - want) <= ulp)
    # SwiGLU eight values a thread (a multiple of 8) and one a thread.
    for shape in ((2, 8192), (3, 1001)):
        announce("swiglu", shape)
        g = fp16_exact(4 * rng.standard_normal(shape))
        u = fp16_exact(rng.standard_normal(shape))
        got = m.swiglu(g, u)
        want = pointwise.swiglu(g, u)
        ulp = np.spacing(np.abs(want).astype(np.float16)).astype(np.float64)
        assert np.all(np.abs(got - want) <= ulp)


def test_rope_table_is_fp64_cos_sin_rounded():
    m = mi()
    t = m.device.RopeTable(128, 1e6)
    t.cover(3000)
    table = t.to_numpy()
    assert table.shape[0] >= 3000
    pos = np.arange(table.shape[0])[:, None]
    inv = 1e6 ** (-np.arange(64) * 2.0 / 128)
    ang = pos * inv[None, :]
    for got, want in ((table[..., 0], np.cos(ang)), (table[..., 1], np.sin(ang))):
        ulp = np.spacing(np.abs(want).astype(np.float32)).astype(np.float64)
        assert np.all(np.abs(got - want) <= ulp)


def test_rope_from_a_table_is_the_rope_kernel_to_the_bit():
    """RoPE with its angles read from a RopeTable (what the prefill runs)
    gives the RoPE kernel's rows bit for bit, head dims 64 and 128, positions
    across the table; both are within the float64 reference's bound."""
    m = mi()
    d = m.device
    rng = np.random.default_rng(4)
    for heads, hd in ((32, 64), (12, 128)):
        announce("rope from table", heads, hd)
        pos = np.array([0, 1, 31, 32, 2047, 4096, 16383, 32767, 5, 32766], np.int32)
        x = fp16_exact(rng.standard_normal((len(pos), heads, hd)))
        table = d.RopeTable(hd, 1e6)
        table.cover(32768)
        at = d.DeviceIndex(pos)
        xs = m.upload_fp16(x.reshape(-1))
        a, b = d.empty(x.size), d.empty(x.size)
        d.rope(xs, at, a, len(pos), heads, hd, 1e6)
        d.rope_from_table(xs, at, table, b, len(pos), heads, hd)
        np.testing.assert_array_equal(b.to_numpy(), a.to_numpy())
        want = pointwise.rope(x, pos, 1e6)
        ulp = np.spacing(np.abs(want).astype(np.float16)).astype(np.float64)
        got = b.to_numpy().reshape(x.shape)
        assert np.all(np.abs(got - want) <= 2 * ulp + 1e-6 * np.abs(x).max())


def test_the_general_path_takes_what_the_fast_kernels_do_not():
    """Head dims 96 and 80 (neither fast kernel's), contiguous, one query
    and a chunk, with the key bias; a long decode split into runs and not;
    and a cache of 48-token FP16 pages decoding with per-page mass: all
    against the float64 oracle."""
    from conftest import assert_mass_close
    from test_gpu_kv_pages import page_sizes, put
    m = mi()
    d = m.device
    rng = np.random.default_rng(31)
    for hd in (96, 80):
        heads, kv = 8, 2
        for seq_q, seq_k in ((1, 700), (9, 300)):
            announce("general", hd, seq_q, seq_k)
            q, k, v = qkv(seq_q, seq_k, heads, kv, hd, seed=hd + seq_k)
            bias = fp16_exact(2 * rng.standard_normal((kv, hd)))
            got = m.attention(q, k, v, k_bias=bias, theta=1e4)
            want, w = att.attention64(q, k, v, k_bias=bias, theta=1e4)
            assert_attention_close(got, want, f"general hd {hd} {seq_q}x{seq_k}",
                                   att.attention_bound(q, k, v, w, k_bias=bias, theta=1e4))
        seq_k = 5000
        q, k, v = qkv(1, seq_k, heads, kv, hd, seed=hd)
        want, w = att.attention64(q, k, v)
        for partials in (d.empty_f32(d.attention_partials(hd)), None):
            announce("general split", hd, partials is not None)
            out = d.empty(q.size)
            d.attention(m.upload_fp16(q), m.upload_fp16(k), m.upload_fp16(v), None, None, out, 1,
                        seq_k, heads, kv, hd, partials)
            assert_attention_close(out.to_numpy().reshape(q.shape), want, f"split hd {hd}",
                                   att.attention_bound(q, k, v, w))
    P, heads, kv, hd = 48, 12, 2, 128
    seq = P * 20 + 7
    pages = -(-seq // P)
    alloc = m.PagedKVCache(page_sizes(P, kv, hd), [64] * 4)
    cache = d.KVPages(alloc, 1, P, kv, hd, 0, d.Halves.Both, [], False)
    q, k, v = qkv(1, seq, heads, kv, hd, seed=48)
    cache.reserve(seq)
    cache.store(0, put(k), put(v), 0, seq)
    want, w = att.attention64(q, k, v)
    for partials in (d.empty_f32(d.attention_partials(hd)), None):
        announce("48-token pages", partials is not None)
        out, mass = d.empty(heads * hd), d.empty_f32(heads * pages)
        cache.attention(0, put(q), None, None, out, 1, seq, heads, kv, hd, None, None, mass,
                        partials)
        assert_attention_close(out.to_numpy().reshape(1, heads, hd), want, "48-token pages",
                               att.attention_bound(q, k, v, w))
        assert_mass_close(mass.to_numpy().reshape(heads, pages), att.page_mass(w[:, -1, :], P),
                          "48-token page mass")
