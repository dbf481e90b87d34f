"""The allocation-free decode entry point, mi_attention_paged_causal_noalloc,
against the entry point it is a variant of, mi_attention_paged_causal (given
a partials buffer, so both split across pages), through the C ABI: outputs,
masses and folded scores to the bit, on two calls in a row, the second over a
smaller cache; both against the float64 oracle at the 1e-3 bar; and a decode
whose scratch would not fit is refused with nothing written.

GPU test. The caches here are built by hand: pages quantised by the oracle on
the host, uploaded, and a page table of their device addresses."""

import ctypes as C

import numpy as np
import pytest

from conftest import announce, assert_attention_close, assert_mass_close, fp16_exact
from oracle import attention as att
from oracle import quant

pytestmark = pytest.mark.gpu

P = 32


def mi():
    from microinfer import _microinfer
    return _microinfer


class Cache:
    """A causal cache of one layer on the device, by hand: `own` sealed pages
    (tiers cycling through all four) in one device allocation with their
    address and tier tables, the own page's rows before the query in an FP16
    open page, and the query's own row."""

    def __init__(self, heads, kv, hd, seq, seed):
        m = mi()
        rng = np.random.default_rng(seed)
        self.heads, self.kv, self.hd, self.seq = heads, kv, hd, seq
        k = fp16_exact(rng.standard_normal((seq, kv, hd)))
        v = fp16_exact(rng.standard_normal((seq, kv, hd)))
        k[:, :, rng.choice(hd, 2, replace=False)] *= 10
        self.k, self.v = fp16_exact(k), fp16_exact(v)
        self.q = fp16_exact(rng.standard_normal((1, heads, hd)))
        self.own = (seq - 1) // P
        self.tiers = [(1, 0, 3, 2)[i % 4] for i in range(self.own)]
        self.raw = []
        for i, t in enumerate(self.tiers):
            kp = self.k[i * P:(i + 1) * P].astype(np.float16)
            vp = self.v[i * P:(i + 1) * P].astype(np.float16)
            self.raw.append(quant.fp16_page(kp, vp) if t == 0 else quant.quantise_page(kp, vp, t, P))
        # Pages at 256-byte-aligned offsets of one allocation.
        offsets, at = [], 0
        for r in self.raw:
            offsets.append(at)
            at += -(-len(r) // 256) * 256
        self.pages = m._Storage(max(at, 256))
        for r, o in zip(self.raw, offsets):
            m._h2d(self.pages.ptr + o, np.asarray(r, np.uint8))
        base = self.pages.ptr
        table = np.array([base + o for o in offsets] or [base], np.uint64)
        self.table = m._Storage(table.nbytes)
        m._h2d(self.table.ptr, table)
        tiers = np.array(self.tiers or [0], np.uint8)
        self.tier_table = m._Storage(max(tiers.nbytes, 16))
        m._h2d(self.tier_table.ptr, tiers)
        open_page = np.zeros((2 * P, kv * hd), np.float16)
        rows = self.k[self.own * P:seq - 1].reshape(-1, kv * hd)
        open_page[:len(rows)] = rows
        open_page[P:P + len(rows)] = self.v[self.own * P:seq - 1].reshape(-1, kv * hd)
        self.open = m.upload_fp16(open_page.astype(np.float32))
        self.q_dev = m.upload_fp16(self.q)
        self.ck = m.upload_fp16(self.k[-1:])
        self.cv = m.upload_fp16(self.v[-1:])
        self.pages_total = self.own + 1

    def oracle(self):
        return att.causal_decode(self.q, self.raw, self.tiers, self.k[self.own * P:],
                                 self.v[self.own * P:], self.kv, self.hd, P, with_bound=True)


def run(cache, noalloc, scores):
    """One decode through the C ABI; returns (out, mass)."""
    m = mi()
    d = m.device
    out = d.empty(cache.heads * cache.hd)
    mass = d.empty_f32(cache.heads * cache.pages_total)
    args = (C.c_void_p(cache.q_dev.address), C.c_void_p(cache.table.ptr),
            C.c_void_p(cache.tier_table.ptr), 0b1111, C.c_void_p(cache.open.address),
            C.c_void_p(cache.ck.address), C.c_void_p(cache.cv.address), P)
    if noalloc:
        status = m.lib.mi_attention_paged_causal_noalloc(
            *args, C.c_void_p(out.address), cache.seq, cache.heads, cache.kv, cache.hd,
            C.c_void_p(mass.address), C.c_void_p(scores), C.c_float(0.2), None)
    else:
        partials = d.empty_f32(d.attention_partials(cache.hd))
        status = m.lib.mi_attention_paged_causal(
            *args, None, None, 0, C.c_void_p(out.address), 1, cache.seq, cache.heads, cache.kv,
            cache.hd, C.c_void_p(mass.address), C.c_void_p(scores), C.c_float(0.2),
            C.c_void_p(partials.address), None)
    m._check(status)
    m.synchronize()
    return (out.to_numpy().reshape(1, cache.heads, cache.hd),
            mass.to_numpy().reshape(cache.heads, cache.pages_total))


def test_no_alloc_decode_is_the_allocating_one_twice_in_a_row():
    d = mi().device
    # The second call is over a smaller cache than the first.
    for heads, kv, hd, seq in ((12, 2, 128, P * 300 + 17), (12, 2, 128, P * 9 + 5),
                               (32, 8, 64, P * 40 + 1)):
        announce("no-alloc decode", heads, kv, hd, seq)
        cache = Cache(heads, kv, hd, seq, seed=seq)
        got_scores = d.ImportanceScores(1, cache.pages_total)
        want_scores = d.ImportanceScores(1, cache.pages_total)
        got, got_mass = run(cache, True, got_scores.row(0))
        want, want_mass = run(cache, False, want_scores.row(0))
        np.testing.assert_array_equal(got, want)
        np.testing.assert_array_equal(got_mass, want_mass)
        np.testing.assert_array_equal(got_scores.download(), want_scores.download())
        ref, ref_mass, bound = cache.oracle()
        assert_attention_close(got, ref, f"no-alloc {heads}x{kv}x{hd} seq {seq}", bound)
        assert_mass_close(got_mass, ref_mass, "no-alloc mass")


def test_a_decode_beyond_the_scratch_is_refused():
    """A cache whose page statistics alone exceed the 8 MiB scratch: the call
    fails with ValueError before any launch, and the output is untouched."""
    m = mi()
    d = m.device
    heads, kv, hd = 16, 1, 64
    seq = 70000 * P            # 16 heads x 70,000 pages x 2 floats > 2M floats
    out = d.empty(heads * hd)
    before = out.to_numpy().copy()
    q = m.upload_fp16(np.zeros((heads, hd), np.float32))
    rows = m.upload_fp16(np.zeros((2 * P, kv * hd), np.float32))
    # Every table entry names the one valid FP16 page, at tier FP16.
    table = m._Storage(8 * (seq // P))
    m._h2d(table.ptr, np.full(seq // P, rows.address, np.uint64))
    tiers = m._Storage(seq // P)
    m._h2d(tiers.ptr, np.zeros(seq // P, np.uint8))
    announce("no-alloc refusal")
    status = m.lib.mi_attention_paged_causal_noalloc(
        C.c_void_p(q.address), C.c_void_p(table.ptr), C.c_void_p(tiers.ptr), 1,
        C.c_void_p(rows.address), C.c_void_p(rows.address), C.c_void_p(rows.address), P,
        C.c_void_p(out.address), seq, heads, kv, hd, None, None, C.c_float(0.2), None)
    with pytest.raises(ValueError, match="scratch"):
        m._check(status)
    np.testing.assert_array_equal(out.to_numpy(), before)
