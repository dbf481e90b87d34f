"""The dense projections (hipBLASLt), the embedding gather and the greedy
argmax on the device, against the float64 oracle (tests/test_linear.py).

GPU parity tests: projections within the reference's ulp gate with the fp32
accumulation floor; fp32 outputs (logits, the accumulate form) within the
fp32 accumulation bound itself; the gather bit for bit; the argmax to the
index, ties to the lowest."""

import math

import numpy as np
import pytest

from conftest import accumulation_floor, announce, assert_within_gate, each, fp16_exact
from oracle import dense

pytestmark = pytest.mark.gpu

#: (hidden, kv_width, intermediate) of the three model shapes the configs name:
#: Qwen2.5-0.5B, Qwen2.5-1.5B, Llama-3.2-1B.
MODELS = {"qwen0.5b": (896, 128, 4864), "qwen1.5b": (1536, 256, 8960),
          "llama1b": (2048, 512, 8192)}


def mi():
    from microinfer import _microinfer
    return _microinfer


def projections(hidden, kv, inter, bias):
    return {"q_proj": (hidden, hidden, bias), "k_proj": (hidden, kv, bias),
            "v_proj": (hidden, kv, bias), "o_proj": (hidden, hidden, False),
            "gate_proj": (hidden, inter, False), "up_proj": (hidden, inter, False),
            "down_proj": (inter, hidden, False)}


def make_case(rows, in_f, out_f, bias, seed=0):
    rng = np.random.default_rng(seed)
    x = fp16_exact(rng.standard_normal((rows, in_f)))
    w = fp16_exact(rng.standard_normal((out_f, in_f)) / math.sqrt(max(in_f, 1)))
    b = fp16_exact(rng.standard_normal(out_f)) if bias else None
    return x, w, b


def within_gate(got, x, w, b=None, what=""):
    want, terms = dense.linear(x, w, b)
    n = x.shape[1] + (b is not None)
    return assert_within_gate(got, want, accumulation_floor(terms, n), what)


def check(x, w, b):
    announce("linear", x.shape, w.shape, b is not None)
    within_gate(mi().linear(x, w, b), x, w, b, f"{x.shape} x {w.shape}")


def test_every_projection_shape_at_decode_and_prefill_rows():
    cases = []
    for name, (hidden, kv, inter) in MODELS.items():
        for proj, (in_f, out_f, bias) in projections(hidden, kv, inter,
                                                     name.startswith("qwen")).items():
            for rows in (1, 64):
                cases.append((rows, in_f, out_f, bias, in_f + out_f + rows))
    cases += [(3, 5, 7, True, 1), (1, 1, 1, True, 2), (17, 33, 65, True, 3), (2, 896, 3, True, 4),
              (4, 896, 151936 // 8, False, 11)]
    each(cases, lambda rows, in_f, out_f, bias, seed: check(*make_case(rows, in_f, out_f, bias,
                                                                        seed)))


def test_the_weight_is_out_by_in_the_bias_added_once_and_rows_independent():
    m = mi()
    x, w, _ = make_case(4, 128, 128, False)
    got = m.linear(x, w)
    within_gate(got, x, w)
    assert not np.allclose(got, x.astype(np.float64) @ w.astype(np.float64), atol=1e-2)
    x, w, b = make_case(5, 64, 32, True)
    with_bias = m.linear(x, w, b)
    within_gate(with_bias, x, w, b)
    assert not np.array_equal(with_bias, m.linear(x, w))
    x, w, b = make_case(16, 256, 96, True)
    all_rows = m.linear(x, w, b)
    for i in (0, 9, 15):
        within_gate(m.linear(x[i:i + 1].copy(), w, b), x[i:i + 1], w, b)
        within_gate(all_rows[i:i + 1], x[i:i + 1], w, b)


def test_malformed_operands_are_refused():
    m = mi()
    x, w, b = make_case(2, 64, 32, True)
    with pytest.raises(ValueError, match="64"):
        m.linear(x, w[:, :48].copy())
    with pytest.raises(ValueError, match="32"):
        m.linear(x, w, b[:16].copy())
    with pytest.raises(ValueError):
        m.linear(np.zeros(64, np.float32), w)
    d = m.device
    out = d.empty(2 * 32)
    with pytest.raises(ValueError, match="weight"):
        d.linear(m.upload_fp16(x), m.upload_fp16(w[:16]), None, out, 2, 64, 32)


def test_device_linear_and_the_fp32_accumulate_form():
    m = mi()
    d = m.device
    rows, in_f, out_f = 8, 2048, 8192
    x, w, b = make_case(rows, in_f, out_f, True, seed=5)
    dx, dw, db = m.upload_fp16(x), m.upload_fp16(w), m.upload_fp16(b)
    out = d.empty(rows * out_f)
    announce("device.linear", rows, in_f, out_f)
    d.linear(dx, dw, db, out, rows, in_f, out_f)
    within_gate(out.to_numpy().reshape(rows, out_f), x, w, b)
    # out += x W^T in fp32 onto a residual: never rounded to fp16.
    rng = np.random.default_rng(6)
    residual = rng.standard_normal((rows, out_f)).astype(np.float32)
    acc = d.upload_f32(residual)
    announce("linear_accumulate", rows, in_f, out_f)
    d.linear_accumulate(dx, dw, acc, rows, in_f, out_f)
    want, terms = dense.linear(x, w)
    want += residual
    terms += np.abs(residual)
    got = acc.to_numpy().reshape(rows, out_f).astype(np.float64)
    bound = math.sqrt(in_f + 1) * 2.0**-24 * terms
    assert np.all(np.abs(got - want) <= bound), np.max(np.abs(got - want) / bound)
    # Twice: the second adds onto the first.
    d.linear_accumulate(dx, dw, acc, rows, in_f, out_f)
    got2 = acc.to_numpy().reshape(rows, out_f).astype(np.float64)
    assert np.all(np.abs(got2 - (want + dense.linear(x, w)[0])) <= 2 * bound + 2.0**-23 * np.abs(got2))


def test_embed_gathers_bit_for_bit_and_zeroes_unknown_ids():
    m = mi()
    d = m.device
    vocab, hidden = 1000, 2048
    rng = np.random.default_rng(7)
    table = rng.standard_normal((vocab, hidden)).astype(np.float16)
    dt = m.upload_fp16(table.astype(np.float32))
    ids = np.array([5, 999, 0, -1, 1000, 5, 123], np.int32)
    di = d.index(ids)
    announce("embed", len(ids), hidden)
    out = d.empty(len(ids) * hidden)
    d.embed(di, dt, out, hidden, vocab)
    want = dense.embed(ids, table)
    np.testing.assert_array_equal(out.to_numpy().reshape(len(ids), hidden).astype(np.float16),
                                  want)
    out32 = d.empty_f32(len(ids) * hidden)
    d.embed_f32(di, dt, out32, hidden, vocab)
    np.testing.assert_array_equal(out32.to_numpy().reshape(len(ids), hidden),
                                  want.astype(np.float32))


def test_logits_and_greedy():
    m = mi()
    d = m.device
    rows, hidden, vocab = 5, 896, 4099
    x, w, _ = make_case(rows + 2, hidden, vocab, False, seed=9)
    w[7] = w[3]                       # logits 3 and 7 equal in every row
    x[2] = 0.0                        # every logit of output row 1 (x row 2) is 0: index 0
    dx, dh = m.upload_fp16(x), m.upload_fp16(w)
    scratch = d.empty(d.scratch_elements(rows, vocab))
    announce("logits", rows, hidden, vocab)
    got = d.logits(dx, dh, scratch, 1, rows, hidden, vocab)
    want, terms = dense.linear(x[1:1 + rows], w)
    bound = math.sqrt(hidden) * 2.0**-24 * terms
    assert got.dtype == np.float32 and got.shape == (rows, vocab)
    assert np.all(np.abs(got - want) <= bound + 1e-30)
    ids = d.greedy(dx, dh, scratch, 1, rows, hidden, vocab)
    np.testing.assert_array_equal(ids, dense.argmax_rows(got))
    assert ids[1] == 0
    # A row that cannot fit its scratch, and one with no finite logit.
    with pytest.raises(ValueError, match="scratch"):
        d.greedy(dx, dh, d.empty(10), 0, rows, hidden, vocab)
    bad = x.copy()
    bad[0, 0] = np.inf
    w_nan = w.copy()
    w_nan[:, 0] = 0.0                 # inf * 0 = NaN in every logit of row 0
    with pytest.raises(RuntimeError, match="no finite logit"):
        d.greedy(m.upload_fp16(bad), m.upload_fp16(w_nan), scratch, 0, 1, hidden, vocab)
    assert m.cuda_driver_version() > 0
