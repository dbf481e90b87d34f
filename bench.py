"""Benchmark of the paged mixed-precision KV-cache hot path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1]

The step (the headline workload, config 3): one decode token's attention
over every layer of a Qwen2.5-1.5B-shaped cache at 32K positions -- 28
layers, 12 query / 2 KV heads, head_dim 128, 32-token pages born at
seeded-importance tiers 20% FP16, 30% INT8, 40% INT4, 10% INT2 -- one launch
pair a layer, in layer order as a decode step visits them, each keeping its
page statistics, then one launch that forms every layer's per-page attention
mass and folds it into the importance scores (EWMA): the same bits as folding
a layer at a time. The 57 launches are captured once in a HIP graph and
replayed; K steps are timed with hipEvents on the stream they run on. Inputs
are resident in HBM before timing starts.

Also measured, outside the timed region: the same step with the fold fused
into each layer, in one launch over all layers, and with the key bias;
config 2 (0.5B, 8K, all FP16: RMSNorm, RoPE, store and decode a layer);
whole decode steps (every projection, the paged decode, the head and the
greedy token, one graph a token) at the 1.5B shape at 32K and the Llama-3.2-1B
shape at 16K; the requantisation plan of config 4 against its host-link
bound; the prefill attention; and the CPU reference path (the oracle) on the
configuration-1 pass and a config-3 layer. Prints one JSON line.
"""

from __future__ import annotations

import argparse
import faulthandler
import hashlib
import json
import os
import statistics
import sys
import time
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent
PKG = REPO / "semantic-aware_adaptive_kv_cache_precision_amd"
sys.path.insert(0, str(PKG))
sys.path.insert(0, str(REPO))

METRIC = "mixed-tier decode-attn GB/s (% HBM peak) & µs/token @32K; requant pages/s"
PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0  # dense fp16 / bf16
P = 32
TRAFFIC_PROFILE = REPO / "profiles" / "decode_attention_config3_hbm_bytes.md"


def log(*what) -> None:
    print("[bench]", *what, file=sys.stderr, flush=True)


def tier_sizes(m, shape):
    return [m.device.page_bytes(P, shape.kv_width)] + [
        m.quantised_page_layout(t, shape.kv_heads, shape.head_dim, P)["page_bytes"]
        for t in (1, 2, 3)]


def sealing_cache(m, shape, layers, pages, tier_map):
    cap = [layers * pages + 2 * layers + 8] * 4
    alloc = m.PagedKVCache(tier_sizes(m, shape), cap)
    cache = m.device.KVPages(alloc, layers, P, shape.kv_heads, shape.head_dim, m.Tier.FP16,
                             m.device.Halves.Both, tier_map, True)
    return alloc, cache


def fill_rows(m, cache, shape, layers, positions, rng, keep_last=False):
    """Every layer's first `positions` rows stored, seeded N(0,1) fp16 with
    outlier key channels; with keep_last, each layer's rows kept on the host."""
    from microinfer import workloads as w
    outliers = w.outlier_channels(rng, shape.kv_width)
    cache.reserve(positions)
    kept = []
    for layer in range(layers):
        k, v = w.kv_rows(rng, positions, shape, outliers)
        cache.store(layer, m.upload_fp16(k.astype(np.float32)), m.upload_fp16(v.astype(np.float32)),
                    0, positions)
        if keep_last:
            kept.append((k, v))
    m.synchronize()
    return kept


def build_config3(m, shape, context, layers, seed=0):
    """The config-3 cache: every layer's rows before the query's stored
    (pages sealed at their birth tiers), then each layer's decode row."""
    from microinfer import workloads as w
    sealed = context // P - 1
    tier_map = w.tier_map(seed, layers, sealed, w.MIX_CONFIG3)
    alloc, cache = sealing_cache(m, shape, layers, sealed + 1, tier_map)
    rng = np.random.default_rng(seed)
    host = fill_rows(m, cache, shape, layers, context - 1, rng, keep_last=True)
    cache.reserve(context)
    rows = []
    for layer in range(layers):
        kr = m.upload_fp16(rng.standard_normal(shape.kv_width).astype(np.float32))
        vr = m.upload_fp16(rng.standard_normal(shape.kv_width).astype(np.float32))
        cache.store(layer, kr, vr, context - 1, 1)
        rows.append((kr, vr))
    m.synchronize()
    return alloc, cache, tier_map, rows, host


def layer_bytes(m, shape, tiers_of_layer, heads) -> int:
    """Algorithmic bytes one layer's decode must move: every sealed page at
    its tier (metadata included), the own page at FP16, the page table
    (8 B address + 1 B tier a page), q and out (fp16), the decode row, and
    the scores read and written."""
    sizes = tier_sizes(m, shape)
    pages = len(tiers_of_layer)
    kv_bytes = sum(sizes[t] for t in tiers_of_layer) + sizes[0]
    return (kv_bytes + 9 * pages + 2 * 2 * heads * shape.head_dim + 2 * 2 * shape.kv_width
            + 2 * 4 * (pages + 1))


def timed_graph(m, stream, body, steps, warmup) -> float:
    """Milliseconds a replay of `body`, captured once as a HIP graph on
    `stream`, averaged over `steps` replays after `warmup`."""
    body()
    m.synchronize()
    graph = m.Graph(stream)
    with graph.capture():
        body()
    for _ in range(warmup):
        graph.launch()
    stream.synchronize()
    timer = m.Timer(stream)
    timer.start()
    for _ in range(steps):
        graph.launch()
    timer.stop()
    stream.synchronize()
    return timer.elapsed_ms() / steps


def relative_gap(a, b) -> float:
    """The largest |a - b| over the largest |b|: two product paths' agreement."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def copy_peak(m, page=32768, count=32768, reps=10) -> float:
    """The achieved HBM rate of a plain device copy (1 GiB read + 1 GiB
    written a launch, the batched page-copy kernel), GB/s of read + write."""
    arena = m.DeviceArena(2 * page * count)
    src = [arena.address + i * page for i in range(count)]
    copy = m.PageCopy(src, [a + page * count for a in src], page)
    copy.launch()
    m.synchronize()
    timer = m.Timer()
    timer.start()
    for _ in range(reps):
        copy.launch()
    timer.stop()
    m.synchronize()
    return 2 * page * count * reps / (timer.elapsed_ms() * 1e-3) / 1e9


def decode_source_hash() -> str:
    h = hashlib.sha256()
    # decode.hip and every header it includes.
    for name in ("decode.hip", "dequant.hpp", "common.hpp", "lane_ops.hpp", "kernels.hpp",
                 "page_tasks.hpp", "quant_core.hpp"):
        h.update((PKG / "csrc" / name).read_bytes())
    return h.hexdigest()[:16]


def profiled_traffic():
    """HBM bytes one layer's decode moves in the headline form, from the
    committed counter summary of this bench (FETCH_SIZE and WRITE_SIZE per
    dispatch, scaled by the copy reference), when that summary was taken of
    the decode sources as they are now; else None, and why."""
    try:
        text = TRAFFIC_PROFILE.read_text()
    except OSError:
        return None, "no counter summary"
    fields = dict(line.split(":", 1) for line in text.splitlines()
                  if line.startswith(("traffic_bytes_per_layer:", "decode_sources:")))
    if fields.get("decode_sources", "").strip() != decode_source_hash():
        return None, "the counter summary predates the decode sources"
    return int(fields["traffic_bytes_per_layer"].strip()), "counter summary of these sources"


# ---- config 3: the headline and its variants ------------------------------------------------

def decode_legs(m, shape, context, layers, steps, warmup):
    d = m.device
    heads, hd, kv = shape.heads, shape.head_dim, shape.kv_heads
    t0 = time.perf_counter()
    alloc, cache, tier_map, rows, host = build_config3(m, shape, context, layers)
    log(f"config-3 cache built in {time.perf_counter() - t0:.1f}s")
    per_layer = [layer_bytes(m, shape, tier_map[l], heads) for l in range(layers)]
    step_bytes = sum(per_layer)
    rng = np.random.default_rng(1)
    q_host = rng.standard_normal((layers, heads * hd)).astype(np.float32)
    qs = [m.upload_fp16(q_host[l]) for l in range(layers)]
    stream = m.Stream()
    out = {}

    # The headline: each layer kept, one fold a step.
    outs_kept = [d.empty(heads * hd) for _ in range(layers)]
    scores_kept = d.ImportanceScores(layers, context // P)

    def step_kept():
        for l in range(layers):
            kr, vr = rows[l]
            cache.attention_kept(l, qs[l], None, None, outs_kept[l], context, heads, kv, hd, kr, vr)
        cache.fold_kept(scores=scores_kept)

    ms = timed_graph(m, stream, step_kept, steps, warmup)
    log(f"per-layer, fold once: {ms * 1e3:.1f} us/token, {step_bytes / ms / 1e6:.0f} GB/s")
    out["kept"] = ms

    # The floor of the headline's structure, live: a graph of as many
    # dependent launches (2 a layer and the fold), each writing one float.
    dummy = d.empty_f32(1)
    launches = 2 * layers + 1

    def empty_launches():
        for _ in range(launches):
            m._check(m.lib.mi_fill_f32(dummy.address, 1, 0.0, None))

    out["launch_floor"] = timed_graph(m, stream, empty_launches, steps, warmup) / launches
    log(f"dependent launch floor: {out['launch_floor'] * 1e3:.2f} us a launch, "
        f"{out['launch_floor'] * launches * 1e3:.1f} us for the headline's {launches}")

    # The fold fused into each layer's combine.
    outs_fused = [d.empty(heads * hd) for _ in range(layers)]
    scores_fused = d.ImportanceScores(layers, context // P)
    partials = d.empty_f32(d.attention_partials(hd))

    def step_fused():
        for l in range(layers):
            kr, vr = rows[l]
            cache.attention(l, qs[l], None, None, outs_fused[l], 1, context, heads, kv, hd, kr, vr,
                            None, partials, scores=scores_fused)

    out["fused"] = timed_graph(m, stream, step_fused, steps, warmup)
    log(f"per-layer, fold fused: {out['fused'] * 1e3:.1f} us/token")

    # Every layer in one launch (a caller holding every layer's query).
    q_all = m.upload_fp16(q_host.reshape(-1))
    out_all = d.empty(layers * heads * hd)
    k_all = m.upload_fp16(np.stack([rows[l][0].to_numpy() for l in range(layers)])
                          .reshape(-1).astype(np.float32))
    v_all = m.upload_fp16(np.stack([rows[l][1].to_numpy() for l in range(layers)])
                          .reshape(-1).astype(np.float32))
    scores_all = d.ImportanceScores(layers, context // P)

    def step_all():
        cache.attention_layers(0, layers, q_all, out_all, context, heads, kv, hd, k_all, v_all,
                               None, scores=scores_all)

    out["one_launch"] = timed_graph(m, stream, step_all, steps, warmup)
    log(f"one launch: {out['one_launch'] * 1e3:.1f} us/token")

    # Self-consistency of the product paths: the kept and fused forms give
    # the same bits (outputs and scores, after as many folds each); the one
    # launch splits the pages differently, within the attention tolerance.
    got_kept = np.stack([o.to_numpy() for o in outs_kept])
    got_fused = np.stack([o.to_numpy() for o in outs_fused])
    if not np.array_equal(got_kept, got_fused):
        raise AssertionError("the kept and fused decode forms differ")
    gap = relative_gap(out_all.to_numpy().reshape(layers, -1), got_kept)
    if not np.isfinite(got_kept).all() or gap > 2e-3:
        raise AssertionError(f"one launch and per-layer decode part by {gap:.3g}")
    out["one_launch_gap"] = gap

    # The key bias on (reported apart, as config 3 asks).
    bias = (3 * rng.standard_normal((layers, kv, hd))).astype(np.float16)
    rope = d.RopeTable(hd, shape.rope_theta)
    rope.cover(context)
    bs = [m.upload_fp16(bias[l].astype(np.float32)) for l in range(layers)]
    outs_bias = [d.empty(heads * hd) for _ in range(layers)]
    scores_bias = d.ImportanceScores(layers, context // P)

    def step_bias():
        for l in range(layers):
            kr, vr = rows[l]
            cache.attention_kept(l, qs[l], bs[l], rope, outs_bias[l], context, heads, kv, hd, kr,
                                 vr)
        cache.fold_kept(scores=scores_bias)

    out["bias"] = timed_graph(m, stream, step_bias, steps, warmup)
    log(f"per-layer with the key bias: {out['bias'] * 1e3:.1f} us/token")
    return out, step_bytes, per_layer, (alloc, cache, host, rows, rope, bs, stream)


# ---- config 2: 0.5B, 8K, FP16, RMSNorm + RoPE + store + decode a layer ----------------------

def config2(m, steps, warmup, seed=0):
    from microinfer import workloads as w
    d = m.device
    shape = w.QWEN_05B
    layers, heads, kv, hd, hidden = shape.layers, shape.heads, shape.kv_heads, shape.head_dim, \
        shape.hidden
    context = 8192
    pages = context // P
    alloc = m.PagedKVCache(tier_sizes(m, shape), [layers * pages + 8] * 4)
    cache = d.KVPages(alloc, layers, P, kv, hd, m.Tier.FP16, d.Halves.Both, [], False)
    rng = np.random.default_rng(seed)
    fill_rows(m, cache, shape, layers, context, rng)
    x = d.upload_f32(rng.standard_normal(hidden).astype(np.float32))
    norm_w = [m.upload_fp16(rng.uniform(0.5, 1.5, hidden).astype(np.float32)) for _ in range(layers)]
    normed = d.empty(hidden)
    qk_raw = [m.upload_fp16(rng.standard_normal((heads + kv) * hd).astype(np.float32))
              for _ in range(layers)]
    qk = [d.empty((heads + kv) * hd) for _ in range(layers)]
    v_rows = [m.upload_fp16(rng.standard_normal(kv * hd).astype(np.float32)) for _ in range(layers)]
    positions = d.DeviceIndex([context - 1])
    outs = [d.empty(heads * hd) for _ in range(layers)]
    partials = d.empty_f32(d.attention_partials(hd))
    q_width = heads * hd
    rope = d.RopeTable(hd, shape.rope_theta)
    rope.cover(context)

    def calls():
        # The reference's operator sequence: five launches a layer.
        for l in range(layers):
            d.rmsnorm_f32(x, norm_w[l], normed, 1, hidden, shape.rms_eps)
            d.rope(qk_raw[l], positions, qk[l], 1, heads + kv, hd, shape.rope_theta)
            k_row = d.view(qk[l], q_width, kv * hd)
            cache.store(l, k_row, v_rows[l], context - 1, 1)
            cache.attention(l, d.view(qk[l], 0, q_width), None, None, outs[l], 1, context, heads,
                            kv, hd, k_row, v_rows[l], None, partials)

    def three():
        # The same work in three launches a layer: RMSNorm, RoPE and the
        # store as one, then the pages kernel and the combine.
        for l in range(layers):
            cache.rope_store(l, qk_raw[l], qk[l], heads, positions, rope, v_rows[l],
                             norm=(x, norm_w[l], normed, shape.rms_eps))
            cache.attention(l, d.view(qk[l], 0, q_width), None, None, outs[l], 1, context, heads,
                            kv, hd, d.view(qk[l], q_width, kv * hd), v_rows[l], None, partials)

    def fused():
        # Two launches a layer: the pages kernel turns q and the row's k,
        # stores the row and forms the RMSNorm; then the combine.
        for l in range(layers):
            cache.attend_row(l, qk_raw[l], qk[l], heads, context, rope, v_rows[l], outs[l],
                             norm=(x, norm_w[l], normed, shape.rms_eps))

    stream = m.Stream()
    ms_calls = timed_graph(m, stream, calls, steps, warmup)
    want = np.stack([o.to_numpy() for o in outs])
    want_qk = np.stack([t.to_numpy() for t in qk])
    ms_three = timed_graph(m, stream, three, steps, warmup)
    got_three = np.stack([o.to_numpy() for o in outs])
    for i, t in enumerate(qk):
        d.random_half(t, 900 + i, 1.0)  # so that the turned rows are written again
    ms = timed_graph(m, stream, fused, steps, warmup)
    got = np.stack([o.to_numpy() for o in outs])
    if not np.isfinite(got).all():
        raise AssertionError("config 2: a non-finite output")
    if not (np.array_equal(got, want) and np.array_equal(got_three, want)
            and np.array_equal(np.stack([t.to_numpy() for t in qk]), want_qk)):
        raise AssertionError("config 2: the fused launches and the operator calls disagree")
    fp16_page = tier_sizes(m, shape)[0]
    per_layer = (pages * fp16_page + pages * 8 + 2 * 2 * q_width       # pages, table, q, out
                 + 2 * 2 * (heads + kv) * hd                           # RoPE in and out
                 + 4 * hidden + 2 * hidden + 2 * hidden                 # RMSNorm x, w, out
                 + 2 * 2 * kv * hd)                                     # the stored row
    step_bytes = layers * per_layer
    gbs = step_bytes / (ms * 1e-3) / 1e9
    log(f"config 2: {ms * 1e3:.1f} us/token, {gbs:.0f} GB/s (three launches a layer: "
        f"{ms_three * 1e3:.1f} us/token; operator calls: {ms_calls * 1e3:.1f} us/token)")
    return {"us_per_token": round(ms * 1e3, 2), "gb_per_s": round(gbs, 1),
            "pct_hbm_peak": round(100 * gbs / PEAK_GBS, 2), "bytes_per_token": step_bytes,
            "launches_per_layer": 2,
            "row_launch": {"us_per_token": round(ms_three * 1e3, 2), "launches_per_layer": 3},
            "operator_calls": {"us_per_token": round(ms_calls * 1e3, 2),
                               "gb_per_s": round(step_bytes / (ms_calls * 1e-3) / 1e9, 1),
                               "launches_per_layer": 5},
            "config": "qwen2.5-0.5b 14q/2kv/hd64, 24 layers, 8K FP16 pages (cache that does not "
                      "seal); a layer: RMSNorm (hidden 896), RoPE of q and k, the decode row "
                      "stored, split decode; HIP graph of 48 launches (the pages kernel turns q "
                      "and k, stores the row and forms the RMSNorm, then the combine); "
                      "row_launch: RMSNorm, RoPE and the store as a launch of their own before "
                      "the pages kernel and the combine; operator_calls: the reference's five "
                      "calls a layer; all three give the same outputs to the bit"}


# ---- whole decode steps (every projection, one graph a token) -------------------------------

def random_model(m, shape, key_bias, seed):
    """Random fp16 weights of `shape` on the device (norm weights ones):
    (embed, final norm, head, layers)."""
    d = m.device
    L, H, I, V = shape.layers, shape.hidden, shape.intermediate, shape.vocab
    qw, kw = shape.heads * shape.head_dim, shape.kv_width
    counter = [seed * 1000]

    def rand(count, scale):
        t = d.empty(count)
        counter[0] += 1
        d.random_half(t, counter[0], scale)
        return t

    ones = m.upload_fp16(np.ones(max(H, 8), np.float32))
    layers = []
    for _ in range(L):
        layers.append({
            "input_norm": ones, "post_norm": ones,
            "q_w": rand(qw * H, H ** -0.5), "k_w": rand(kw * H, H ** -0.5),
            "v_w": rand(kw * H, H ** -0.5), "o_w": rand(H * qw, qw ** -0.5),
            "gate_w": rand(I * H, H ** -0.5), "up_w": rand(I * H, H ** -0.5),
            "down_w": rand(H * I, I ** -0.5),
            "q_b": rand(qw, 0.5) if key_bias else None, "k_b": rand(kw, 4.0) if key_bias else None,
            "v_b": rand(kw, 0.5) if key_bias else None})
    embed = rand(V * H, 1.0)
    head = rand(V * H, H ** -0.5)
    return embed, ones, head, layers


def prefill_flops(shape, start, n):
    """Flops of a prefill of n prompt rows after `start` positions: every
    projection (2 flops a weight a row), attention's QK^T and PV over the
    positions each row attends (causal), and the last row's head."""
    H, I = shape.hidden, shape.intermediate
    qw, kw = shape.heads * shape.head_dim, shape.kv_width
    per_row = 2 * shape.layers * (H * qw + 2 * H * kw + qw * H + 3 * H * I)
    attended = n * start + n * (n + 1) // 2
    attention = 4 * shape.layers * shape.heads * shape.head_dim * attended
    return per_row * n + attention + 2 * H * shape.vocab


def full_step(m, shape, context, steps, warmup, mix, key_bias, seed, prompt_chunk=None,
              graphed=True):
    """`steps` greedy decode steps of a random-weight model of `shape` from
    position `context` (the cache born at `mix` over the whole run), after
    `warmup` steps: tokens/s from the replays' device time, and HBM GB/s of
    the weights and pages a step reads. With `prompt_chunk`, the context is
    a random prompt prefilled through the whole model in chunks of that many
    rows (timed on the device, after one chunk into a throwaway cache);
    otherwise its rows are stored directly."""
    from microinfer import workloads as w
    d = m.device
    L, H, I, V = shape.layers, shape.hidden, shape.intermediate, shape.vocab
    embed, ones, head, layers = random_model(m, shape, key_bias, seed)
    end = context + warmup + steps
    pages = -(-end // P)
    tier_map = w.tier_map(seed, L, pages, mix)
    alloc, cache = sealing_cache(m, shape, L, pages, tier_map)
    scores = d.ImportanceScores(L, pages)
    step = d.DecodeStep(cache, w.model_dict(shape), embed, ones, head, layers, scores, 1)
    rng = np.random.default_rng(seed)
    t0 = time.perf_counter()
    prefilled = None
    if prompt_chunk:
        _, spare = sealing_cache(m, shape, L, -(-prompt_chunk // P), tier_map)
        spare_step = d.DecodeStep(spare, w.model_dict(shape), embed, ones, head, layers)
        spare_step.prefill(rng.integers(0, V, prompt_chunk), 0, prompt_chunk)
        del spare_step, spare
        ids = rng.integers(0, V, context)
        t0 = time.perf_counter()
        first, prefill_ms = step.prefill(ids, 0, prompt_chunk)
        prefill_wall = time.perf_counter() - t0
        flops = prefill_flops(shape, 0, context)
        tflops = flops / (prefill_ms * 1e-3) / 1e12
        prefilled = {"prompt": context, "chunk": prompt_chunk, "device_ms": round(prefill_ms, 2),
                     "wall_ms": round(prefill_wall * 1e3, 2),
                     "tokens_per_s": round(context / (prefill_ms * 1e-3), 1),
                     "tflops": round(tflops, 1), "flops": flops,
                     "pct_fp16_mfma_peak": round(100 * tflops / 2500.0, 2),
                     "first_token": int(first)}
        log(f"{shape.name}: {context}-token prefill in {prompt_chunk}-row chunks "
            f"{prefill_ms:.1f} ms on the device ({tflops:.0f} TFLOP/s)")
        token = int(first)
    else:
        fill_rows(m, cache, shape, L, context, rng)
        log(f"{shape.name}: {context} positions stored in {time.perf_counter() - t0:.1f}s")
        token = 1
    if warmup:
        tokens, _ = step.run(token, context, warmup, graphed=graphed)
        token = int(tokens[-1])
    t0 = time.perf_counter()
    tokens, ms = step.run(token, context + warmup, steps, graphed=graphed)
    wall = time.perf_counter() - t0
    logits = step.logits()
    if not np.isfinite(logits).all() or not ((tokens >= 0) & (tokens < V)).all():
        raise AssertionError(f"{shape.name}: a step gave non-finite logits or no token")
    # Bytes a step reads: the weights, and every layer's pages at the run's
    # middle position at their tiers.
    sizes = tier_sizes(m, shape)
    mid = context + warmup + steps // 2
    kv_bytes = sum(sum(sizes[t] for t in tier_map[l][:mid // P]) + sizes[0] for l in range(L))
    weight_bytes = w.weight_bytes_per_step(shape)
    step_bytes = weight_bytes + kv_bytes
    per_step = ms / steps
    gbs = step_bytes / (per_step * 1e-3) / 1e9
    log(f"{shape.name} whole step @{mid}: {per_step * 1e3:.1f} us, {steps / ms * 1e3:.0f} tok/s, "
        f"{gbs:.0f} GB/s")
    out = {"tokens_per_s": round(steps / (ms * 1e-3), 1), "ms_per_token": round(per_step, 4),
            "gb_per_s": round(gbs, 1), "pct_hbm_peak": round(100 * gbs / PEAK_GBS, 2),
            "weight_bytes": weight_bytes, "kv_bytes": kv_bytes,
            "launches_per_token": step.launches, "positions": [context + warmup, end],
            "run_wall_s_with_capture": round(wall, 4),
            "config": f"{shape.name} ({L} layers, hidden {H}, FFN {I}, vocab {V}), fp16 random "
                      f"weights, pages at {'/'.join(str(int(f * 100)) for _, f in reversed(mix))} "
                      f"% of FP16..{'INT2' if len(mix) > 3 else 'INT4'}, scores folded every "
                      f"step; {steps} greedy steps replaying one graph"}
    if prefilled:
        out["prefill"] = prefilled
        out["config"] = (f"{context}-token random prompt prefilled in {prompt_chunk}-row chunks "
                         f"(hipBLASLt projections, matrix-core chunk attention over sealed pages), "
                         f"then {out['config']}")
    return out


# ---- prefill attention ---------------------------------------------------------------------

def prefill_tile(m, shape, cache, host, rows, rope, bs, layers, context, stream, steps, warmup):
    """The reference's prefill-tile measurement (benchmark.jsonl:3292-3296:
    16 queries at the end of a 32K context, key bias on, one launch a
    layer) on the config-3 cache."""
    d = m.device
    heads, hd, kv = shape.heads, shape.head_dim, shape.kv_heads
    n = 16
    rng = np.random.default_rng(2)
    q = rng.standard_normal((layers, n, heads, hd)).astype(np.float16)
    qs = [m.upload_fp16(q[l].astype(np.float32)) for l in range(layers)]
    ks = [m.upload_fp16(host[l][0][-(n - 1):].astype(np.float32)) for l in range(layers)]
    vs = [m.upload_fp16(host[l][1][-(n - 1):].astype(np.float32)) for l in range(layers)]
    k_chunk, v_chunk = [], []
    for l in range(layers):
        k_chunk.append(d.empty(n * kv * hd))
        v_chunk.append(d.empty(n * kv * hd))
        d.copy(ks[l], k_chunk[l], (n - 1) * kv * hd)
        d.copy(vs[l], v_chunk[l], (n - 1) * kv * hd)
        d.copy(rows[l][0], d.view(k_chunk[l], (n - 1) * kv * hd, kv * hd), kv * hd)
        d.copy(rows[l][1], d.view(v_chunk[l], (n - 1) * kv * hd, kv * hd), kv * hd)
    outs = [d.empty(n * heads * hd) for _ in range(layers)]
    partials = d.empty_f32(d.attention_partials(hd))

    def body():
        for l in range(layers):
            cache.attention(l, qs[l], bs[l], rope, outs[l], n, context, heads, kv, hd, k_chunk[l],
                            v_chunk[l], None, partials)

    ms = timed_graph(m, stream, body, steps, warmup)
    if not all(np.isfinite(o.to_numpy()).all() for o in outs):
        raise AssertionError("prefill tile: a non-finite output")
    return {"us_per_launch": round(ms * 1e3 / layers, 2),
            "ms_per_token_all_layers": round(ms * shape.layers / layers, 4),
            "queries": n, "context": context, "key_bias": True,
            "reference_us_per_launch_rtx4050": [6160.9, 7132.3],
            "note": "config-3 cache (tiers 20/30/40/10 %), one launch a layer, HIP graph of "
                    f"{layers} launches; MFMA chunk kernel with split-K + combine"}


def prefill_chunks(m, stream, steps, warmup, seed=5):
    """Config 5's prefill attention: Llama-3.2-1B shape, 16K positions in 2K
    chunks over pages born at 30/40/30 % FP16/INT8/INT4 (seeded importance);
    each chunk's 2048 queries attend the pages before their own at their
    tiers and their own at FP16. One layer's 8 chunk launches, timed as a
    graph; TFLOP/s of the causal attention's algorithmic work
    4 * heads * head_dim * (keys each query sees), against the dense fp16
    MFMA peak."""
    from microinfer import workloads as w
    d = m.device
    shape = w.LLAMA_1B
    heads, hd, kv = shape.heads, shape.head_dim, shape.kv_heads
    context, chunk = 16384, 2048
    pages = context // P
    tier_map = w.tier_map(seed, 1, pages, w.MIX_CONFIG5)
    alloc, cache = sealing_cache(m, shape, 1, pages, tier_map)
    rng = np.random.default_rng(seed)
    k, v = w.kv_rows(rng, context, shape, w.outlier_channels(rng, shape.kv_width))
    cache.reserve(context)
    cache.store(0, m.upload_fp16(k.astype(np.float32)), m.upload_fp16(v.astype(np.float32)), 0,
                context)
    q = rng.standard_normal((context, heads, hd)).astype(np.float16)
    qs, ks, vs, outs = [], [], [], []
    for c in range(context // chunk):
        r = slice(c * chunk, (c + 1) * chunk)
        qs.append(m.upload_fp16(q[r].astype(np.float32)))
        ks.append(m.upload_fp16(k[r].astype(np.float32)))
        vs.append(m.upload_fp16(v[r].astype(np.float32)))
        outs.append(d.empty(chunk * heads * hd))
    partials = d.empty_f32(d.attention_partials(hd))

    def body():
        for c in range(context // chunk):
            cache.attention(0, qs[c], None, None, outs[c], chunk, (c + 1) * chunk, heads, kv, hd,
                            ks[c], vs[c], None, partials)

    ms = timed_graph(m, stream, body, steps, warmup)
    if not all(np.isfinite(o.to_numpy()).all() for o in outs):
        raise AssertionError("prefill chunks: a non-finite output")
    flop = 4.0 * heads * hd * context * (context + 1) / 2
    tflops = flop / (ms * 1e-3) / 1e12
    return {"ms_per_layer": round(ms, 4), "ms_all_layers": round(ms * shape.layers, 3),
            "tflops": round(tflops, 1),
            "roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": MFMA_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(tflops / MFMA_PEAK_TFLOPS, 4),
                         "algorithmic_flop_per_layer": flop},
            "config": "llama-3.2-1b 32q/8kv/hd64, 16K in 2K chunks, tiers FP16/INT8/INT4 30/40/30 %"}


# ---- the batch quantiser ---------------------------------------------------------------------

def quantise_batches(m, stream, steps, warmup, seed=4, single_launch_graphs=False):
    """The batch quantiser (mi_quantise_pages; reference quant.cu:419-436)
    at the 1.5B page shape (2 KV heads x head_dim 128, 32 tokens): N FP16
    pages quantised to a tier in one launch, timed as a HIP graph. Bytes a
    launch must move: every FP16 page read (32 KiB) and every quantised page
    written (its layout's page_bytes)."""
    from microinfer import workloads as w
    shape = w.QWEN_15B
    kv, hd = shape.kv_heads, shape.head_dim
    fp16 = m.device.page_bytes(P, shape.kv_width)
    most = 4096
    rng = np.random.default_rng(seed)
    k, v = w.kv_rows(rng, most * P, shape, w.outlier_channels(rng, shape.kv_width))
    pages = np.concatenate([k.reshape(most, P * shape.kv_width),
                            v.reshape(most, P * shape.kv_width)], axis=1)
    src = m._Storage(most * fp16)
    m._h2d(src.ptr, pages.view(np.uint8).reshape(-1))
    out = {}
    for tier, n in ((2, 409), (1, 409), (3, 102), (2, 4096), (1, 4096), (3, 4096)):
        pb = m.quantised_page_layout(tier, kv, hd, P)["page_bytes"]
        dst = m._Storage(n * pb)
        table = np.array([src.ptr + i * fp16 for i in range(n)] +
                         [dst.ptr + i * pb for i in range(n)], np.uint64)
        tab = m._Storage(table.nbytes)
        m._h2d(tab.ptr, table)

        def launches(count):
            def body():
                for _ in range(count):
                    m._check(m.lib.mi_quantise_pages(tab.ptr, tab.ptr + 8 * n, n, tier, P, kv,
                                                     hd, None))
            return body

        # Launches of tens of microseconds: enough replays that the clocks
        # have risen and the timed region is not a handful of launches. A
        # launch is timed as one of ten back to back in a graph (a batch
        # among others, as a plan's tiers go), and alone in its graph (the
        # graph launch's own overhead included).
        alone = timed_graph(m, stream, launches(1), max(steps, 400), max(warmup, 400))
        if single_launch_graphs:
            ms = alone
        else:
            back_to_back = 10
            ms = timed_graph(m, stream, launches(back_to_back), max(steps, 100),
                             max(warmup, 100)) / back_to_back
        moved = n * (fp16 + pb)
        gbs = moved / (ms * 1e-3) / 1e9
        name = {1: "INT8", 2: "INT4", 3: "INT2"}[tier]
        out[f"{name}_{n}"] = {"us": round(ms * 1e3, 2), "gb_per_s": round(gbs, 1),
                              "frac_hbm": round(gbs / PEAK_GBS, 4), "bytes": moved,
                              "us_alone_in_a_graph": round(alone * 1e3, 2)}
        log(f"quantise {n} pages to {name}: {ms * 1e3:.2f} us ({alone * 1e3:.2f} alone), "
            f"{gbs:.0f} GB/s")
    return out


# ---- config 4: the requantisation plan against its host-link bound ---------------------------

def link_rates(m, nbytes=256 << 20, reps=3):
    """The host link as the moves use it, GB/s: DMA copies between device
    memory and pinned host memory each way, and the page-copy kernel writing
    into pinned host memory mapped for the device (how shadows are taken)
    and reading from it (how a restore brings them back)."""
    host = m.HostBuffer(nbytes)
    arena = m.DeviceArena(nbytes)
    best = {"d2h_dma": 0.0, "h2d_dma": 0.0, "d2h_kernel": 0.0, "h2d_kernel": 0.0}
    page = 32768
    count = nbytes // page
    to_host = m.PageCopy([arena.address + i * page for i in range(count)],
                         [host.address + i * page for i in range(count)], page)
    from_host = m.PageCopy([host.address + i * page for i in range(count)],
                           [arena.address + i * page for i in range(count)], page)
    for _ in range(reps):
        for name, kind in (("d2h_dma", 1), ("h2d_dma", 0)):
            m.synchronize()
            t0 = time.perf_counter()
            dst, src = (host.array.ctypes.data, arena.address) if kind == 1 else \
                (arena.address, host.array.ctypes.data)
            m._check(m.lib.mi_memcpy(dst, src, nbytes, kind))
            best[name] = max(best[name], nbytes / (time.perf_counter() - t0) / 1e9)
        for name, copy in (("d2h_kernel", to_host), ("h2d_kernel", from_host)):
            timer = m.Timer()
            timer.start()
            copy.launch()
            timer.stop()
            m.synchronize()
            best[name] = max(best[name], nbytes / (timer.elapsed_ms() * 1e-3) / 1e9)
    return {k: round(v, 2) for k, v in best.items()}


def requant_plan(m, shape, context, layers, link, seed=0):
    """Config 4: 28 x 1024 sealed FP16 pages; one batch moves 50% to INT4 and
    25% to INT2 (first downgrades, shadows taken, their pinned host memory
    pinned ahead), then one batch moves 10% of the INT4 pages to INT8 from
    their retained shadows. Pages/s of each, the granule release counted in
    the comparable figure, against max(host-link bytes / the link rate
    measured in this run, HBM bytes / 8 TB/s)."""
    from microinfer import workloads as w
    pages = context // P
    alloc, cache = sealing_cache(m, shape, layers, pages, [])
    fill_rows(m, cache, shape, layers, context, np.random.default_rng(seed))
    keys = [(l, p) for l in range(layers) for p in range(pages)]
    order = np.random.default_rng(seed).permutation(len(keys))
    n4, n2 = len(keys) // 2, len(keys) // 4
    down = [(*keys[i], 2) for i in order[:n4]] + [(*keys[i], 3) for i in order[n4:n4 + n2]]
    t0 = time.perf_counter()
    cache.pin_shadows(len(down))
    pin_s = time.perf_counter() - t0
    # The target ranges' granules mapped ahead as well (the driver maps a
    # granule of a range never used before in ~0.2 ms): spare granules kept
    # beyond each range's tail, which the batch's pages then take.
    sizes = tier_sizes(m, shape)
    g = alloc.granule_bytes
    ahead = {2: -(-n4 * sizes[2] // g), 3: -(-n2 * sizes[3] // g)}
    t0 = time.perf_counter()
    for tier, granules in ahead.items():
        alloc.keep_spare_granules(tier, granules)
    map_s = time.perf_counter() - t0
    m.synchronize()
    down_moves = np.asarray(down, np.int32)
    t0 = time.perf_counter()
    cache.move_pages(down_moves)
    down_s = time.perf_counter() - t0
    down_batch = cache.last_batch
    for tier in ahead:
        alloc.keep_spare_granules(tier, 0)
    t0 = time.perf_counter()
    alloc.drain_releases()
    release_s = time.perf_counter() - t0
    n8 = int(round(0.1 * n4))  # 10% of the INT4 pages: 1,434 of 14,336
    up = np.asarray([(*keys[i], 1) for i in order[:n8]], np.int32)
    # The restores' INT8 granules mapped ahead as well, as a spare run.
    up_ahead = -(-n8 * sizes[1] // g)
    t0 = time.perf_counter()
    alloc.keep_spare_granules(1, up_ahead)
    up_map_s = time.perf_counter() - t0
    m.synchronize()
    t0 = time.perf_counter()
    cache.move_pages(up)
    up_s = time.perf_counter() - t0
    up_batch = cache.last_batch
    alloc.keep_spare_granules(1, 0)
    t0 = time.perf_counter()
    alloc.drain_releases()
    up_release_s = time.perf_counter() - t0
    tiers = cache.page_tiers()
    if any(int(tiers[l, p]) != t for l, p, t in down[n8:] + [tuple(x) for x in up]):
        raise AssertionError("a moved page is not at the tier its move named")
    fp16 = sizes[0]
    # Algorithmic bytes: a first downgrade reads its FP16 page, writes its
    # codes, and sends the page over the link as its shadow; a restore from
    # the shadow brings the page over the link and writes its codes.
    down_hbm = n4 * (fp16 + sizes[2]) + n2 * (fp16 + sizes[3])
    down_link = (n4 + n2) * fp16
    up_hbm = n8 * sizes[1]
    up_link = n8 * fp16
    d2h = max(link["d2h_dma"], link["d2h_kernel"])
    h2d = link["h2d_dma"]
    down_bound = max(down_link / (d2h * 1e9), down_hbm / (PEAK_GBS * 1e9))
    up_bound = max(up_link / (h2d * 1e9), up_hbm / (PEAK_GBS * 1e9))
    return {"downgrades": len(down), "downgrade_seconds": round(down_s, 5),
            "downgrade_pages_per_s": round(len(down) / down_s),
            "granule_release_seconds": round(release_s, 5),
            "downgrade_pages_per_s_with_release": round(len(down) / (down_s + release_s)),
            "shadow_pin_ahead_seconds": round(pin_s, 5),
            "granule_map_ahead_seconds": round(map_s, 5),
            "granules_mapped_ahead": sum(ahead.values()),
            "downgrade_pages_per_s_with_map_ahead_and_release":
                round(len(down) / (down_s + release_s + map_s)),
            "downgrade_batch_phases_seconds": {
                k: round(down_batch[k], 5) for k in ("seconds", "prepare_seconds",
                                                     "allocate_seconds", "finish_seconds")},
            "restore_batch_phases_seconds": {
                k: round(up_batch[k], 5) for k in ("seconds", "prepare_seconds",
                                                   "allocate_seconds", "finish_seconds")},
            "restores_int4_to_int8": len(up), "restore_seconds": round(up_s, 5),
            "restore_pages_per_s": round(len(up) / up_s),
            "restore_granule_map_ahead_seconds": round(up_map_s, 5),
            "restore_granule_release_seconds": round(up_release_s, 5),
            "restore_pages_per_s_with_map_ahead_and_release":
                round(len(up) / (up_s + up_map_s + up_release_s)),
            "link_gb_per_s": link,
            "roofline": {
                "downgrade": {"bound": "host link" if down_link / d2h > down_hbm / PEAK_GBS
                              else "hbm", "bound_seconds": round(down_bound, 5),
                              "host_link_bytes": down_link, "hbm_bytes": down_hbm,
                              "frac": round(down_bound / down_s, 4),
                              "frac_with_release": round(down_bound / (down_s + release_s), 4)},
                "restore": {"bound": "host link" if up_link / h2d > up_hbm / PEAK_GBS else "hbm",
                            "bound_seconds": round(up_bound, 5), "host_link_bytes": up_link,
                            "hbm_bytes": up_hbm, "frac": round(up_bound / up_s, 4)}},
            "reference_rtx4050": {"downgrade_moves_per_s": 183000, "restore_pages_per_s": 201700}}


def restore_all(m, shape, context, layers, seed=0):
    """The reference's batched restore (benchmark.jsonl:3320): every page
    of a 28-layer 1.5B cache at 32K (28,672 pages) downgraded to INT4 in
    one batch, then every page back to FP16 from its shadow in one batch,
    timed with the given-back granules' release counted."""
    pages = context // P
    alloc, cache = sealing_cache(m, shape, layers, pages, [])
    fill_rows(m, cache, shape, layers, context, np.random.default_rng(seed))
    keys = np.asarray([(l, p) for l in range(layers) for p in range(pages)], np.int32)
    sizes = tier_sizes(m, shape)
    g = alloc.granule_bytes
    cache.pin_shadows(len(keys))
    alloc.keep_spare_granules(2, -(-len(keys) * sizes[2] // g))
    cache.move_pages(np.column_stack([keys, np.full(len(keys), 2, np.int32)]))
    alloc.keep_spare_granules(2, 0)
    alloc.drain_releases()
    m.synchronize()
    alloc.keep_spare_granules(0, -(-len(keys) * sizes[0] // g))
    m.synchronize()
    t0 = time.perf_counter()
    cache.move_pages(np.column_stack([keys, np.zeros(len(keys), np.int32)]))
    up_s = time.perf_counter() - t0
    alloc.keep_spare_granules(0, 0)
    t0 = time.perf_counter()
    alloc.drain_releases()
    release_s = time.perf_counter() - t0
    tiers = cache.page_tiers()[:, :pages]
    if not (tiers == 0).all():
        raise AssertionError("a restored page is not at FP16")
    return {"pages": len(keys), "seconds": round(up_s, 5),
            "pages_per_s": round(len(keys) / up_s),
            "granule_release_seconds": round(release_s, 5),
            "pages_per_s_with_release": round(len(keys) / (up_s + release_s)),
            "reference_rtx4050_pages_per_s": 201700}


#: The reference's single-move latency groups (tools/requantisation_latency.py:
#: 53-55): the INT8 group's round of the quantised tiers after FP16 -> INT8.
MOVE_ROUND = (("downgrade", 2), ("downgrade", 3), ("upgrade", 1), ("downgrade", 3),
              ("upgrade", 2), ("upgrade", 1))


def move_latency(m, shape, positions=4096, samples=256, seed=97):
    """Single-page moves by tier pair, each timed by last_move (the whole
    move's wall time, once the device has finished earlier work; the
    shadow's copy apart), as tools/requantisation_latency.py times them:
    three groups of `samples` pages, one a quantised tier T, go FP16 -> T (a
    first downgrade), T -> FP16, FP16 -> T (the shadow held); the INT8 group
    then goes round the quantised tiers. Three pages make every move first,
    untimed. Median, P90 and max microseconds a pair."""
    layers = shape.layers
    pages = positions // P
    alloc, cache = sealing_cache(m, shape, layers, pages, [])
    fill_rows(m, cache, shape, layers, positions, np.random.default_rng(seed))
    keys = [(l, i) for i in range(pages) for l in range(layers)]
    warm, groups = keys[:3], [keys[3 + k * samples:3 + (k + 1) * samples] for k in range(3)]
    names = {0: "FP16", 1: "INT8", 2: "INT4", 3: "INT2"}
    records = {}

    def move(layer, page, frm, to, first=False):
        (cache.downgrade if to > frm else cache.upgrade)(layer, page, to)
        last = cache.last_move
        name = f"{names[frm]}->{names[to]}" + (" first" if first else "")
        records.setdefault(name, []).append((last["seconds"], last["shadow_seconds"]))

    for layer, page in warm:
        for frm, to in ((0, 1), (1, 2), (2, 3), (3, 1), (1, 0)):
            (cache.downgrade if to > frm else cache.upgrade)(layer, page, to)
    for tier, group in zip((1, 2, 3), groups):
        for layer, page in group:
            move(layer, page, 0, tier, first=True)
        for layer, page in group:
            move(layer, page, tier, 0)
        for layer, page in group:
            move(layer, page, 0, tier)
    at = 1
    for _, to in MOVE_ROUND:
        for layer, page in groups[0]:
            move(layer, page, at, to)
        at = to
    out = {}
    for name, rec in records.items():
        sec = np.asarray([r[0] for r in rec]) * 1e6
        sh = np.asarray([r[1] for r in rec]) * 1e6
        out[name] = {"moves": len(rec), "median_us": round(float(np.median(sec)), 2),
                     "p90_us": round(float(np.percentile(sec, 90)), 2),
                     "max_us": round(float(sec.max()), 2),
                     "shadow_median_us": round(float(np.median(sh)), 2)}
    out["reference_rtx4050_median_us"] = {
        "FP16->INT8": 13.4, "FP16->INT4": 19.3, "FP16->INT2": 29.7, "FP16->INT8 first": 23.0,
        "FP16->INT4 first": 28.8, "FP16->INT2 first": 39.3, "INT8->FP16": 7.7,
        "INT4->FP16": 7.7, "INT2->FP16": 7.7, "INT8->INT4": 31.7, "INT8->INT2": 37.0,
        "INT4->INT2": 37.2, "INT4->INT8": 20.7, "INT2->INT8": 20.7, "INT2->INT4": 26.3}
    return out


def decode_tier_rows(m, shape, stream, steps, warmup, seed=204):
    """The reference's per-tier decode rows (tools/attention_speed.py,
    benchmark.jsonl:3292-3296): a one-layer cache of `length` positions at
    one tier (FP16, INT8, INT4, INT2) or born from a map cycling the four
    tiers page by page, keys completed by a key bias (x30) with RoPE, one
    query over every position with the per-page mass and without; one
    launch's device time (a graph of 20 launches), microseconds, and the
    whole model's ms a token (x28)."""
    d = m.device
    heads, kv, hd = shape.heads, shape.kv_heads, shape.head_dim
    sizes = tier_sizes(m, shape)
    out = {}
    for length in (32768, 16384):
        pages = -(-length // P)
        for name, tier in (("FP16", 0), ("INT8", 1), ("INT4", 2), ("INT2", 3), ("mixed", None)):
            rng = np.random.default_rng(seed)
            if tier is None:
                tmap = [[(0, 1, 2, 3)[i % 4] for i in range(pages)]]
                born, cap = 0, [pages + 4] * 4
            else:
                tmap, born = [], tier
                cap = [0, 0, 0, 0]
                cap[tier] = pages + 2
            cap[0] += 2
            alloc = m.PagedKVCache(sizes, cap)
            cache = d.KVPages(alloc, 1, P, kv, hd, born, d.Halves.Both, tmap, False)
            width = kv * hd
            start = 0
            for n in [4096] * ((length - 1) // 4096) + [(length - 1) % 4096, 1]:
                if n == 0:
                    continue
                cache.reserve(start + n)
                k = m.upload_fp16(rng.standard_normal(n * width).astype(np.float32))
                v = m.upload_fp16(rng.standard_normal(n * width).astype(np.float32))
                cache.store(0, k, v, start, n)
                start += n
            rope = d.RopeTable(hd, shape.rope_theta)
            rope.cover(length)
            bias = m.upload_fp16((rng.standard_normal(width) * 30).astype(np.float32))
            q = m.upload_fp16(rng.standard_normal(heads * hd).astype(np.float32))
            o = d.empty(heads * hd)
            mass = d.empty_f32(heads * pages)
            part = d.empty_f32(d.attention_partials(hd))
            row = {}
            for with_mass in (True, False):
                def body():
                    for _ in range(20):
                        cache.attention(0, q, bias, rope, o, 1, length, heads, kv, hd, k, v,
                                        mass if with_mass else None, part)
                us = timed_graph(m, stream, body, max(steps // 5, 3), max(warmup // 5, 1)) \
                    * 1e3 / 20
                row["with_mass" if with_mass else "plain"] = {
                    "us_per_launch": round(us, 2), "ms_per_token_x28": round(us * 28 / 1e3, 3)}
            kv_bytes = sum(sizes[int(alloc.locate(0, i)[0])] for i in range(pages - 1)) + sizes[0]
            row["kv_bytes"] = kv_bytes
            row["gb_per_s_plain"] = round(kv_bytes / (row["plain"]["us_per_launch"] * 1e-6) / 1e9,
                                          1)
            out[f"{name}_{length // 1024}K"] = row
            del cache, alloc
    out["reference_rtx4050_us_per_launch"] = {
        "32K": {"FP16": 572.0, "INT8": 683.8, "INT4": 751.8, "INT2": 728.5, "mixed": 792.2},
        "32K_with_mass": {"FP16": 672.6, "INT8": 879.6, "INT4": 886.4, "INT2": 777.2,
                          "mixed": 886.6},
        "16K": {"FP16": 391.5, "INT8": 361.8, "INT4": 378.8, "INT2": 389.6, "mixed": 363.3}}
    out["note"] = ("one layer, key bias on, a launch = decode pages kernel + combine; the "
                   "reference times the host launch loop over batches of 20")
    return out


# ---- the CPU reference path (the oracle) -----------------------------------------------------

def blas_threads() -> int:
    try:
        from threadpoolctl import threadpool_info
        return max((p.get("num_threads", 1) for p in threadpool_info()
                    if p.get("user_api") == "blas"), default=1)
    except Exception:  # threadpoolctl absent: numpy's default
        return 1


def config1_pass_bytes(m, shape) -> int:
    """The configuration-1 pass (a 0.5B layer of 2048 positions, 64 pages),
    per quantised tier: the 64 FP16 pages in (1 MiB), the pages' codes and
    metadata out, q and out, the masses."""
    sizes = tier_sizes(m, shape)
    q_out = 2 * 2 * shape.heads * shape.head_dim
    mass = 4 * shape.heads * 64
    return sum(64 * sizes[0] + 64 * sizes[t] + q_out + mass for t in (1, 2, 3))


def cpu_config1(repeats=5, seed=0):
    """Configuration 1 on the host, with the oracle: one 0.5B-shaped layer,
    2048 positions in 64 pages; for INT8, INT4 and INT2 every page
    quantised and dequantised, then the decode at position 2047 over the
    dequantised pages (the own page at FP16) with per-page mass. Median
    seconds of `repeats` passes after one."""
    from microinfer import workloads as w
    from oracle import attention as att
    from oracle import quant
    shape = w.QWEN_05B
    kv, hd = shape.kv_heads, shape.head_dim
    rng = np.random.default_rng(seed)
    k, v = w.kv_rows(rng, 2048, shape, w.outlier_channels(rng, shape.kv_width))
    q = rng.standard_normal((1, shape.heads, hd)).astype(np.float16)

    def one_pass():
        for tier in (1, 2, 3):
            ks, vs = [], []
            for i in range(64):
                page = quant.quantise_page(k[i * P:(i + 1) * P], v[i * P:(i + 1) * P], tier, P)
                kd, vd = quant.dequantise_page(page, tier, kv, hd, P)
                ks.append(kd)
                vs.append(vd)
            K = np.concatenate(ks[:63] + [k[63 * P:]])
            V = np.concatenate(vs[:63] + [v[63 * P:]])
            _, weights = att.attention64(q, K, V)
            att.page_mass(weights[:, -1, :], P)

    one_pass()
    times = []
    for _ in range(repeats):
        t0 = time.perf_counter()
        one_pass()
        times.append(time.perf_counter() - t0)
    return statistics.median(times)


def cpu_config3_layer(m, shape, context, seed=0):
    """One config-3 layer decoded by the oracle from its page bytes (float64
    attention over the dequantised pages, fp32 EWMA): seconds."""
    from microinfer import workloads as w
    from oracle import attention as att
    from oracle import ewma, quant
    sealed = context // P - 1
    tiers = w.tier_map(seed, 1, sealed, w.MIX_CONFIG3)[0]
    rng = np.random.default_rng(seed)
    k, v = w.kv_rows(rng, context, shape, w.outlier_channels(rng, shape.kv_width))
    pages = [quant.fp16_page(k[i * P:(i + 1) * P], v[i * P:(i + 1) * P]) if t == 0 else
             quant.quantise_page(k[i * P:(i + 1) * P], v[i * P:(i + 1) * P], t, P)
             for i, t in enumerate(tiers)]
    q = rng.standard_normal((1, shape.heads, shape.head_dim)).astype(np.float16)
    scores = np.full((1, sealed + 1), np.nan, np.float32)
    t0 = time.perf_counter()
    _, mass = att.causal_decode(q, pages, tiers, k[sealed * P:], v[sealed * P:], shape.kv_heads,
                                shape.head_dim, P)
    ewma.fold(scores, 0, mass.astype(np.float32))
    return time.perf_counter() - t0, layer_bytes(m, shape, tiers, shape.heads)


def gpu_config1(m, stream, steps, warmup, seed=0):
    """The configuration-1 pass on the GPU, for the speed-up: per tier a
    cache born at that tier takes the 2048 rows (its 63 full pages
    quantised as they seal) and decodes position 2047 with mass. A graph of
    the three tiers' stores and decodes; milliseconds a pass."""
    from microinfer import workloads as w
    d = m.device
    shape = w.QWEN_05B
    kv, hd, heads = shape.kv_heads, shape.head_dim, shape.heads
    rng = np.random.default_rng(seed)
    k, v = w.kv_rows(rng, 2048, shape, w.outlier_channels(rng, shape.kv_width))
    kd, vd = m.upload_fp16(k.astype(np.float32)), m.upload_fp16(v.astype(np.float32))
    q = m.upload_fp16(rng.standard_normal(heads * hd).astype(np.float32))
    row = 2047 * kv * hd
    caches, outs, masses = [], [], []
    partials = d.empty_f32(d.attention_partials(hd))
    for tier in (1, 2, 3):
        alloc = m.PagedKVCache(tier_sizes(m, shape), [72] * 4)
        cache = d.KVPages(alloc, 1, P, kv, hd, tier, d.Halves.Both, [], False)
        cache.reserve(2048)
        caches.append((alloc, cache))
        outs.append(d.empty(heads * hd))
        masses.append(d.empty_f32(heads * 64))

    def body():
        for (_, cache), out, mass in zip(caches, outs, masses):
            cache.store(0, kd, vd, 0, 2048)
            cache.attention(0, q, None, None, out, 1, 2048, heads, kv, hd,
                            d.view(kd, row, kv * hd), d.view(vd, row, kv * hd), mass, partials)

    return timed_graph(m, stream, body, steps, warmup)


def main() -> int:
    # A fatal signal prints every thread's Python stack: where it came from.
    faulthandler.enable()
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--layers", type=int, default=None, help="fewer layers, for a quick look")
    ap.add_argument("--legs",
                    default="decode,tiers,prefill,config2,step,quantise,requant,moves,cpu",
                    help="the legs to run (comma list; decode is the headline)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-requant", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-step", action="store_true", help="skip the whole-step legs")
    ap.add_argument("--eager-step", action="store_true",
                    help="whole steps with their launches made from the host (no graph), so "
                         "that a kernel tracer sees each launch")
    ap.add_argument("--single-launch-graphs", action="store_true",
                    help="quantise batches timed one launch a graph only (for a kernel "
                         "tracer, which fails on the ten-launch graphs)")
    ap.add_argument("--traffic-reference", action="store_true",
                    help="only copy 128 MiB with the page-copy kernel (4096 pages of 32 KiB): "
                         "the known-size launch HBM byte counters are scaled by")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for "
              f"{args.gpus}); run with --gpus 1", file=sys.stderr)
        return 2

    from microinfer import _microinfer as m
    from microinfer import workloads as w
    if args.traffic_reference:
        page, count = 32768, 4096
        arena = m.DeviceArena(2 * page * count)
        src = [arena.address + i * page for i in range(count)]
        m.copy_pages(src, [a + page * count for a in src], page)
        m.synchronize()
        log(f"copied {page * count} bytes in one copy_pages launch")
        return 0
    legs = set(args.legs.split(","))
    for flag, leg in ((args.no_cpu, "cpu"), (args.no_requant, "requant"),
                      (args.no_prefill, "prefill"), (args.no_step, "step")):
        if flag:
            legs.discard(leg)
    log("device", m.device_name())
    copy_gbs = copy_peak(m)
    log(f"device copy: {copy_gbs:.0f} GB/s (read + write)")
    shape = w.QWEN_15B
    context = 32768
    layers = args.layers or shape.layers
    stream = m.Stream()

    ms = gbs = us_token = traffic = None
    times, step_bytes, traffic_note = {}, 0, None
    if "decode" in legs:
        times, step_bytes, per_layer, held = decode_legs(m, shape, context, layers, args.steps,
                                                        args.warmup)
        alloc3, cache3, host3, rows3, rope3, bs3, stream = held
        ms = times["kept"]
        gbs = step_bytes / (ms * 1e-3) / 1e9
        us_token = ms * 1e3 * shape.layers / layers
        traffic, traffic_note = profiled_traffic()

    def leg_gbs(t):
        return round(step_bytes / (t * 1e-3) / 1e9, 1)

    prefill = None
    if "prefill" in legs:
        # The tile runs on the headline's cache; the chunks build their own.
        prefill = {"chunks": prefill_chunks(m, stream, max(args.steps // 5, 3),
                                            max(args.warmup // 5, 1))}
        if "decode" in legs:
            prefill["tile"] = prefill_tile(m, shape, cache3, host3, rows3, rope3, bs3, layers,
                                           context, stream, args.steps, args.warmup)
        log(f"prefill: {prefill}")
    if "decode" in legs:
        del alloc3, cache3, host3, rows3

    tier_rows = (decode_tier_rows(m, shape, stream, args.steps, args.warmup)
                 if "tiers" in legs else None)
    if tier_rows is not None:
        log(f"decode rows by tier: {tier_rows}")

    c2 = config2(m, args.steps, args.warmup) if "config2" in legs else None

    steps_out = None
    if "step" in legs:
        steps_out = {
            "qwen2.5-1.5b_32k": full_step(m, w.QWEN_15B, 32768 - 64 - 8, 64, 8, w.MIX_CONFIG3,
                                          True, 3, graphed=not args.eager_step),
            "llama-3.2-1b_16k_config5": full_step(m, w.LLAMA_1B, 16384, 256, 0, w.MIX_CONFIG5,
                                                  False, 5, prompt_chunk=2048,
                                                  graphed=not args.eager_step)}
        steps_out["reference_rtx4050_tokens_per_s"] = {"qwen2.5-1.5b_fp16_32k": 29.5,
                                                       "qwen2.5-1.5b_fp16_16k": 40.1}

    quantise = (quantise_batches(m, stream, args.steps, args.warmup,
                                 single_launch_graphs=args.single_launch_graphs)
                if "quantise" in legs else None)

    requant = None
    if "requant" in legs:
        t0 = time.perf_counter()
        link = link_rates(m)
        log(f"host link: {link}")
        requant = requant_plan(m, shape, context, layers, link)
        requant["restore_all_int4_to_fp16"] = restore_all(m, shape, context, layers)
        log(f"requant plan in {time.perf_counter() - t0:.1f}s: {requant}")

    moves = None
    if "moves" in legs:
        moves = move_latency(m, shape)
        log(f"single-page moves: {moves}")

    cpu = None
    if "cpu" in legs:
        threads = blas_threads()
        pass_s = cpu_config1()
        pass_bytes = config1_pass_bytes(m, w.QWEN_05B)
        gpu_pass_ms = gpu_config1(m, stream, args.steps, args.warmup)
        layer_s, layer_b = cpu_config3_layer(m, shape, context)
        cpu = {"value": round(pass_bytes / pass_s / 1e9, 4), "unit": "GB/s", "cores": threads,
               "kind": "port",
               "sample": f"BASELINE configuration 1 (0.5B layer, 2048 positions, 64 pages): per "
                         f"INT8/INT4/INT2 every page quantised and dequantised by the oracle, then "
                         f"float64 decode with per-page mass at 2047; median of 5 passes after 1: "
                         f"{pass_s * 1e3:.1f} ms a pass over {pass_bytes} algorithmic bytes. "
                         f"NumPy, BLAS threads {threads} (elementwise work on one thread)",
               "pass_ms": round(pass_s * 1e3, 2),
               "gpu_pass_ms": round(gpu_pass_ms, 4),
               "gpu_speedup": round(pass_s * 1e3 / gpu_pass_ms, 1),
               "os_cpu_count": os.cpu_count(),
               "affinity_cores": len(os.sched_getaffinity(0)),
               "blas_threads": threads,
               "config3_layer": {"ms_per_layer": round(layer_s * 1e3, 1),
                                 "ms_per_token_x28": round(layer_s * 28 * 1e3, 1),
                                 "gb_per_s": round(layer_b / layer_s / 1e9, 4)}}
        log(f"cpu: {cpu}")

    if ms is None:
        print(json.dumps({"metric": METRIC, "value": None, "legs": sorted(legs), "config2": c2,
                          "decode_step": steps_out, "prefill": prefill, "quantise": quantise,
                          "requant": requant, "single_page_moves": moves,
                          "decode_by_tier": tier_rows, "cpu_baseline": cpu}),
              flush=True)
        return 0
    result = {
        "metric": METRIC, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic: seeded N(0,1) fp16 K/V with 2% outlier K channels x10, "
                "tiers by seeded lognormal importance; random fp16 weights for whole steps",
        "config": {"workload": "config3 decode attention over every layer, a layer at a time, "
                               "with per-page mass folded into the scores (EWMA) once a step; "
                               "HIP graph of 28 launch pairs + 1 fold",
                   "shape": "qwen2.5-1.5b 12q/2kv/hd128", "layers": layers,
                   "context": context, "page_tokens": P,
                   "tiers": "FP16/INT8/INT4/INT2 20/30/40/10 %", "parallelism": "single GPU"},
        "us_per_token": round(us_token, 2),
        "pct_hbm_peak": round(100 * gbs / PEAK_GBS, 2),
        "bytes_per_step": step_bytes,
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_GBS, 4), "traffic": traffic,
                     "traffic_source": traffic_note,
                     "kernel": "decode_pages_kernel + decode_combine_kernel (a layer's launch "
                               "pair) and 1/28 of the fold; achieved = algorithmic bytes a layer "
                               "/ live per-layer time (HIP events on the graph's stream)",
                     "algorithmic_bytes_per_layer": round(step_bytes / layers),
                     "measured_copy_gb_per_s": round(copy_gbs, 1)},
        "decode_forms_us_per_token": {
            "per_layer_fold_once": round(ms * 1e3 * shape.layers / layers, 2),
            "per_layer_fold_fused": round(times["fused"] * 1e3 * shape.layers / layers, 2),
            "one_launch_all_layers": round(times["one_launch"] * 1e3 * shape.layers / layers, 2),
            "per_layer_key_bias_on": round(times["bias"] * 1e3 * shape.layers / layers, 2),
            "gb_per_s": {"fold_fused": leg_gbs(times["fused"]),
                         "one_launch": leg_gbs(times["one_launch"]),
                         "key_bias_on": leg_gbs(times["bias"])},
            "one_launch_vs_per_layer_gap": round(times["one_launch_gap"], 6),
            "dependent_launch_floor_us": round(times["launch_floor"] * 1e3, 3),
            "per_layer_launch_floor_us_per_token": round(
                times["launch_floor"] * 1e3 * (2 * shape.layers + 1), 1),
            "note": "same bytes; the one launch takes every layer's query at once, not the "
                    "per-layer decode order; the launch floor is a graph of as many dependent "
                    "one-float launches as the headline's (2 a layer + the fold), timed live"},
        "decode_by_tier": tier_rows,
        "config2": c2,
        "decode_step": steps_out,
        "cpu_baseline": cpu,
        "quantise": quantise,
        "requant": requant,
        "single_page_moves": moves,
        "prefill": prefill,
    }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
