"""Benchmark of the paged mixed-precision KV-cache hot path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1]

The step (the headline workload, config 3): one decode step's attention over every layer
of a Qwen2.5-1.5B-shaped cache at 32K positions -- 28 layers, 12 query / 2 KV
heads, head_dim 128, 32-token pages born at seeded-importance tiers 20%
FP16, 30% INT8, 40% INT4, 10% INT2 -- with each layer's per-page attention
mass folded into its importance scores (EWMA) in the same pass. The 28
per-layer launches are captured once in a HIP graph and replayed; K steps are
timed with hipEvents on the stream they run on. Inputs are resident in HBM
before timing starts.

Also measured, outside the timed region: the requantisation plan of config 4
(batched moves, pages/s), the prefill attention (the reference's 16-query
tile at 32K with key bias, and config 5's 16K prefill in 2K chunks on the
matrix cores), and the CPU oracle on a bounded sample of the same workload.
Prints one JSON line.
"""

from __future__ import annotations

import argparse
import faulthandler
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "semantic-aware_adaptive_kv_cache_precision_amd"))
sys.path.insert(0, str(REPO))

METRIC = "mixed-tier decode-attn GB/s (% HBM peak) & µs/token @32K; requant pages/s"
PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0  # dense fp16 / bf16
P = 32


def log(*what) -> None:
    print("[bench]", *what, file=sys.stderr, flush=True)


def build_cache(m, shape, context, seed=0, layers=None):
    """The config-3 cache: every layer's rows stored (pages sealed at their
    birth tiers in batched launches), plus the decode row of each layer."""
    from microinfer import workloads as w
    d = m.device
    layers = layers or shape.layers
    sealed = context // P - 1       # pages before the query's own
    tier_map = w.tier_map(seed, layers, sealed, w.MIX_CONFIG3)
    sizes = [d.page_bytes(P, shape.kv_width)] + [
        m.quantised_page_layout(t, shape.kv_heads, shape.head_dim, P)["page_bytes"]
        for t in (1, 2, 3)]
    cap = [layers * (sealed + 1) + 2 * layers + 8] * 4
    alloc = m.PagedKVCache(sizes, cap)
    cache = d.KVPages(alloc, layers, P, shape.kv_heads, shape.head_dim, m.Tier.FP16,
                      d.Halves.Both, tier_map, True)
    rng = np.random.default_rng(seed)
    outliers = w.outlier_channels(rng, shape.kv_width)
    cache.reserve(context - 1)
    last_rows = []
    for layer in range(layers):
        k, v = w.kv_rows(rng, context, shape, outliers)
        kd = m.upload_fp16(k[:context - 1].astype(np.float32))
        vd = m.upload_fp16(v[:context - 1].astype(np.float32))
        cache.store(layer, kd, vd, 0, context - 1)
        last_rows.append((k, v))
    cache.reserve(context)
    rows = []
    for layer in range(layers):
        k, v = last_rows[layer]
        kr, vr = m.upload_fp16(k[-1:].astype(np.float32)), m.upload_fp16(v[-1:].astype(np.float32))
        cache.store(layer, kr, vr, context - 1, 1)
        rows.append((kr, vr))
    m.synchronize()
    return alloc, cache, tier_map, rows, last_rows


def layer_bytes(m, shape, tiers_of_layer, heads) -> int:
    """Algorithmic bytes one layer's launch must move: every sealed page at
    its tier (metadata included), the own page at FP16, the page table
    (8 B address + 1 B tier a page), q and out (fp16), the decode row, and
    the scores read and written."""
    sizes = [m.device.page_bytes(P, shape.kv_width)] + [
        m.quantised_page_layout(t, shape.kv_heads, shape.head_dim, P)["page_bytes"]
        for t in (1, 2, 3)]
    pages = len(tiers_of_layer)
    kv_bytes = sum(sizes[t] for t in tiers_of_layer) + sizes[0]
    return (kv_bytes + 9 * pages + 2 * 2 * heads * shape.head_dim + 2 * 2 * shape.kv_width
            + 2 * 4 * (pages + 1))


def cpu_baseline(shape, context, sample_layers, seed=0):
    """The oracle (NumPy, float64 attention over the dequantised pages, fp32
    EWMA), timed on a bounded sample of the same workload: `sample_layers`
    layers of the config-3 cache, each decoded once from its page bytes."""
    from threadpoolctl import threadpool_limits
    from microinfer import workloads as w
    from oracle import attention as att
    from oracle import ewma, quant
    sealed = context // P - 1
    tier_map = w.tier_map(seed, sample_layers, sealed, w.MIX_CONFIG3)
    rng = np.random.default_rng(seed)
    outliers = w.outlier_channels(rng, shape.kv_width)
    total = 0.0
    total_bytes = 0
    with threadpool_limits(limits=1):
        for layer in range(sample_layers):
            k, v = w.kv_rows(rng, context, shape, outliers)
            pages = []
            for i, t in enumerate(tier_map[layer]):
                kp, vp = k[i * P:(i + 1) * P], v[i * P:(i + 1) * P]
                pages.append(quant.fp16_page(kp, vp) if t == 0 else
                             quant.quantise_page(kp, vp, t, P))
            q = rng.standard_normal((1, shape.heads, shape.head_dim)).astype(np.float16)
            scores = np.full((1, sealed + 1), np.nan, np.float32)
            t0 = time.perf_counter()
            out, mass = att.causal_decode(q, pages, tier_map[layer], k[sealed * P:],
                                          v[sealed * P:], shape.kv_heads, shape.head_dim, P)
            ewma.fold(scores, 0, mass.astype(np.float32))
            total += time.perf_counter() - t0
            total_bytes += sum(len(p) for p in pages) + 32768
    return total, total_bytes


def requant_plan(m, shape, context, seed=0, layers=None):
    """Config 4: 28 x 1024 sealed FP16 pages; one batch moves 50% to INT4 and
    25% to INT2 (first downgrades, shadows taken), then one batch moves 10%
    of the INT4 pages to INT8 from their retained shadows. Pages/s of each."""
    from microinfer import workloads as w
    d = m.device
    layers = layers or shape.layers
    pages = context // P
    sizes = [d.page_bytes(P, shape.kv_width)] + [
        m.quantised_page_layout(t, shape.kv_heads, shape.head_dim, P)["page_bytes"]
        for t in (1, 2, 3)]
    cap = [layers * pages + 2 * layers + 8] * 4
    alloc = m.PagedKVCache(sizes, cap)
    cache = d.KVPages(alloc, layers, P, shape.kv_heads, shape.head_dim, m.Tier.FP16,
                      d.Halves.Both, [], True)
    rng = np.random.default_rng(seed)
    cache.reserve(context)
    for layer in range(layers):
        k, v = w.kv_rows(rng, context, shape, w.outlier_channels(rng, shape.kv_width))
        cache.store(layer, m.upload_fp16(k.astype(np.float32)), m.upload_fp16(v.astype(np.float32)),
                    0, context)
    m.synchronize()
    keys = [(l, p) for l in range(layers) for p in range(pages)]
    order = np.random.default_rng(seed).permutation(len(keys))
    n4, n2 = len(keys) // 2, len(keys) // 4
    down = [(*keys[i], 2) for i in order[:n4]] + [(*keys[i], 3) for i in order[n4:n4 + n2]]
    t0 = time.perf_counter()
    cache.move_pages(down)
    down_s = time.perf_counter() - t0
    # The granules the FP16 range gave up go back to the driver on the
    # cache's release thread after move_pages returns: timed apart.
    t0 = time.perf_counter()
    alloc.drain_releases()
    release_s = time.perf_counter() - t0
    n8 = n4 // 10
    up = [(*keys[i], 1) for i in order[:n8]]
    t0 = time.perf_counter()
    cache.move_pages(up)
    up_s = time.perf_counter() - t0
    # Bit-exactness spot check of a few moved pages against the oracle.
    from oracle import quant
    for layer, page, _ in (down[0], down[n4], down[-1], up[0], up[-1]):
        tier = int(cache.page_tier(layer, page))
        shadow = cache.shadow(layer, page)
        kp, vp = quant.read_fp16_page(shadow, P, shape.kv_heads, shape.head_dim)
        if not np.array_equal(alloc.read(layer, page), quant.quantise_page(kp, vp, tier, P)):
            raise AssertionError(f"moved page ({layer}, {page}) is not the oracle's bytes")
    return {"downgrades": len(down), "downgrade_seconds": down_s,
            "downgrade_pages_per_s": len(down) / down_s,
            "granule_release_seconds_after_downgrade": release_s,
            "downgrade_pages_per_s_with_release": len(down) / (down_s + release_s),
            "restores_int4_to_int8": len(up),
            "restore_seconds": up_s, "restore_pages_per_s": len(up) / up_s,
            "shadows_taken": cache.last_batch and len(down)}


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


def prefill_tile(m, shape, cache, alloc, host_rows, layers, context, stream, steps, warmup):
    """The reference's prefill-tile measurement (benchmark.jsonl:3292-3296:
    16 queries at the end of a 32K context, key bias on, one launch a
    layer) on the config-3 cache: microseconds a launch, and parity of
    layer 0 against the oracle."""
    from oracle import attention as att
    d = m.device
    heads, hd, kv = shape.heads, shape.head_dim, shape.kv_heads
    n = 16
    rng = np.random.default_rng(2)
    q = rng.standard_normal((layers, n, heads, hd)).astype(np.float16)
    bias = (3 * rng.standard_normal((layers, kv, hd))).astype(np.float16)
    rope = d.RopeTable(hd, shape.rope_theta)
    rope.cover(context)
    qs = [m.upload_fp16(q[l].astype(np.float32)) for l in range(layers)]
    bs = [m.upload_fp16(bias[l].astype(np.float32)) for l in range(layers)]
    ks = [m.upload_fp16(host_rows[l][0][-n:].astype(np.float32)) for l in range(layers)]
    vs = [m.upload_fp16(host_rows[l][1][-n:].astype(np.float32)) for l in range(layers)]
    outs = [d.empty(n * heads * hd) for _ in range(layers)]
    partials = d.empty_f32(d.attention_partials(hd))

    def body():
        for l in range(layers):
            cache.attention(l, qs[l], bs[l], rope, outs[l], n, context, heads, kv, hd, ks[l],
                            vs[l], None, partials)

    ms = timed_graph(m, stream, body, steps, warmup)
    sealed = (context - 1) // P
    pages = [alloc.read(0, i) for i in range(sealed)]
    tiers = [int(alloc.locate(0, i)[0]) for i in range(sealed)]
    k, v = host_rows[0]
    want, bound = att.causal_chunk(q[0].astype(np.float64), pages, tiers, k, v, kv, hd, P,
                                   bias[0].astype(np.float64), shape.rope_theta, with_bound=True)
    check_gate(outs[0].to_numpy().reshape(n, heads, hd), want, bound, "prefill tile layer 0")
    return {"us_per_launch": round(ms * 1e3 / layers, 2),
            "ms_per_token_all_layers": round(ms * shape.layers / layers, 4),
            "queries": n, "context": context, "key_bias": True,
            "reference_us_per_launch_rtx4050": [6160.9, 7132.3],
            "note": "config-3 cache (tiers 20/30/40/10 %), one launch a layer, HIP graph of "
                    f"{layers} launches; MFMA chunk kernel with split-K + combine"}


def decode_bias_on(m, shape, cache, alloc, host_rows, layers, context, stream, steps, warmup,
                   step_bytes):
    """Config 3 with the key bias on (reported apart, as the configuration
    asks): one query a layer at the end of the 32K context, keys completed as
    k + RoPE(bias) in fp32, the mass and EWMA fused as in the headline
    figure. Microseconds a token over the layers, and parity of layer 0."""
    from oracle import attention as att
    d = m.device
    heads, hd, kv = shape.heads, shape.head_dim, shape.kv_heads
    rng = np.random.default_rng(3)
    q = rng.standard_normal((layers, 1, heads, hd)).astype(np.float16)
    bias = (3 * rng.standard_normal((layers, kv, hd))).astype(np.float16)
    rope = d.RopeTable(hd, shape.rope_theta)
    rope.cover(context)
    qs = [m.upload_fp16(q[l].astype(np.float32)) for l in range(layers)]
    bs = [m.upload_fp16(bias[l].astype(np.float32)) for l in range(layers)]
    ks = [m.upload_fp16(host_rows[l][0][-1:].astype(np.float32)) for l in range(layers)]
    vs = [m.upload_fp16(host_rows[l][1][-1:].astype(np.float32)) for l in range(layers)]
    outs = [d.empty(heads * hd) for _ in range(layers)]
    partials = d.empty_f32(d.attention_partials(hd))
    scores = d.ImportanceScores(layers, context // P)

    def body():
        for l in range(layers):
            cache.attention(l, qs[l], bs[l], rope, outs[l], 1, context, heads, kv, hd, ks[l],
                            vs[l], None, partials, scores=scores)

    ms = timed_graph(m, stream, body, steps, warmup)
    sealed = (context - 1) // P
    pages = [alloc.read(0, i) for i in range(sealed)]
    tiers = [int(alloc.locate(0, i)[0]) for i in range(sealed)]
    k, v = host_rows[0]
    want, bound = att.causal_chunk(q[0].astype(np.float64), pages, tiers, k, v, kv, hd, P,
                                   bias[0].astype(np.float64), shape.rope_theta, with_bound=True)
    check_gate(outs[0].to_numpy().reshape(1, heads, hd), want, bound, "bias-on decode layer 0")
    return {"us_per_token": round(ms * 1e3 * shape.layers / layers, 2),
            "gb_per_s": round(step_bytes / (ms * 1e-3) / 1e9, 1),
            "note": "config-3 cache and bytes, key bias on (k + RoPE(bias) formed in fp32), "
                    "mass and EWMA fused; per-layer launches in a HIP graph"}


def prefill_chunks(m, stream, steps, warmup, seed=5):
    """Config 5's prefill attention: Llama-3.2-1B shape, 16K positions in 2K
    chunks over pages born at 30/40/30 % FP16/INT8/INT4 (seeded importance);
    each chunk's 2048 queries attend the pages before their own at their
    tiers and their own at FP16. One layer's 8 chunk launches, timed as a
    graph; TFLOP/s of the causal attention's algorithmic work
    4 * heads * head_dim * (keys each query sees), against the dense fp16
    MFMA peak."""
    from microinfer import workloads as w
    from oracle import attention as att
    d = m.device
    shape = w.LLAMA_1B
    heads, hd, kv = shape.heads, shape.head_dim, shape.kv_heads
    context, chunk = 16384, 2048
    pages = context // P
    tier_map = w.tier_map(seed, 1, pages, w.MIX_CONFIG5)
    sizes = [d.page_bytes(P, shape.kv_width)] + [
        m.quantised_page_layout(t, kv, hd, P)["page_bytes"] for t in (1, 2, 3)]
    alloc = m.PagedKVCache(sizes, [pages + 8] * 4)
    cache = d.KVPages(alloc, 1, P, kv, hd, m.Tier.FP16, d.Halves.Both, tier_map, True)
    rng = np.random.default_rng(seed)
    k, v = w.kv_rows(rng, context, shape, w.outlier_channels(rng, shape.kv_width))
    cache.reserve(context)
    cache.store(0, m.upload_fp16(k.astype(np.float32)), m.upload_fp16(v.astype(np.float32)), 0,
                context)
    q = rng.standard_normal((context, heads, hd)).astype(np.float16)
    qs, ks, vs, outs = [], [], [], []
    for c in range(context // chunk):
        rows = slice(c * chunk, (c + 1) * chunk)
        qs.append(m.upload_fp16(q[rows].astype(np.float32)))
        ks.append(m.upload_fp16(k[rows].astype(np.float32)))
        vs.append(m.upload_fp16(v[rows].astype(np.float32)))
        outs.append(d.empty(chunk * heads * hd))
    partials = d.empty_f32(d.attention_partials(hd))

    def body():
        for c in range(context // chunk):
            cache.attention(0, qs[c], None, None, outs[c], chunk, (c + 1) * chunk, heads, kv, hd,
                            ks[c], vs[c], None, partials)

    ms = timed_graph(m, stream, body, steps, warmup)
    flop = 4.0 * heads * hd * context * (context + 1) / 2
    tflops = flop / (ms * 1e-3) / 1e12
    # Parity: the last 64 queries of the last chunk against the oracle.
    n = 64
    sealed = (context - 1) // P
    pp = [alloc.read(0, i) for i in range(sealed)]
    tiers = [int(alloc.locate(0, i)[0]) for i in range(sealed)]
    want, bound = att.causal_chunk(q[-n:].astype(np.float64), pp, tiers, k, v, kv, hd, P,
                                   with_bound=True)
    got = outs[-1].to_numpy().reshape(chunk, heads, hd)[-n:]
    check_gate(got, want, bound, "prefill chunk 7, last 64 queries")
    return {"ms_per_layer": round(ms, 4), "ms_all_layers": round(ms * shape.layers, 3),
            "tflops": round(tflops, 1),
            "roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": MFMA_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(tflops / MFMA_PEAK_TFLOPS, 4),
                         "algorithmic_flop_per_layer": flop},
            "config": "llama-3.2-1b 32q/8kv/hd64, 16K in 2K chunks, tiers FP16/INT8/INT4 30/40/30 %"}


def check_gate(got, want, bound, what) -> None:
    """The reference's error gate (tests/ulp_gate.py, tests/test_attention.py:
    58-115) held to 1e-3: relative error floored at fp16's least normal and
    where the fp32 error bound spends the budget; mean under 2^-11."""
    from oracle import attention as att
    floor = np.maximum(att.FP16_MIN_NORMAL, bound / 1e-3)
    err = np.abs(got - want) / np.maximum(np.abs(want), floor)
    if err.max() >= 1e-3 or err.mean() >= 2.0**-11:
        raise AssertionError(f"{what}: off the oracle: max {err.max():.3g}, mean {err.mean():.3g}")


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


def profiled_traffic(path=REPO / "profiles" / "decode_attention_config3_hbm_bytes.md"):
    """HBM bytes one layer's decode launch pair moves, from the committed
    counter summary of this bench (FETCH_SIZE and WRITE_SIZE per dispatch,
    scaled by the copy reference); None when the summary is absent."""
    try:
        for line in path.read_text().splitlines():
            if line.startswith("traffic_bytes_per_layer:"):
                return int(line.split(":", 1)[1].strip())
    except OSError:
        pass
    return None


def main() -> int:
    # A fatal signal prints every thread's Python stack: where it came from.
    faulthandler.enable()
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--layers", type=int, default=None, help="fewer layers, for a quick look")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-requant", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
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
    d = m.device
    if args.traffic_reference:
        page, count = 32768, 4096
        arena = m.DeviceArena(2 * page * count)
        src = [arena.address + i * page for i in range(count)]
        m.copy_pages(src, [a + page * count for a in src], page)
        log(f"copied {page * count} bytes in one copy_pages launch")
        return 0
    copy_gbs = copy_peak(m)
    log(f"device copy: {copy_gbs:.0f} GB/s (read + write)")
    shape = w.QWEN_15B
    context = 32768
    layers = args.layers or shape.layers
    log("device", m.device_name())
    t0 = time.perf_counter()
    alloc, cache, tier_map, rows, host_rows = build_cache(m, shape, context, layers=layers)
    log(f"cache built in {time.perf_counter() - t0:.1f}s")

    heads, hd = shape.heads, shape.head_dim
    rng = np.random.default_rng(1)
    q_host = rng.standard_normal((layers, heads * hd)).astype(np.float32)
    qs = [m.upload_fp16(q_host[layer]) for layer in range(layers)]
    outs = [d.empty(heads * hd) for _ in range(layers)]
    partials = d.empty_f32(d.attention_partials(hd))
    scores = d.ImportanceScores(layers, context // P)

    def step():
        for layer in range(layers):
            kr, vr = rows[layer]
            cache.attention(layer, qs[layer], None, None, outs[layer], 1, context, heads,
                            shape.kv_heads, hd, kr, vr, None, partials, scores=scores)

    step()            # eager: resolves the page tables, sizes scratch
    m.synchronize()
    stream = m.Stream()
    graph = m.Graph(stream)
    with graph.capture():
        step()
    for _ in range(args.warmup):
        graph.launch()
    stream.synchronize()
    timer = m.Timer(stream)
    timer.start()
    for _ in range(args.steps):
        graph.launch()
    timer.stop()
    ms = timer.elapsed_ms() / args.steps
    stream.synchronize()

    per_layer = [layer_bytes(m, shape, tier_map[l], heads) for l in range(layers)]
    step_bytes = sum(per_layer)
    gbs = step_bytes / (ms * 1e-3) / 1e9
    us_token = ms * 1e3 * shape.layers / layers
    log(f"{ms * 1e3:.1f} us/step over {layers} layers: {gbs:.0f} GB/s")

    # The same step as one launch over every layer (a caller holding all
    # layers' queries at once): the streaming rate the kernel reaches when
    # one layer's latency does not bound it. Reported beside the value.
    q_all = m.upload_fp16(q_host.reshape(-1))
    out_all = d.empty(layers * heads * hd)
    k_all = m.upload_fp16(np.stack([host_rows[l][0][-1] for l in range(layers)]).reshape(-1)
                          .astype(np.float32))
    v_all = m.upload_fp16(np.stack([host_rows[l][1][-1] for l in range(layers)]).reshape(-1)
                          .astype(np.float32))
    scores_all = d.ImportanceScores(layers, context // P)

    def step_all():
        cache.attention_layers(0, layers, q_all, out_all, context, heads, shape.kv_heads, hd,
                               k_all, v_all, None, scores=scores_all)

    step_all()
    m.synchronize()
    graph_all = m.Graph(stream)
    with graph_all.capture():
        step_all()
    for _ in range(args.warmup):
        graph_all.launch()
    stream.synchronize()
    timer.start()
    for _ in range(args.steps):
        graph_all.launch()
    timer.stop()
    ms_all = timer.elapsed_ms() / args.steps
    stream.synchronize()
    gbs_all = step_bytes / (ms_all * 1e-3) / 1e9
    log(f"one launch over {layers} layers: {ms_all * 1e3:.1f} us/step, {gbs_all:.0f} GB/s")
    got_all = out_all.to_numpy().reshape(layers, 1, heads, hd)

    # Parity of both timed paths against the oracle on three layers.
    from oracle import attention as att
    for layer in sorted({0, layers // 2, layers - 1}):
        sealed = context // P - 1
        pages = [alloc.read(layer, i) for i in range(sealed)]
        tiers = [int(alloc.locate(layer, i)[0]) for i in range(sealed)]
        k, v = host_rows[layer]
        q = qs[layer].raw().reshape(1, heads, hd)
        want, _, bound = att.causal_decode(q, pages, tiers, k[sealed * P:], v[sealed * P:],
                                           shape.kv_heads, hd, P, with_bound=True)
        for name, got in (("per-layer", outs[layer].to_numpy().reshape(1, heads, hd)),
                          ("one-launch", got_all[layer])):
            check_gate(got, want, bound, f"layer {layer}: the {name} output")
    log("parity of both timed paths: ok")

    bias_on = decode_bias_on(m, shape, cache, alloc, host_rows, layers, context, stream,
                             args.steps, args.warmup, step_bytes)
    log(f"decode with the key bias on: {bias_on}")

    prefill = None
    if not args.no_prefill:
        prefill = {"tile": prefill_tile(m, shape, cache, alloc, host_rows, layers, context,
                                        stream, args.steps, args.warmup),
                   "chunks": prefill_chunks(m, stream, max(args.steps // 5, 3),
                                            max(args.warmup // 5, 1))}
        log(f"prefill: {prefill}")

    requant = None
    if not args.no_requant:
        t0 = time.perf_counter()
        requant = requant_plan(m, shape, context, layers=layers)
        log(f"requant plan in {time.perf_counter() - t0:.1f}s: {requant}")

    cpu = None
    if not args.no_cpu:
        sample = 2
        secs, nbytes = cpu_baseline(shape, context, sample)
        per_layer_s = secs / sample
        cpu = {"value": round(sum(per_layer[:sample]) / secs / 1e9, 4), "unit": "GB/s",
               "cores": 1, "kind": "port",
               "sample": f"{sample} layers of config 3 (32K, 1.5B shape), one decode each: "
                         f"float64 NumPy attention over the oracle-dequantised pages + fp32 EWMA, "
                         f"BLAS limited to 1 thread; {per_layer_s * 1e3:.0f} ms/layer = "
                         f"{per_layer_s * shape.layers * 1e3:.0f} ms/token",
               "us_per_token": round(per_layer_s * shape.layers * 1e6, 1)}

    result = {
        "metric": METRIC, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic: seeded N(0,1) fp16 K/V with 2% outlier K channels x10, "
                "tiers by seeded lognormal importance",
        "config": {"workload": "config3 decode attention + fused per-page mass/EWMA, "
                               "all layers per step (HIP graph of per-layer launches)",
                   "shape": "qwen2.5-1.5b 12q/2kv/hd128", "layers": layers,
                   "context": context, "page_tokens": P,
                   "tiers": "FP16/INT8/INT4/INT2 20/30/40/10 %", "parallelism": "single GPU"},
        "us_per_token": round(us_token, 2),
        "pct_hbm_peak": round(100 * gbs / PEAK_GBS, 2),
        "bytes_per_step": step_bytes,
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_GBS, 4), "traffic": profiled_traffic(),
                     "kernel": "decode_pages_kernel + decode_combine_kernel, one layer's "
                               "launch pair; achieved = algorithmic bytes a layer / live "
                               "per-layer time (HIP events on the graph's stream)",
                     "algorithmic_bytes_per_layer": round(step_bytes / layers),
                     "measured_copy_gb_per_s": round(copy_gbs, 1)},
        "one_launch_all_layers": {"us_per_token": round(ms_all * 1e3 * shape.layers / layers, 2),
                                  "gb_per_s": round(gbs_all, 1),
                                  "pct_hbm_peak": round(100 * gbs_all / PEAK_GBS, 2),
                                  "note": "same bytes and results; all layers' queries in one "
                                          "launch, not the per-layer decode order"},
        "cpu_baseline": cpu,
        "requant": requant,
        "decode_key_bias_on": bias_on,
        "prefill": prefill,
    }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
