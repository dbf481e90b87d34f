"""Benchmark of the paged mixed-precision KV-cache hot path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1]

The step: one decode step's attention over every layer
of a Qwen2.5-1.5B-shaped cache at 32K positions -- 28 layers, 12 query / 2 KV
heads, head_dim 128, 32-token pages born at seeded-importance tiers 20%
FP16, 30% INT8, 40% INT4, 10% INT2 -- with each layer's per-page attention
mass folded into its importance scores (EWMA) in the same pass. The 28
per-layer launches are captured once in a HIP graph and replayed; K steps are
timed with hipEvents on the stream they run on. Inputs are resident in HBM
before timing starts.

Also measured, outside the timed region: the requantisation plan of config 4
(batched moves, pages/s) and the CPU oracle on a bounded sample of the same
workload. Prints one JSON line.
"""

from __future__ import annotations

import argparse
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
            "downgrade_pages_per_s": len(down) / down_s, "restores_int4_to_int8": len(up),
            "restore_seconds": up_s, "restore_pages_per_s": len(up) / up_s,
            "shadows_taken": cache.last_batch and len(down)}


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
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--layers", type=int, default=None, help="fewer layers, for a quick look")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-requant", action="store_true")
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
        # The reference's error gate (tests/ulp_gate.py, tests/test_attention.py:58-115)
        # held to 1e-3: relative error floored at fp16's least normal and where the
        # fp32 error bound spends the budget.
        floor = np.maximum(att.FP16_MIN_NORMAL, bound / 1e-3)
        for name, got in (("per-layer", outs[layer].to_numpy().reshape(1, heads, hd)),
                          ("one-launch", got_all[layer])):
            err = np.abs(got - want) / np.maximum(np.abs(want), floor)
            if err.max() >= 1e-3 or err.mean() >= 2.0**-11:
                raise AssertionError(f"layer {layer}: the {name} output is off the oracle: "
                                     f"max {err.max():.3g}, mean {err.mean():.3g}")
    log("parity of both timed paths: ok")

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
    }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
