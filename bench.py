"""Benchmark: talker paged decode attention at 576 rows on one MI355X.

One step = one frame of the talker = 28 decode-attention layer calls (engine/talker.py:66-77) over
the 576-row workload: 518 live rows with ctx = round(exp(U[ln 64, ln 1800])), 58 padded rows with
ctx = 0, GQA 16/8, head_dim 128, bf16, 16-token pages, every layer with its own seeded random
page table over one 131,072-page pool (8.59 GB of K+V).  Inputs are resident in HBM before the
timed region.  Prints one JSON line.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--no-extra]
                  [--workload decode576|decode256|decode1x64|decode-small|decode-scaling|cp512|prefill32|admit|probe]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "qwen3-tts-engine_amd"))

HBM_PEAK_GBPS = 8000.0
METRIC = "paged decode attn µs/step and HBM GB/s (% peak) at 576 seats, 1×MI355X"
LAYERS = 28


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def host_cpus() -> dict:
    """The host's CPU facts: os.cpu_count(), the affinity mask, the cgroup CPU quota, and lscpu's model and
    socket/core/thread counts."""
    info = {"os_cpu_count": os.cpu_count(), "affinity": len(os.sched_getaffinity(0))}
    try:
        quota, period = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        info["cgroup_cpus"] = None if quota == "max" else round(int(quota) / int(period), 2)
    except (OSError, ValueError):
        info["cgroup_cpus"] = None
    keys = {"Model name": "model", "Socket(s)": "sockets", "Core(s) per socket": "cores_per_socket",
            "Thread(s) per core": "threads_per_core"}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for ln in out.splitlines():
            k, _, v = ln.partition(":")
            if k.strip() in keys:
                v = v.strip()
                info[keys[k.strip()]] = int(v) if v.isdigit() else v
    except Exception:
        pass
    if isinstance(info.get("sockets"), int) and isinstance(info.get("cores_per_socket"), int):
        info["lscpu_cores"] = info["sockets"] * info["cores_per_socket"]
    return info


def cpu_threads() -> int:
    """All of the host's cores for the CPU baselines: torch.set_num_threads(os.cpu_count())."""
    import torch

    n = os.cpu_count() or 1
    torch.set_num_threads(n)
    return torch.get_num_threads()


def cpu_baseline(wl, reps_min: int = 3, budget_s: float = 12.0):
    """The reference's per-row fp32 torch attention (engine/talker.py:82-88 with the page gather),
    on the host cores, over layer 0 of the same workload (all rows).  Reported per frame (x28)."""
    import numpy as np
    import torch

    from oracle.torch_cpu import paged_decode_rows

    L = wl.layers[0]
    page = wl.page_size
    bt = L.block_table.cpu().numpy().astype(np.int64)
    need = [bt[b, : (int(c) + page - 1) // page] for b, c in enumerate(wl.ctx)]
    uniq = np.unique(np.concatenate([n for n in need if len(n)]))
    remap = np.full(int(bt.max()) + 1, -1, np.int64)
    remap[uniq] = np.arange(len(uniq))
    table = np.zeros_like(bt)
    for b, n in enumerate(need):
        table[b, : len(n)] = remap[n]
    idx = torch.from_numpy(uniq).to(wl.k_cache.device)
    k = wl.k_cache.index_select(0, idx).float().cpu()
    v = wl.v_cache.index_select(0, idx).float().cpu()
    q = L.q.float().cpu()
    sl = torch.from_numpy(wl.ctx)
    tb = torch.from_numpy(table)
    threads = cpu_threads()
    paged_decode_rows(q, k, v, sl, tb, wl.scale)                # warm-up (two, as the reference's timing does)
    paged_decode_rows(q, k, v, sl, tb, wl.scale)
    times = []
    t_start = time.perf_counter()
    while len(times) < max(reps_min, 5) or (time.perf_counter() - t_start < budget_s and len(times) < 200):
        t0 = time.perf_counter()
        paged_decode_rows(q, k, v, sl, tb, wl.scale)
        times.append(time.perf_counter() - t0)
    per_call_us = statistics.median(times) * 1e6
    return {
        "value": round(per_call_us * LAYERS, 1),
        "unit": "us/step",
        "cores": threads,
        "kind": "port",
        "sample": (f"layer 0 of the same {wl.batch}-row workload (all rows, {int(wl.ctx.sum())} context tokens), "
                   f"median of {len(times)} calls of the reference's per-row fp32 torch loop "
                   f"(engine/talker.py:82-88 + page gather) = {per_call_us:.0f} us/call, x{LAYERS} layers per step; "
                   f"torch.set_num_threads(os.cpu_count() = {os.cpu_count()})"),
        "host": host_cpus(),
        "us_per_layer_call": round(per_call_us, 1),
        "gbps": round(wl.algorithmic_bytes() / (per_call_us * 1e-6) / 1e9, 2),
    }


def measured_traffic():
    """HBM bytes per decode-kernel launch from the committed rocprofv3 --pmc summary (FETCH_SIZE and
    WRITE_SIZE scaled by a plain-copy calibration), or None when the summary is absent."""
    path = os.path.join(ROOT, "profiles", "paged_decode_576rows.md")
    try:
        for ln in open(path):
            if ln.startswith("traffic_bytes_per_launch"):
                return int(ln.split("=")[1])
    except OSError:
        pass
    return None


def time_graph(dev, frame_fn, steps: int, warmup: int, min_warm_s: float = 0.0):
    """Capture frame_fn once into a HIP graph (as the engine does, engine/talker.py:115-137), check a replay
    against the eager result, then time `steps` replays with a HIP event pair around each.  The untimed warmup is
    `warmup` replays, continued until min_warm_s seconds have passed (the short extra runs set it, so the GPU's
    clocks are back up after the host-only CPU baselines).  Returns (wall ms per step, list of per-replay event ms)."""
    import torch

    stream = torch.cuda.Stream(dev)
    stream.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(stream):
        eager = [o.clone() for o in frame_fn()]
    torch.cuda.current_stream(dev).wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        static_out = frame_fn()
    graph.replay()
    torch.cuda.synchronize()
    if not all(torch.equal(a, b) for a, b in zip(static_out, eager)):
        raise RuntimeError("graph replay differs from the eager frame")
    cur = torch.cuda.current_stream(dev)
    t_warm = time.perf_counter()
    n = 0
    while n < warmup or time.perf_counter() - t_warm < min_warm_s:
        graph.replay()
        n += 1
        if min_warm_s and n % 8 == 0:
            torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    for i in range(steps):
        ev[i][0].record(cur)
        graph.replay()
        ev[i][1].record(cur)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_start
    return wall * 1e3 / steps, [a.elapsed_time(b) for a, b in ev], graph


def base_record(metric, value, unit, args, ms_per_step, higher_is_better, config):
    return {
        "metric": metric, "value": value, "unit": unit, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4), "higher_is_better": higher_is_better, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic", "config": config,
    }


def bench_decode(args, dev, name, cpu_budget_s: float = 12.0):
    import torch

    import q3attn
    from q3attn import workloads as W

    t0 = time.time()
    wl = W.make_decode(name, dev, layers=LAYERS, seed=args.seed)
    torch.cuda.synchronize()
    log(f"[bench] workload {name} built in {time.time() - t0:.1f} s: rows={wl.batch} live={(wl.ctx > 0).sum()} "
        f"sum_ctx={int(wl.ctx.sum())} pool={tuple(wl.k_cache.shape)}")
    nbytes = wl.algorithmic_bytes()

    def layer_call(L):
        return q3attn.paged_decode(L.q, wl.k_cache, wl.v_cache, wl.cache_seqlens, L.block_table,
                                   wl.scale, args.split)

    # The engine's frame passes one ctx and one table to all 28 calls (engine/talker.py:77, 107-112), so one plan per
    # frame serves them (q3attn.decode_plan); here each layer has its own table, so the frame's plan launch builds 28
    # plans, one per table, inside the timed graph.
    bts = torch.stack([L.block_table for L in wl.layers])
    plan_ok = args.split == 0 and not args.no_plan and q3attn.decode_plan(
        wl.cache_seqlens, bts, wl.page_size) is not None

    def planned_frame():
        plans = q3attn.decode_plan(wl.cache_seqlens, bts, wl.page_size)
        return [q3attn.paged_decode(L.q, wl.k_cache, wl.v_cache, wl.cache_seqlens, bts[i], wl.scale, plan=plans[i])
                for i, L in enumerate(wl.layers)]

    unplanned_ms, unplanned_frame_ms, _ = time_graph(dev, lambda: [layer_call(L) for L in wl.layers], args.steps,
                                                     args.warmup, getattr(args, "min_warm_s", 0.0))
    unplanned_us = statistics.mean(unplanned_frame_ms) * 1e3 / LAYERS
    log(f"[bench] unplanned: {args.steps} graph replays of {LAYERS} calls: events "
        f"{statistics.mean(unplanned_frame_ms):.3f} ms/frame = {unplanned_us:.1f} us/call")
    if plan_ok:
        ms_per_step, frame_ms, _ = time_graph(dev, planned_frame, args.steps, args.warmup,
                                              getattr(args, "min_warm_s", 0.0))
    else:
        ms_per_step, frame_ms = unplanned_ms, unplanned_frame_ms
    avg_call_us = statistics.mean(frame_ms) * 1e3 / LAYERS
    achieved = nbytes / (avg_call_us * 1e-6) / 1e9
    log(f"[bench] {'planned' if plan_ok else 'unplanned'}: {args.steps} graph replays of {LAYERS} calls: wall "
        f"{ms_per_step:.3f} ms/step; events {statistics.mean(frame_ms):.3f} ms/frame (min {min(frame_ms):.3f}) = "
        f"{avg_call_us:.1f} us/call; {achieved:.0f} GB/s = {achieved / HBM_PEAK_GBPS:.1%} of peak")

    # Eager calls with an event pair around each (host launch gaps excluded): extra information.
    cur = torch.cuda.current_stream(dev)
    eg = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(LAYERS)]
    for i, L in enumerate(wl.layers):
        eg[i][0].record(cur)
        layer_call(L)
        eg[i][1].record(cur)
    torch.cuda.synchronize()
    eager_call_us = statistics.mean(a.elapsed_time(b) for a, b in eg) * 1e3

    append = None
    if not args.no_append:
        append = bench_decode_append(args, dev, wl)

    cpu = None
    if not args.no_cpu_baseline:
        t0 = time.time()
        cpu = cpu_baseline(wl, budget_s=cpu_budget_s)
        log(f"[bench] cpu baseline {cpu['us_per_layer_call']:.0f} us/call in {time.time() - t0:.1f} s")

    if name == "decode576":
        desc = ("talker paged decode attention, 576 rows (518 live, ctx log-uniform [64,1800]; 58 padded ctx=0), "
                "GQA 16/8, head_dim 128, bf16 K/V, fp32 softmax/accumulate, 16-token pages, 131072-page pool, "
                "28 layer calls per step with per-layer random tables")
        metric = METRIC
    elif name == "decode256":
        desc = (f"talker paged decode attention, {wl.batch} rows, ctx U[200,1200], GQA 16/8, head_dim 128, bf16, "
                "16-token pages, 65536-page pool, 28 layer calls per step with per-layer random tables")
        metric = f"paged decode attn µs/step and HBM GB/s (% peak) at {wl.batch} seats, 1×MI355X"
    else:
        desc = ("talker paged decode attention, 1 row of 64 tokens, GQA 16/8, head_dim 128, bf16, 16-token pages, "
                "identity table, 28 layer calls per step")
        metric = "paged decode attn µs/step at 1 seat x 64 tokens, 1×MI355X"
    rec = base_record(metric, round(ms_per_step * 1e3, 2), "us/step", args, ms_per_step, False, {
        "workload": desc, "rows": wl.batch, "sum_ctx": int(wl.ctx.sum()), "layers_per_step": LAYERS,
        "split_tokens": args.split or "stream-K", "parallelism": "single GPU",
        "decode_plan": "one plan launch per frame (28 tables) inside the timed graph" if plan_ok else "none"})
    rec.update({
        "us_per_layer_call": round(avg_call_us, 2),
        "us_per_layer_call_unplanned": round(unplanned_us, 2),
        "us_per_layer_call_eager": round(eager_call_us, 2),
        "hbm_gbps": round(achieved, 1),
        "pct_hbm_peak": round(100 * achieved / HBM_PEAK_GBPS, 2),
        "roofline": {
            "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": measured_traffic() if name == "decode576" else None,
            "kernel": decode_kernel_name(wl, args.split, plan_ok) + ", per call inside the graph",
            "bytes_per_call": nbytes,
        },
        "cpu_baseline": cpu,
    })
    if append is not None:
        rec["append_form"] = append
    return rec


def make_planned_frame(wl, bts):
    """A frame of the workload's layer calls with the frame's plan (q3attn.decode_plan over the stacked per-layer
    tables, built inside the frame), or None when the library has no plan for the shape."""
    import q3attn

    if q3attn.decode_plan(wl.cache_seqlens, bts, wl.page_size) is None:
        return None

    def frame():
        plans = q3attn.decode_plan(wl.cache_seqlens, bts, wl.page_size)
        return [q3attn.paged_decode(L.q, wl.k_cache, wl.v_cache, wl.cache_seqlens, bts[i], wl.scale, plan=plans[i])
                for i, L in enumerate(wl.layers)]
    return frame


def decode_kernel_name(wl, split, planned=False):
    """The kernels one decode call of this workload launches (the library needs no workspace exactly when it takes
    the row-parallel path, for split 0)."""
    from q3attn import _lib

    if planned:
        return "paged decode call (planned stream-K decode kernel + combine kernel; the frame's plan kernel shared)"

    L = wl.layers[0]
    lib = _lib.lib()
    ws = lambda code: lib.q3a_paged_decode_workspace_bytes(wl.batch, 16, wl.k_cache.shape[2], 128,
                                                           L.block_table.shape[1], wl.page_size, code)
    if split > 0:
        return "paged decode call (fixed-split decode kernel + combine kernel)"
    if split == -1 or (split == 0 and ws(0) == 0):
        return "paged decode call (row-parallel kernel, one launch)"
    if split == -2 or (split == 0 and ws(0) == ws(-2)):
        return "paged decode call (chunked decode kernel + chunk combine kernel)"
    return "paged decode call (stream-K decode kernel + combine kernel)"


SMALL_SHAPES = ((1, 64), (1, 256), (1, 1024), (1, 1800), (2, 1800), (4, 1024), (4, 1800), (8, 512), (8, 1800),
                (16, 1024), (16, 1800), (32, 512), (32, 1024), (32, 1800), (64, 256), (64, 512), (64, 1024))
SMALL_PATHS = (("row_parallel", -1), ("chunks", -2), ("stream_k", -3), ("auto", 0))


PLAN_SWEEP = ((96, "log"), (128, "log"), (256, "uniform"), (384, "log"), (576, "log"), (1024, "log"),
              (2048, "uniform"), (4096, "short"))


def bench_decode_plan_sweep(args, dev):
    """The frame's plan against no plan over batch sizes the library decodes with stream-K: rows' contexts
    log-uniform in [64, 1800] ("log"), uniform in [200, 1200] ("uniform") or in [16, 300] ("short"); 8 layer calls per
    graph replay, each with its own random table over a pool sized to the batch; unplanned and planned frames timed
    twice each, alternating."""
    import numpy as np
    import torch

    import q3attn
    from q3attn import workloads as W

    layers = 8
    out = {}
    for B, kind in PLAN_SWEEP:
        rng = np.random.default_rng(B)
        if kind == "log":
            ctx = np.exp(rng.uniform(np.log(64), np.log(1800), B)).astype(np.int64)
        elif kind == "uniform":
            ctx = rng.integers(200, 1201, B)
        else:
            ctx = rng.integers(16, 300, B)
        maxc = int(ctx.max()) + 16
        wl = W.make_decode("plan-sweep", dev, layers=layers, ctx=ctx, num_pages=B * -(-maxc // 16) + 64,
                           max_ctx=maxc, seed=B)
        bts = torch.stack([L.block_table for L in wl.layers])
        unplanned = lambda: [q3attn.paged_decode(L.q, wl.k_cache, wl.v_cache, wl.cache_seqlens, L.block_table,
                                                 wl.scale, 0) for L in wl.layers]
        planned = make_planned_frame(wl, bts)
        t = {"unplanned": [], "planned": []}
        for name, fn in (("unplanned", unplanned), ("planned", planned)) * 2:
            if fn is not None:
                _, ms, _ = time_graph(dev, fn, args.steps, args.warmup, 0.5)
                t[name].append(round(statistics.mean(ms) * 1e3 / layers, 2))
        out[f"{B}x{kind}"] = {"tiles": int(((ctx + 15) // 16).sum()), "unplanned_us_per_call": t["unplanned"],
                              "planned_us_per_call": t["planned"]}
        log(f"[bench] {B} rows ({kind}): unplanned {t['unplanned']} planned {t['planned']} us/call")
        del wl
        torch.cuda.empty_cache()
    gains = [statistics.mean(r["unplanned_us_per_call"]) / statistics.mean(r["planned_us_per_call"])
             for r in out.values() if r["planned_us_per_call"]]
    rec = base_record("paged decode attn speed-up of the frame's plan (mean over batch sizes), 1×MI355X",
                      round(statistics.mean(gains), 4), "x", args, 0.0, True, {
                          "workload": "talker paged decode attention, 96-4,096 rows, 8 layer calls per step with "
                                      "per-layer random tables, with and without the frame's plan",
                          "shapes": list(out), "parallelism": "single GPU"})
    rec["per_shape"] = out
    return rec


def bench_decode_scaling(args, dev):
    """The 576-row workload with every row's context scaled by 1/2, 1 and 2 (the same rows, each scale its own
    131,072-page pool and tables of the scaled capacity, all three built first; 28 layer calls per graph replay, each
    timing after a second of warm replays), timed in the order 1, 1/2, 2, 2, 1/2, 1 so that a drift of the GPU's
    clocks over the run falls on every scale alike.  The least-squares line through (bytes per call, mean us per call)
    gives the decode's marginal read rate (its slope) and its fixed cost per call (its intercept), the figures to set
    beside the access pattern's own ceiling (`--workload probe`)."""
    import numpy as np
    import torch

    import q3attn
    from q3attn import workloads as W

    base = W.draw_contexts("decode576", args.seed)
    scales = (0.5, 1.0, 2.0)
    wls = {}
    for scale in scales:
        ctx = np.rint(base * scale).astype(np.int64)
        wls[scale] = W.make_decode("decode576", dev, layers=LAYERS, seed=args.seed, ctx=ctx,
                                   max_ctx=int(math.ceil(W.MAX_CTX["decode576"] * scale)))
    times = {scale: [] for scale in scales}
    ptimes = {scale: [] for scale in scales}   # the same frames with the frame's plan
    bts = {scale: torch.stack([L.block_table for L in wls[scale].layers]) for scale in scales}
    for scale in (1.0, 0.5, 2.0, 2.0, 0.5, 1.0):
        wl = wls[scale]
        _, frame_ms, _ = time_graph(dev, lambda: [q3attn.paged_decode(L.q, wl.k_cache, wl.v_cache, wl.cache_seqlens,
                                                                       L.block_table, wl.scale, args.split)
                                                  for L in wl.layers], args.steps, args.warmup, 1.0)
        us = statistics.mean(frame_ms) * 1e3 / LAYERS
        times[scale].append(us)
        pf = make_planned_frame(wl, bts[scale])
        pus = float("nan")
        if pf is not None:
            _, frame_ms, _ = time_graph(dev, pf, args.steps, args.warmup, 1.0)
            pus = statistics.mean(frame_ms) * 1e3 / LAYERS
            ptimes[scale].append(pus)
        log(f"[bench] contexts x{scale}: {us:.1f} us/call, {pus:.1f} with the frame's plan")
    pts = []
    for scale in scales:
        wl = wls[scale]
        nbytes = wl.algorithmic_bytes()
        us = statistics.mean(times[scale])
        pts.append({"ctx_scale": scale, "sum_ctx": int(wl.ctx.sum()), "bytes_per_call": nbytes,
                    "us_per_layer_call": [round(t, 2) for t in times[scale]], "gbps": round(nbytes / us / 1e3, 1)})
        log(f"[bench] contexts x{scale}: sum_ctx {int(wl.ctx.sum())}, {nbytes / 1e6:.1f} MB per call, "
            f"{us:.1f} us/call (mean of {len(times[scale])}), {nbytes / us / 1e3:.0f} GB/s")
    del wls
    torch.cuda.empty_cache()
    x = np.array([p["bytes_per_call"] for p in pts], dtype=np.float64)
    y = np.array([statistics.mean(times[p["ctx_scale"]]) for p in pts], dtype=np.float64)
    slope, icpt = np.polyfit(x, y, 1)
    rate = 1.0 / slope / 1e3  # bytes per us -> GB/s
    log(f"[bench] least squares over the three scales: marginal rate {rate:.0f} GB/s = {rate / HBM_PEAK_GBPS:.1%} of "
        f"peak, fixed cost {icpt:.1f} us per call")
    rec = {"metric": "paged decode us/call against bytes/call at context scales 1/2, 1, 2 (576 rows)",
           "points": pts, "marginal_gbps": round(float(rate), 1),
           "marginal_pct_peak": round(float(rate) / HBM_PEAK_GBPS * 100, 2), "fixed_us_per_call": round(float(icpt), 2)}
    if all(ptimes[sc] for sc in scales):
        yp = np.array([statistics.mean(ptimes[p["ctx_scale"]]) for p in pts], dtype=np.float64)
        pslope, picpt = np.polyfit(x, yp, 1)
        prate = 1.0 / pslope / 1e3
        for p in pts:
            p["us_per_layer_call_planned"] = [round(t, 2) for t in ptimes[p["ctx_scale"]]]
        rec["planned"] = {"marginal_gbps": round(float(prate), 1),
                          "marginal_pct_peak": round(float(prate) / HBM_PEAK_GBPS * 100, 2),
                          "fixed_us_per_call": round(float(picpt), 2)}
        log(f"[bench] with the frame's plan: marginal rate {prate:.0f} GB/s = {prate / HBM_PEAK_GBPS:.1%} of peak, "
            f"fixed cost {picpt:.1f} us per call")
    return rec


def bench_decode_small(args, dev):
    """Decode at small batches: every row of B rows at the same context length, 28 layer calls per graph replay
    over one pool with per-layer random 2,048-token tables.  Each shape runs through each kernel (the path codes
    force one: the row-parallel kernel, the chunked kernel + its combine, stream-K + its combine) and through the
    library's own choice (`auto`, the headline value)."""
    import numpy as np
    import torch

    import q3attn
    from q3attn import workloads as W

    shapes = {}
    for B, ctx in SMALL_SHAPES:
        res = {}
        wl = W.make_decode("small", dev, ctx=np.full(B, ctx), num_pages=max(256, B * 130 * 2), max_ctx=2048,
                           layers=LAYERS, seed=args.seed + 1)
        for path, code in SMALL_PATHS:
            _, frame_ms, _ = time_graph(dev, lambda: [q3attn.paged_decode(L.q, wl.k_cache, wl.v_cache, wl.cache_seqlens,
                                                                          L.block_table, wl.scale, code)
                                                      for L in wl.layers], args.steps, args.warmup)
            res[path] = round(statistics.median(frame_ms) * 1e3 / LAYERS, 2)
        res["auto_kernel"] = decode_kernel_name(wl, 0)
        del wl
        torch.cuda.empty_cache()
        shapes[f"{B}x{ctx}"] = res
        log(f"[bench] small batch {B} x {ctx}: row-parallel {res['row_parallel']:.2f}, chunks {res['chunks']:.2f}, "
            f"stream-K {res['stream_k']:.2f}, auto {res['auto']:.2f} us/call ({res['auto_kernel']})")
    mean_auto = statistics.mean(r["auto"] for r in shapes.values())
    rec = base_record("paged decode attn µs/call at small batches (mean over shapes), 1×MI355X", round(mean_auto, 2),
                      "us/call", args, mean_auto * LAYERS / 1e3, False, {
                          "workload": "talker paged decode attention at 1-64 rows of 64-1,800 tokens each, GQA 16/8, "
                                      "head_dim 128, bf16, 16-token pages, 2,048-token tables, 28 layer calls per step",
                          "shapes": [f"{B}x{c}" for B, c in SMALL_SHAPES], "parallelism": "single GPU"})
    rec["per_shape_us_per_call"] = shapes
    return rec


def bench_decode_small_lite(args, dev):
    """The driver line's short small-batch entry: 1 x 1,024, 1 x 1,800 and 8 x 1,800 tokens on 2,048-token tables,
    through the library's choice (the chunked kernel) and the row-parallel kernel, µs per call in a 28-call graph."""
    import numpy as np
    import torch

    import q3attn
    from q3attn import workloads as W

    shapes = {}
    for B, ctx in ((1, 1024), (1, 1800), (8, 1800)):
        wl = W.make_decode("small", dev, ctx=np.full(B, ctx), num_pages=max(256, B * 130 * 2), max_ctx=2048,
                           layers=LAYERS, seed=args.seed + 1)
        res = {}
        for path, code in (("auto", 0), ("row_parallel", -1)):
            _, frame_ms, _ = time_graph(dev, lambda: [q3attn.paged_decode(L.q, wl.k_cache, wl.v_cache, wl.cache_seqlens,
                                                                          L.block_table, wl.scale, code)
                                                      for L in wl.layers], args.steps, args.warmup,
                                        getattr(args, "min_warm_s", 0.0))
            res[path] = round(statistics.median(frame_ms) * 1e3 / LAYERS, 2)
        res["auto_kernel"] = decode_kernel_name(wl, 0)
        shapes[f"{B}x{ctx}"] = res
        del wl
        torch.cuda.empty_cache()
    mean_auto = statistics.mean(r["auto"] for r in shapes.values())
    return {"value": round(mean_auto * LAYERS, 2), "per_shape_us_per_call": shapes}


def bench_decode_append(args, dev, wl):
    """Extra information beside the headline: the same frame with this step's K/V append included, once as the
    engine does it (two index_copy_ scatters per layer, engine/talker.py:72-73, then the decode call) and once
    fused (paged_decode_append).  Each layer's new token is its row's last context token; the step's k/v rows
    are that slot's current contents, so the frame rewrites identical values and stays replayable."""
    import numpy as np
    import torch

    import q3attn

    page = wl.page_size
    live = wl.ctx > 0
    pos = np.where(live, wl.ctx - 1, 0)
    old = torch.from_numpy(wl.ctx - 1).to(torch.int32).to(dev)
    kflat = wl.k_cache.view(-1, wl.k_cache.shape[2], wl.k_cache.shape[3])
    vflat = wl.v_cache.view(-1, wl.v_cache.shape[2], wl.v_cache.shape[3])
    steps = []
    for L in wl.layers:
        bt = L.block_table.cpu().numpy().astype(np.int64)
        slot = bt[np.arange(wl.batch), pos // page] * page + pos % page
        # padded rows (ctx 0) write nothing in the fused form; the scatter form writes them to a scratch slot
        # (the reference sends padded rows to a scratch seat) -- here slot 0 with its own value
        slot = torch.from_numpy(np.where(live, slot, 0)).to(dev)
        steps.append((L, slot, kflat.index_select(0, slot), vflat.index_select(0, slot)))

    def fused():
        return [q3attn.paged_decode_append(L.q, k, v, wl.k_cache, wl.v_cache, old, L.block_table, wl.scale,
                                           args.split) for (L, _, k, v) in steps]

    def scatter_then_decode():
        out = []
        for (L, slot, k, v) in steps:
            kflat.index_copy_(0, slot, k)
            vflat.index_copy_(0, slot, v)
            out.append(q3attn.paged_decode(L.q, wl.k_cache, wl.v_cache, wl.cache_seqlens, L.block_table, wl.scale,
                                           args.split))
        return out

    # The frame's plan (one per layer table, built in the frame) for the planned forms.
    bts = torch.stack([L.block_table for (L, _, _, _) in steps])
    planned = args.split == 0 and not args.no_plan and q3attn.decode_plan(old, bts, page, form="append") is not None

    def fused_planned():
        plans = q3attn.decode_plan(old, bts, page, form="append")
        return [q3attn.paged_decode_append(L.q, k, v, wl.k_cache, wl.v_cache, old, bts[i], wl.scale, plan=plans[i])
                for i, (L, _, k, v) in enumerate(steps)]

    _, fr_split, _ = time_graph(dev, scatter_then_decode, args.steps, args.warmup)
    _, fr_fused, _ = time_graph(dev, fused, args.steps, args.warmup)
    a = statistics.mean(fr_fused) * 1e3 / LAYERS
    b = statistics.mean(fr_split) * 1e3 / LAYERS
    rec = {"fused_us_per_layer_call": round(a, 2), "index_copy_then_decode_us_per_layer_call": round(b, 2),
           "fused_us_per_step": round(a * LAYERS, 1), "index_copy_then_decode_us_per_step": round(b * LAYERS, 1)}
    msg = ""
    if planned:
        _, fr_plan, _ = time_graph(dev, fused_planned, args.steps, args.warmup)
        c = statistics.mean(fr_plan) * 1e3 / LAYERS
        rec["fused_planned_us_per_layer_call"] = round(c, 2)
        msg = f"; fused with the frame's plan {c:.1f}"
    log(f"[bench] append form: fused {a:.1f} us/layer call; index_copy_ x2 + decode {b:.1f} us/layer call{msg}")
    rec["norm_rope_form"] = bench_decode_rope(args, dev, wl, steps, old, bts if planned else None)
    return rec


def bench_decode_rope(args, dev, wl, steps, old, bts=None):
    """The talker's whole attention block per layer (engine/talker.py:69-77): q/k RMSNorm + RoPE, the K/V append and
    the decode, three ways over the same frame: paged_decode_append_rope (one launch); paged_decode_append on q and k
    normalised beforehand (the attention and append alone, what the producers cost nothing in); and the producers as
    eager torch ops (engine/ops.py:51-60) followed by paged_decode_append.  The raw rows are the append form's; the
    slots the frame rewrites are restored afterwards."""
    import numpy as np
    import torch

    import q3attn
    from q3attn import workloads as W

    rng = np.random.default_rng(3)
    qn = torch.from_numpy(rng.uniform(0.5, 1.5, 128).astype(np.float32)).to(dev).to(torch.bfloat16)
    kn = torch.from_numpy(rng.uniform(0.5, 1.5, 128).astype(np.float32)).to(dev).to(torch.bfloat16)
    cos_t, sin_t = W.rope_tables(int(wl.ctx.max()) + 1, dev)
    pos = torch.from_numpy(np.maximum(wl.ctx - 1, 0)).to(dev)
    cos = cos_t[pos].to(torch.bfloat16)[:, None, :]
    sin = sin_t[pos].to(torch.bfloat16)[:, None, :]
    kflat = wl.k_cache.view(-1, wl.k_cache.shape[2], wl.k_cache.shape[3])
    vflat = wl.v_cache.view(-1, wl.v_cache.shape[2], wl.v_cache.shape[3])
    saved = [(slot, kflat.index_select(0, slot), vflat.index_select(0, slot)) for (_, slot, _, _) in steps]

    def rms(x, w, eps=1e-6):
        xf = x.float()
        xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
        return w * xf.to(x.dtype)

    def rope(x):
        h = x.shape[-1] // 2
        return x * cos + torch.cat((-x[..., h:], x[..., :h]), dim=-1) * sin

    def fused():
        return [q3attn.paged_decode_append_rope(L.q, k, v, qn, kn, cos, sin, wl.k_cache, wl.v_cache, old,
                                                L.block_table, wl.scale) for (L, _, k, v) in steps]

    def append_only():
        return [q3attn.paged_decode_append(L.q, k, v, wl.k_cache, wl.v_cache, old, L.block_table, wl.scale)
                for (L, _, k, v) in steps]

    def fused_planned():
        plans = q3attn.decode_plan(old, bts, wl.page_size, form="append_rope")
        return [q3attn.paged_decode_append_rope(L.q, k, v, qn, kn, cos, sin, wl.k_cache, wl.v_cache, old, bts[i],
                                                wl.scale, plan=plans[i]) for i, (L, _, k, v) in enumerate(steps)]

    def eager_producers():
        return [q3attn.paged_decode_append(rope(rms(L.q, qn)), rope(rms(k, kn)), v, wl.k_cache, wl.v_cache, old,
                                           L.block_table, wl.scale) for (L, _, k, v) in steps]

    res = {}
    forms = [("append_on_normalised", append_only), ("fused", fused), ("torch_producers_then_append", eager_producers)]
    if bts is not None:
        forms.append(("fused_planned", fused_planned))
    for name, fn in forms:
        # The layers share one pool, so a layer can read a slot another layer rewrites: one untimed frame first
        # leaves every slot at the value the frame writes, and the replays then see the state the eager frame saw.
        fn()
        torch.cuda.synchronize()
        _, fr, _ = time_graph(dev, fn, args.steps, args.warmup)
        res[f"{name}_us_per_layer_call"] = round(statistics.mean(fr) * 1e3 / LAYERS, 2)
    for slot, k, v in saved:
        kflat.index_copy_(0, slot, k)
        vflat.index_copy_(0, slot, v)
    torch.cuda.synchronize()
    log(f"[bench] norm/rope form: fused {res['fused_us_per_layer_call']:.1f} us/layer call; append on normalised "
        f"q/k {res['append_on_normalised_us_per_layer_call']:.1f}; torch producers + append "
        f"{res['torch_producers_then_append_us_per_layer_call']:.1f}" +
        (f"; fused with the frame's plan {res['fused_planned_us_per_layer_call']:.1f}" if bts is not None else ""))
    return res


def bench_cp(args, dev):
    """Code predictor: 512 rows, 16 steps x 5 layers per frame (engine/code_predictor.py:52-69).  Each call is
    the slot write of step p plus the attention over slots 0..p: the fused cp_attn_append launch is timed, and
    beside it the engine's three-launch form (K.index_copy_, V.index_copy_, attention; code_predictor.py:58)."""
    import torch

    import q3attn
    from q3attn import workloads as W

    B, L = 512, 5
    scale = W.HEAD_DIM ** -0.5
    layers = [W.make_cp(B, dev, seed=args.seed + l) for l in range(L)]
    gen = torch.Generator(device=dev).manual_seed(args.seed + 99)
    rows = {}
    for l in range(L):
        for p in range(16):
            qkv = torch.randn(B, 4096, generator=gen, device=dev).to(torch.bfloat16)
            rows[l, p] = (qkv[:, 2048:3072].view(B, 8, 128).contiguous(), qkv[:, 3072:].view(B, 8, 128))
    pidx = [torch.tensor([p], device=dev) for p in range(16)]
    order = [(p, l) for p in range(16) for l in range(L)]
    nbytes = sum(W.cp_bytes(B, p + 1, append=True) for (p, _) in order)

    def fused():
        return [q3attn.cp_attn_append(layers[l][0][p], *rows[l, p], layers[l][1], layers[l][2], p, scale)
                for (p, l) in order]

    def three_launch():
        out = []
        for (p, l) in order:
            _, K, V = layers[l]
            k, v = rows[l, p]
            K.index_copy_(2, pidx[p], k.unsqueeze(2))
            V.index_copy_(2, pidx[p], v.unsqueeze(2))
            out.append(q3attn.cp_attn(layers[l][0][p], K, V, p + 1, scale))
        return out

    warm_s = getattr(args, "min_warm_s", 0.0)
    ms_split, frame_split, _ = time_graph(dev, three_launch, args.steps, args.warmup, warm_s)
    ms_per_step, frame_ms, graph = time_graph(dev, fused, args.steps, args.warmup, warm_s)
    frame_us = statistics.mean(frame_ms) * 1e3
    split_us = statistics.mean(frame_split) * 1e3
    # The same frame with the 256 MB Infinity Cache and the L2s flushed before each replay (a 512 MiB read-modify-write
    # between frames, outside the timed events): in the engine the code predictor's weights stream between steps, so
    # the scratch is not necessarily cache-resident when a step starts.
    evict = torch.zeros(256 << 20, dtype=torch.float16, device=dev)
    cur = torch.cuda.current_stream(dev)
    cold = []
    for _ in range(max(5, args.steps // 2)):
        evict.add_(1)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(cur)
        graph.replay()
        e1.record(cur)
        torch.cuda.synchronize()
        cold.append(e0.elapsed_time(e1) * 1e3)
    del evict
    cold_us = statistics.median(cold)
    # Launch floor: a graph of as many one-workgroup kernels (a one-element add) as the frame has calls, in one stream.
    tiny = torch.zeros(1, device=dev)
    _, floor_ms, _ = time_graph(dev, lambda: [tiny + 1 for _ in order], args.steps, args.warmup)
    floor_us = statistics.mean(floor_ms) * 1e3 / len(order)
    call_us = frame_us / len(order)
    achieved = nbytes / (frame_us * 1e-6) / 1e9
    log(f"[bench] cp: {len(order)} calls per frame, fused {frame_us:.1f} us/frame = {call_us:.2f} us/call "
        f"(cache-flushed frame {cold_us:.1f} us); index_copy_ x2 + attention {split_us:.1f} us/frame; launch floor "
        f"{floor_us:.2f} us/call; {achieved:.0f} GB/s algorithmic")
    norm_rope = bench_cp_rope(args, dev, layers, order, B, L, scale)
    cpu = None
    if not args.no_cpu_baseline:
        from oracle.torch_cpu import cp_attn_rows
        threads = cpu_threads()
        qs, K, V = layers[0]
        qc, Kc, Vc = [t.cpu() for t in qs], K.cpu(), V.cpu()
        rc = [(rows[0, p][0].cpu(), rows[0, p][1].cpu()) for p in range(16)]
        times = []
        for rep in range(3):
            t0 = time.perf_counter()
            for p in range(16):
                Kc[:, :, p] = rc[p][0]
                Vc[:, :, p] = rc[p][1]
                cp_attn_rows(qc[p], Kc, Vc, p + 1, scale)
            times.append(time.perf_counter() - t0)
        us = statistics.median(times) * 1e6 * L
        cpu = {"value": round(us, 1), "unit": "us/step", "cores": threads, "kind": "port",
               "sample": f"one layer's 16 steps (slot write + attention) at B={B} with the reference's torch bf16 "
                         f"ops on CPU (engine/code_predictor.py:46-47,58), median of 3, x{L} layers"}
    rec = base_record("code-predictor slot write + attention µs/step (16 steps x 5 layers) at 512 rows, 1×MI355X",
                      round(ms_per_step * 1e3, 2), "us/step", args, ms_per_step, False,
                      {"workload": "code-predictor 16-slot causal attention with the step's K/V slot write, 512 rows, "
                                   "GQA 16/8, head_dim 128, bf16, n_live 1..16, 5 layers per step",
                       "rows": B, "calls_per_step": len(order), "parallelism": "single GPU"})
    rec.update({"us_per_call": round(call_us, 3),
                "three_launch_us_per_step": round(split_us, 2),
                "cold_us_per_step": round(cold_us, 2), "cold_us_per_call": round(cold_us / len(order), 3),
                "launch_floor_us_per_call": round(floor_us, 3),
                "algorithmic_gbps": round(achieved, 1), "bytes_per_step": nbytes,
                # 2.1-37.7 MB per call and ~2 flop/B: the call is bound by launch and memory latency, so the roofline
                # is the latency floor of one dependent kernel in the same graph harness (frac = floor / achieved)
                "roofline": {"bound": "latency", "achieved": round(call_us, 3), "peak": round(floor_us, 3),
                             "unit": "us/call", "frac": round(floor_us / call_us, 4), "traffic": None},
                "cpu_baseline": cpu})
    if norm_rope is not None:
        rec["norm_rope_form"] = norm_rope
    return rec


def bench_cp_rope(args, dev, layers, order, B, L, scale):
    """Extra information beside the code-predictor line: the frame with the step's q/k producers
    (engine/code_predictor.py:38-43) folded into the attention call, cp_attn_append_rope on the raw projections,
    against the producers as separate ops before cp_attn_append: compiled by torch.compile as the engine compiles
    _pre (skipped in the short extra runs, whose time budget does not cover a compile) and as eager torch ops.
    Synthetic qkv projections and norm weights; slot p's cos/sin rows."""
    import torch

    import q3attn
    from q3attn import workloads as W

    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed + 98)
    bf = torch.bfloat16
    qkv = {(p, l): torch.randn(B, 4096, generator=gen, device=dev).to(bf) for (p, l) in order}
    qn = [(1.0 + 0.1 * torch.randn(128, generator=gen, device=dev)).to(bf) for _ in range(L)]
    kn = [(1.0 + 0.1 * torch.randn(128, generator=gen, device=dev)).to(bf) for _ in range(L)]
    cos, sin = W.rope_tables(16, dev)
    cos, sin = cos.to(bf), sin.to(bf)

    def producers(x, qw, kw, c, s_):
        def rms(t, w):
            tf = t.float()
            tf = tf * torch.rsqrt(tf.pow(2).mean(-1, keepdim=True) + 1e-6)
            return w * tf.to(t.dtype)

        def rope(t):
            return t * c + torch.cat((-t[..., 64:], t[..., :64]), dim=-1) * s_
        return rope(rms(x[:, :2048].view(B, 16, 128), qw)), rope(rms(x[:, 2048:3072].view(B, 8, 128), kw))

    def fused():
        return [q3attn.cp_attn_append_rope(qkv[p, l][:, :2048].view(B, 16, 128), qkv[p, l][:, 2048:3072].view(B, 8, 128),
                                           qkv[p, l][:, 3072:].view(B, 8, 128), layers[l][1], layers[l][2], p, scale,
                                           qn[l], kn[l], cos[p], sin[p]) for (p, l) in order]

    def separate(fn):
        def frame():
            out = []
            for (p, l) in order:
                q, k = fn(qkv[p, l], qn[l], kn[l], cos[p], sin[p])
                out.append(q3attn.cp_attn_append(q, k, qkv[p, l][:, 3072:].view(B, 8, 128), layers[l][1],
                                                 layers[l][2], p, scale))
            return out
        return frame

    warm_s = getattr(args, "min_warm_s", 0.0)
    res = {}
    forms = [("fused", fused), ("eager_producers_then_append", separate(producers))]
    if not getattr(args, "no_compile", False):
        forms.append(("compiled_producers_then_append", separate(torch.compile(producers, dynamic=False))))
    for name, fn in forms:
        try:
            _, fr, _ = time_graph(dev, fn, args.steps, args.warmup, warm_s)
            res[name + "_us_per_step"] = round(statistics.mean(fr) * 1e3, 2)
        except Exception as e:  # noqa: BLE001 - a compile failure is reported, never fatal
            res[name + "_us_per_step"] = None
            res[name + "_error"] = f"{type(e).__name__}: {e}"[:200]
    log(f"[bench] cp norm/rope form: fused {res['fused_us_per_step']} us/frame; eager producers + append "
        f"{res['eager_producers_then_append_us_per_step']}; compiled producers + append "
        f"{res.get('compiled_producers_then_append_us_per_step')}")
    return res


def bench_prefill(args, dev):
    """Prompt prefill, 32 sequences, lengths U[150,400], K/V read from the paged pool, 28 layers per step,
    each layer with its own q/k/v."""
    import torch

    import q3attn
    from q3attn import workloads as W

    lens = W.prefill_lengths("prefill32", args.seed)
    wls = [W.make_prefill(dev, lens, seed=args.seed + l, paged=True, num_pages=4096) for l in range(LAYERS)]
    w0 = wls[0]

    def call(wl):
        return q3attn.flash_attn_varlen_func(wl.q, wl.k_cache, wl.v_cache, wl.cu_seqlens, wl.cu_seqlens, wl.max_len,
                                             wl.max_len, softmax_scale=wl.scale, causal=True,
                                             block_table=wl.block_table)

    ms_per_step, frame_ms, _ = time_graph(dev, lambda: [call(wl) for wl in wls], args.steps, args.warmup,
                                          getattr(args, "min_warm_s", 0.0))
    call_us = statistics.mean(frame_ms) * 1e3 / LAYERS
    tflops = w0.flops() / (call_us * 1e-6) / 1e12
    gbps = w0.algorithmic_bytes() / (call_us * 1e-6) / 1e9
    log(f"[bench] c4 prefill: {call_us:.1f} us/call, {tflops:.1f} TFLOP/s, {gbps:.0f} GB/s algorithmic")
    prompt_step = None if args.no_append else bench_prefill_append(args, dev, wls)
    cpu = None
    if not args.no_cpu_baseline:
        from oracle.torch_cpu import prefill_rows
        threads = cpu_threads()
        q, k, v = w0.q.float().cpu(), w0.k.float().cpu(), w0.v.float().cpu()
        cu = w0.cu_seqlens.cpu()
        times = []
        for rep in range(3):
            t0 = time.perf_counter()
            prefill_rows(q, k, v, cu, w0.scale)
            times.append(time.perf_counter() - t0)
        us = statistics.median(times) * 1e6
        cpu = {"value": round(us * LAYERS, 1), "unit": "us/step", "cores": threads, "kind": "port",
               "sample": f"layer 0 ({len(lens)} sequences) with the reference's fp32 per-sequence torch prefill "
                         f"(engine/talker.py:165-167), median of 3 = {us:.0f} us, x{LAYERS} layers"}
    rec = base_record("talker prefill attn µs/step (28 layers) at 32 sequences, 1×MI355X",
                      round(ms_per_step * 1e3, 2), "us/step", args, ms_per_step, False,
                      {"workload": "talker prompt prefill, 32 sequences, lengths U[150,400], causal, GQA 16/8, "
                                   "head_dim 128, bf16, K/V read from a 16-token paged pool, 28 layers per step",
                       "tokens": int(lens.sum()), "parallelism": "single GPU"})
    rec.update({"us_per_layer_call": round(call_us, 2), "tflops": round(tflops, 2), "hbm_gbps": round(gbps, 1),
                "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                             "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None,
                             "mfma_tflops": round(tflops, 2), "mfma_peak_tflops": 2500.0,
                             "flops_per_call": w0.flops(), "bytes_per_call": w0.algorithmic_bytes()},
                "cpu_baseline": cpu})
    if prompt_step is not None:
        rec["prompt_step"] = prompt_step
    return rec


def bench_prefill_append(args, dev, wls):
    """Extra information beside the prefill line: the talker's whole prompt step per layer as the engine runs it
    (two index_copy_ scatters of k and v into the pool, engine/talker.py:161-162, then the attention over the packed
    k/v, :169) against prefill_append, which writes the pool inside the attention launch.  The pages are the ones
    the workload's table gives each sequence, so the frame rewrites identical values and stays replayable."""
    import numpy as np
    import torch

    import q3attn

    steps = []
    for wl in wls:
        bt = wl.block_table.cpu().numpy().astype(np.int64)
        page = wl.k_cache.shape[1]
        slot = np.concatenate([bt[s_, np.arange(L) // page] * page + np.arange(L) % page
                               for s_, L in enumerate(wl.lens)])
        steps.append((wl, torch.from_numpy(slot).to(dev)))

    def packed():
        return [q3attn.flash_attn_varlen_func(wl.q, wl.k, wl.v, wl.cu_seqlens, wl.cu_seqlens, wl.max_len, wl.max_len,
                                              softmax_scale=wl.scale, causal=True) for wl, _ in steps]

    def scatter_then_prefill():
        out = []
        for wl, slot in steps:
            wl.k_cache.view(-1, wl.k.shape[1], wl.k.shape[2]).index_copy_(0, slot, wl.k)
            wl.v_cache.view(-1, wl.v.shape[1], wl.v.shape[2]).index_copy_(0, slot, wl.v)
            out.append(q3attn.flash_attn_varlen_func(wl.q, wl.k, wl.v, wl.cu_seqlens, wl.cu_seqlens, wl.max_len,
                                                     wl.max_len, softmax_scale=wl.scale, causal=True))
        return out

    def fused():
        return [q3attn.prefill_append(wl.q, wl.k, wl.v, wl.cu_seqlens, wl.cu_seqlens, wl.max_len, wl.k_cache,
                                      wl.v_cache, wl.block_table, wl.scale, True) for wl, _ in steps]

    # The prompt step with its q/k producers (engine/talker.py:157-169): rope(rms(...)) of q and k as the eager bf16
    # torch ops prefill_hidden runs, the scatters and the attention, against prefill_append_rope.  Synthetic qkv
    # projections and norm weights per layer; cos/sin gathered per token as engine/talker.py:154 does.
    from q3attn.workloads import rope_tables
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed + 78)
    wl0 = steps[0][0]
    T = int(wl0.lens.sum())
    pos = torch.cat([torch.arange(int(L), device=dev) for L in wl0.lens])
    cos, sin = rope_tables(int(wl0.lens.max()), dev)
    cos_t, sin_t = cos.to(torch.bfloat16)[pos][:, None, :], sin.to(torch.bfloat16)[pos][:, None, :]
    blocks = []
    for wl, slot in steps:
        qkv = torch.randn((T, 4096), generator=gen, device=dev).to(torch.bfloat16)
        qn = (1.0 + 0.1 * torch.randn(128, generator=gen, device=dev)).to(torch.bfloat16)
        kn = (1.0 + 0.1 * torch.randn(128, generator=gen, device=dev)).to(torch.bfloat16)
        blocks.append((wl, slot, qkv, qn, kn))

    def rms_t(x, w, eps=1e-6):
        xf = x.float()
        xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
        return w * xf.to(x.dtype)

    def rope_t(x, c, s_):
        return x * c + torch.cat((-x[..., 64:], x[..., :64]), dim=-1) * s_

    def engine_step():
        out = []
        for wl, slot, qkv, qn, kn in blocks:
            q = rope_t(rms_t(qkv[:, :2048].view(T, 16, 128), qn), cos_t, sin_t)
            k = rope_t(rms_t(qkv[:, 2048:3072].view(T, 8, 128), kn), cos_t, sin_t)
            v = qkv[:, 3072:].view(T, 8, 128)
            wl.k_cache.view(-1, 8, 128).index_copy_(0, slot, k)
            wl.v_cache.view(-1, 8, 128).index_copy_(0, slot, v)
            out.append(q3attn.flash_attn_varlen_func(q, k, v, wl.cu_seqlens, wl.cu_seqlens, wl.max_len, wl.max_len,
                                                     softmax_scale=wl.scale, causal=True))
        return out

    def fused_rope():
        return [q3attn.prefill_append_rope(qkv[:, :2048].view(T, 16, 128), qkv[:, 2048:3072].view(T, 8, 128),
                                           qkv[:, 3072:].view(T, 8, 128), qn, kn, cos_t, sin_t, wl.cu_seqlens,
                                           wl.max_len, wl.k_cache, wl.v_cache, wl.block_table, wl.scale)
                for wl, _, qkv, qn, kn in blocks]

    res = {}
    for name, fn in (("packed_prefill", packed), ("index_copy_then_prefill", scatter_then_prefill),
                     ("prefill_append", fused), ("torch_producers_index_copy_then_prefill", engine_step),
                     ("prefill_append_rope", fused_rope)):
        _, fr, _ = time_graph(dev, fn, args.steps, args.warmup, getattr(args, "min_warm_s", 0.0))
        res[name + "_us_per_layer_call"] = round(statistics.mean(fr) * 1e3 / LAYERS, 2)
    log(f"[bench] prompt step: prefill_append {res['prefill_append_us_per_layer_call']:.1f} us/layer call; "
        f"index_copy_ x2 + prefill {res['index_copy_then_prefill_us_per_layer_call']:.1f}; packed prefill alone "
        f"{res['packed_prefill_us_per_layer_call']:.1f}")
    log(f"[bench] prompt step with the q/k producers: prefill_append_rope "
        f"{res['prefill_append_rope_us_per_layer_call']:.1f} us/layer call; eager torch producers + index_copy_ x2 + "
        f"prefill {res['torch_producers_index_copy_then_prefill_us_per_layer_call']:.1f}")
    return res


def bench_admit(args, dev):
    """Fast-admission prefill (engine/arrivals.py:133-152): S = 8 sequences (the largest graphed bucket) of R = 42 new
    tokens over a 35-token shared prefix (n = 77 keys), bottom-right causal (engine/arrivals.py:148), 28 layers per
    step, each layer with its own q/k/v."""
    import torch

    import q3attn
    from q3attn import workloads as W

    S, R, n = 8, 42, 77
    wls = [W.make_admit(dev, S, R, n, seed=args.seed + l) for l in range(LAYERS)]
    w0 = wls[0]

    def call(wl):
        return q3attn.flash_attn_func(wl.q, wl.k, wl.v, softmax_scale=wl.scale, causal=True)

    ms_per_step, frame_ms, _ = time_graph(dev, lambda: [call(wl) for wl in wls], args.steps, args.warmup,
                                          getattr(args, "min_warm_s", 0.0))
    call_us = statistics.mean(frame_ms) * 1e3 / LAYERS
    tflops = w0.flops() / (call_us * 1e-6) / 1e12
    log(f"[bench] admission prefill S={S} R={R} n={n}: {call_us:.2f} us/call, {tflops:.1f} TFLOP/s")
    admission_step = None if args.no_append else bench_admit_append(args, dev, wls)
    cpu = None
    if not args.no_cpu_baseline:
        from oracle.torch_cpu import prefill_prefix_rows
        threads = cpu_threads()
        q, K, V = w0.q.float().cpu(), w0.k.float().cpu(), w0.v.float().cpu()
        times = []
        for rep in range(5):
            t0 = time.perf_counter()
            prefill_prefix_rows(q, K, V, w0.scale)
            times.append(time.perf_counter() - t0)
        us = statistics.median(times) * 1e6
        cpu = {"value": round(us * LAYERS, 1), "unit": "us/step", "cores": threads, "kind": "port",
               "sample": f"layer 0 with the reference's fp32 torch form (engine/arrivals.py:125-131), median of 5 = "
                         f"{us:.0f} us, x{LAYERS} layers"}
    rec = base_record(f"fast-admission prefill attn µs/step (28 layers) at S={S}, R={R}, n={n}, 1×MI355X",
                      round(ms_per_step * 1e3, 2), "us/step", args, ms_per_step, False,
                      {"workload": f"fast-admission prefill: {S} sequences of {R} new tokens over a {n - R}-token "
                                   f"shared prefix, bottom-right causal, GQA 16/8, head_dim 128, bf16, 28 layers",
                       "parallelism": "single GPU"})
    rec.update({"us_per_layer_call": round(call_us, 2), "tflops": round(tflops, 2),
                "roofline": {"bound": "latency (155 MFLOP and 1.4 MB per call)", "achieved": round(tflops, 2),
                             "peak": 2500.0, "unit": "TFLOP/s", "frac": round(tflops / 2500.0, 4), "traffic": None,
                             "flops_per_call": w0.flops()},
                "cpu_baseline": cpu})
    if admission_step is not None:
        rec["admission_step"] = admission_step
    return rec


def bench_admit_append(args, dev, wls):
    """Extra information beside the admission line: the admission layer step as the engine runs it (two index_copy_
    scatters of every K and V row into the seat's cache positions, engine/arrivals.py:144-145, then flash_attn_func
    on the dense K/V, :148) against prefill_dense_append, which writes the pool inside the attention launch.  Each
    layer has its own 256-page pool (16-token pages) and random table; every replay rewrites identical values."""
    import numpy as np
    import torch

    import q3attn
    from q3attn.workloads import rope_tables as W_rope_tables

    S, n = wls[0].k.shape[0], wls[0].k.shape[1]
    P, page, num_pages = -(-n // 16), 16, 256
    steps = []
    for l, wl in enumerate(wls):
        bt = np.random.default_rng(1000 + l).permutation(num_pages)[: S * P].reshape(S, P).astype(np.int32)
        flat = np.concatenate([bt[s_, np.arange(n) // page] * page + np.arange(n) % page for s_ in range(S)])
        kc = torch.zeros(num_pages, page, 8, 128, dtype=torch.bfloat16, device=dev)
        steps.append((wl, kc, torch.zeros_like(kc), torch.from_numpy(bt).to(dev), torch.from_numpy(flat).to(dev)))

    def dense():
        return [q3attn.flash_attn_func(wl.q, wl.k, wl.v, softmax_scale=wl.scale, causal=True)
                for wl, _, _, _, _ in steps]

    def scatter_then_prefill():
        out = []
        for wl, kc, vc, _, flat in steps:
            kc.view(-1, 8, 128).index_copy_(0, flat, wl.k.reshape(-1, 8, 128))
            vc.view(-1, 8, 128).index_copy_(0, flat, wl.v.reshape(-1, 8, 128))
            out.append(q3attn.flash_attn_func(wl.q, wl.k, wl.v, softmax_scale=wl.scale, causal=True))
        return out

    def fused():
        return [q3attn.prefill_dense_append(wl.q, wl.k, wl.v, kc, vc, bt, wl.scale, True, 0)
                for wl, kc, vc, bt, _ in steps]

    # The whole attention block of the admission layer (engine/arrivals.py:112-118, 144-148): q/k RMSNorm + RoPE as the
    # eager bf16 torch ops the uncompiled layer runs, torch.cat of the voice prefix K/V (gathered per admitted slot),
    # the two scatters and the attention, against prefill_dense_append_rope.  Synthetic qkv projections and weights.
    P = n - wls[0].q.shape[1]
    R = wls[0].q.shape[1]
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed + 77)
    cos_t, sin_t = W_rope_tables(n, dev)
    cos_r = cos_t[P:].to(torch.bfloat16)[None, :, None]
    sin_r = sin_t[P:].to(torch.bfloat16)[None, :, None]
    voices = 4
    blocks = []
    for l, (wl, kc, vc, bt, flat) in enumerate(steps):
        qkv = torch.randn((S, R, 4096), generator=gen, device=dev).to(torch.bfloat16)
        pk = wl.k[:voices, :P].contiguous() if S >= voices else wl.k[:, :P].contiguous()
        pv = wl.v[:voices, :P].contiguous() if S >= voices else wl.v[:, :P].contiguous()
        qn = (1.0 + 0.1 * torch.randn(128, generator=gen, device=dev)).to(torch.bfloat16)
        kn = (1.0 + 0.1 * torch.randn(128, generator=gen, device=dev)).to(torch.bfloat16)
        slot = torch.arange(S, device=dev, dtype=torch.int64) % pk.shape[0]
        blocks.append((qkv, pk, pv, qn, kn, slot, kc, vc, bt, flat))

    def rms_t(x, w, eps=1e-6):
        xf = x.float()
        xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
        return w * xf.to(x.dtype)

    def rope_t(x, c, s_):
        return x * c + torch.cat((-x[..., 64:], x[..., :64]), dim=-1) * s_

    def engine_block():
        out = []
        for qkv, pk, pv, qn, kn, slot, kc, vc, bt, flat in blocks:
            q = rope_t(rms_t(qkv[..., :2048].view(S, R, 16, 128), qn), cos_r, sin_r)
            kk = rope_t(rms_t(qkv[..., 2048:3072].view(S, R, 8, 128), kn), cos_r, sin_r)
            K = torch.cat((pk[slot], kk), 1)
            V = torch.cat((pv[slot], qkv[..., 3072:].view(S, R, 8, 128)), 1)
            kc.view(-1, 8, 128).index_copy_(0, flat, K.reshape(-1, 8, 128))
            vc.view(-1, 8, 128).index_copy_(0, flat, V.reshape(-1, 8, 128))
            out.append(q3attn.flash_attn_func(q, K, V, softmax_scale=wls[0].scale, causal=True))
        return out

    def fused_block():
        return [q3attn.prefill_dense_append_rope(qkv[..., :2048].view(S, R, 16, 128),
                                                 qkv[..., 2048:3072].view(S, R, 8, 128),
                                                 qkv[..., 3072:].view(S, R, 8, 128), pk, pv, qn, kn,
                                                 cos_r, sin_r, kc, vc, bt, wls[0].scale, slot)
                for qkv, pk, pv, qn, kn, slot, kc, vc, bt, _ in blocks]

    res = {}
    for name, fn in (("flash_attn_func", dense), ("index_copy_then_prefill", scatter_then_prefill),
                     ("prefill_dense_append", fused), ("torch_producers_cat_index_copy_then_prefill", engine_block),
                     ("prefill_dense_append_rope", fused_block)):
        _, fr, _ = time_graph(dev, fn, args.steps, args.warmup, getattr(args, "min_warm_s", 0.0))
        res[name + "_us_per_layer_call"] = round(statistics.mean(fr) * 1e3 / LAYERS, 2)
    log(f"[bench] admission step: prefill_dense_append {res['prefill_dense_append_us_per_layer_call']:.2f} us/layer "
        f"call; index_copy_ x2 + prefill {res['index_copy_then_prefill_us_per_layer_call']:.2f}; prefill alone "
        f"{res['flash_attn_func_us_per_layer_call']:.2f}")
    log(f"[bench] admission block with the q/k producers: prefill_dense_append_rope "
        f"{res['prefill_dense_append_rope_us_per_layer_call']:.2f} us/layer call; eager torch producers + cat + "
        f"index_copy_ x2 + prefill {res['torch_producers_cat_index_copy_then_prefill_us_per_layer_call']:.2f}")
    return res


def bench_probe(args, dev):
    """Measured HBM ceilings on this GPU (libq3probe.so, beside the attention library): the 576-row decode's exact K/V
    access pattern read with no arithmetic, records or combine (q3p_tile_read over the same 28 per-layer tables and
    contexts, one launch per layer in a captured graph, the resident grid over equal tile ranges), the decode itself on
    the same frame, a plain streaming read of 4 GiB with and without the non-temporal hint (q3p_stream_read), and a
    2 GiB device copy (read + write).  The decode's K/V rate over the probe's is the fraction of the practical ceiling
    of its access pattern; the copy rate bounds kernels that read and write in equal measure."""
    import ctypes

    import numpy as np
    import torch

    import q3attn
    from q3attn import workloads as W

    plib = ctypes.CDLL(os.path.join(ROOT, "qwen3-tts-engine_amd", "q3attn", "libq3probe.so"))
    vp, i64, ci, u32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_uint32
    plib.q3p_tile_read.argtypes = [vp, vp, i64, i64, i64, ci, ci, ci, vp, ci, ci, u32, vp, vp, vp]
    plib.q3p_clear_flags.argtypes = [vp, ci, vp]
    plib.q3p_stream_read.argtypes = [vp, ctypes.c_size_t, ci, ci, u32, vp, vp]
    plib.q3p_resident_grid.argtypes = [ci, ci]
    magic = 0x9E3779B9
    wl = W.make_decode("decode576", dev, layers=LAYERS, seed=args.seed)
    kc, vc = wl.k_cache, wl.v_cache
    kv_bytes = 2 * 8 * 128 * 2 * int(wl.ctx.sum())
    tiles = []
    for L in wl.layers:
        bt = L.block_table.cpu().numpy()
        rows = [np.stack([bt[b, : (c + 15) // 16], np.minimum(16, c - 16 * np.arange((c + 15) // 16))], 1)
                for b, c in enumerate(wl.ctx) if c > 0]
        tiles.append(torch.from_numpy(np.concatenate(rows).astype(np.int32)).to(dev))
    nt = int(tiles[0].shape[0])
    grid = plib.q3p_resident_grid(1, 8)
    sink = torch.zeros(1 << 16, dtype=torch.int32, device=dev)   # one word per workgroup of either probe
    stream = lambda: torch.cuda.current_stream(dev).cuda_stream

    flags = torch.zeros(LAYERS * grid, dtype=torch.int32, device=dev)

    def probe_frame(by_xcd=False):
        if by_xcd and plib.q3p_clear_flags(flags.data_ptr(), flags.numel(), stream()):
            raise RuntimeError("q3p_clear_flags failed")
        for i, t in enumerate(tiles):
            fl = flags[i * grid:].data_ptr() if by_xcd else None
            rc = plib.q3p_tile_read(kc.data_ptr(), vc.data_ptr(), kc.stride(0), kc.stride(1), kc.stride(2),
                                    kc.shape[0], 16, 8, t.data_ptr(), nt, grid, magic, sink.data_ptr(), fl, stream())
            if rc:
                raise RuntimeError(f"q3p_tile_read failed ({rc})")
        return [sink]

    def decode_frame():
        return [q3attn.paged_decode(L.q, kc, vc, wl.cache_seqlens, L.block_table, wl.scale, 0) for L in wl.layers]

    bts = torch.stack([L.block_table for L in wl.layers])

    def planned_decode_frame():
        plans = q3attn.decode_plan(wl.cache_seqlens, bts, wl.page_size)
        return [q3attn.paged_decode(L.q, kc, vc, wl.cache_seqlens, bts[i], wl.scale, plan=plans[i])
                for i, L in enumerate(wl.layers)]

    res = {}
    for name, fn in (("tile_read", probe_frame), ("tile_read_by_xcd", lambda: probe_frame(True)),
                     ("decode", decode_frame), ("decode_planned", planned_decode_frame),
                     ("tile_read_again", probe_frame), ("tile_read_by_xcd_again", lambda: probe_frame(True))):
        _, frame_ms, _ = time_graph(dev, fn, args.steps, args.warmup, 1.0)
        us = statistics.median(frame_ms) * 1e3 / LAYERS
        res[name] = {"us_per_call": round(us, 2), "kv_gbps": round(kv_bytes / (us * 1e-6) / 1e9, 1)}
        log(f"[probe] {name}: {us:.2f} us per layer call, K/V {kv_bytes / (us * 1e-6) / 1e9:.0f} GB/s")
    del wl, tiles
    torch.cuda.empty_cache()
    ceiling = min(res["tile_read"]["us_per_call"], res["tile_read_again"]["us_per_call"])
    res["decode_over_probe"] = round(ceiling / res["decode"]["us_per_call"], 4)
    ceiling_x = min(res["tile_read_by_xcd"]["us_per_call"], res["tile_read_by_xcd_again"]["us_per_call"])
    res["planned_decode_over_probe_by_xcd"] = round(ceiling_x / res["decode_planned"]["us_per_call"], 4)

    sgrid = plib.q3p_resident_grid(0, 0) * 2
    n = 4 << 30
    buf = torch.empty(n, dtype=torch.uint8, device=dev)
    buf.fill_(7)
    for nt_flag in (1, 0):
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        for _ in range(2):
            plib.q3p_stream_read(buf.data_ptr(), n // 16, sgrid, nt_flag, magic, sink.data_ptr(), stream())
        ev[0].record()
        reps = 5
        for _ in range(reps):
            plib.q3p_stream_read(buf.data_ptr(), n // 16, sgrid, nt_flag, magic, sink.data_ptr(), stream())
        ev[1].record()
        torch.cuda.synchronize()
        gbps = n * reps / (ev[0].elapsed_time(ev[1]) * 1e-3) / 1e9
        res["stream_read_nt_gbps" if nt_flag else "stream_read_gbps"] = round(gbps, 1)
        log(f"[probe] streaming read of 4 GiB ({'non-temporal' if nt_flag else 'plain'}): {gbps:.0f} GB/s")
    src, dst = buf[: n // 2], buf[n // 2:]
    for _ in range(2):
        dst.copy_(src)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    ev[0].record()
    for _ in range(5):
        dst.copy_(src)
    ev[1].record()
    torch.cuda.synchronize()
    gbps = 2 * (n // 2) * 5 / (ev[0].elapsed_time(ev[1]) * 1e-3) / 1e9
    res["copy_read_plus_write_gbps"] = round(gbps, 1)
    log(f"[probe] 2 GiB device copy: {gbps:.0f} GB/s read + write")
    del buf
    torch.cuda.empty_cache()
    rec = base_record("HBM read ceiling of the 576-row decode's access pattern, 1×MI355X",
                      res["tile_read"]["kv_gbps"], "GB/s", args, ceiling * LAYERS / 1e3, True, {
                          "workload": "the 576-row decode's K/V tiles (518 live rows, ctx log-uniform [64, 1800], "
                                      "16-token pages, 28 per-layer random tables over a 131072-page pool) read with "
                                      "the decode's loads and no arithmetic; 4 GiB streaming reads; a 2 GiB copy",
                          "tiles_per_call": nt, "grid": grid, "parallelism": "single GPU"})
    rec.update(res)
    rec["roofline"] = {"bound": "hbm", "achieved": res["tile_read"]["kv_gbps"], "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                       "frac": round(res["tile_read"]["kv_gbps"] / HBM_PEAK_GBPS, 4), "traffic": None}
    return rec


def other_workloads(args, dev):
    """Short runs of the other configurations beside the headline (20 graph replays each; `--workload NAME` gives the
    full line of each): the 256-row and 1-row x 64-token decodes (with their CPU baselines unless --no-cpu-baseline),
    the 512-row code predictor, the 32-sequence prefill (with the prompt-step comparison) and the fast-admission
    prefill.  A failure is recorded in place
    of the numbers and does not affect the headline."""
    import copy

    import torch

    lite = copy.copy(args)
    lite.steps, lite.warmup, lite.no_cpu_baseline, lite.no_append = 20, 3, True, True
    lite.no_compile = True                # a torch.compile of the CP producers does not fit these short runs
    lite.min_warm_s = 1.0                 # the GPU sat idle during the CPU baseline before: let clocks ramp
    # Every configuration's CPU baseline (the reference's torch CPU form of the same call, timed on the host's
    # threads) runs unless --no-cpu-baseline: each is a bounded sample of well under a second here.
    lite.no_cpu_baseline = args.no_cpu_baseline
    pre = copy.copy(lite)
    pre.no_append = False                 # the prompt/admission-step comparisons (fused pool writes) are part of these
    out = {}
    for name, fn in (("decode256", lambda: bench_decode(lite, dev, "decode256", cpu_budget_s=6.0)),
                     ("decode1x64", lambda: bench_decode(lite, dev, "decode1x64", cpu_budget_s=2.0)),
                     ("decode_small", lambda: bench_decode_small_lite(lite, dev)),
                     ("cp512", lambda: bench_cp(lite, dev)),
                     ("prefill32", lambda: bench_prefill(pre, dev)), ("admission_prefill", lambda: bench_admit(pre, dev))):
        try:
            r = fn()
            keep = {k: r[k] for k in ("us_per_layer_call", "us_per_call", "hbm_gbps", "pct_hbm_peak", "tflops",
                                      "three_launch_us_per_step", "cold_us_per_call", "launch_floor_us_per_call",
                                      "prompt_step", "admission_step", "norm_rope_form",
                                      "per_shape_us_per_call") if k in r}
            keep["us_per_step"] = r["value"]
            if "roofline" in r:
                keep["roofline_frac"] = r["roofline"]["frac"]
                keep["roofline_unit"] = r["roofline"]["unit"]
            if r.get("cpu_baseline"):
                keep["cpu_baseline"] = {k: r["cpu_baseline"][k] for k in ("value", "unit", "us_per_layer_call", "gbps",
                                                                        "cores", "kind", "sample")
                                        if k in r["cpu_baseline"]}
            out[name] = keep
        except Exception as e:  # noqa: BLE001 - reported, never fatal for the headline
            out[name] = {"error": f"{type(e).__name__}: {e}"}
        torch.cuda.empty_cache()
    return out


def rocprof_summary(src: str, dst: str) -> None:
    """Condense rocprofv3 CSV output (one directory per run under src) into small files under dst: each run's
    kernel_stats.csv as it is, and for counter runs the dispatch count, median and mean of every counter per kernel
    (this library's kernels, the probe's and the device copy used for calibration).  Raw per-dispatch counter files of
    a full bench run are tens of MB; these summaries are what profiles/*.md cite."""
    import csv
    import glob

    os.makedirs(dst, exist_ok=True)
    for d in sorted(glob.glob(os.path.join(src, "*"))):
        name = os.path.basename(d)
        for f in glob.glob(os.path.join(d, "*kernel_stats.csv")):
            with open(f) as i, open(os.path.join(dst, f"{name}_kernel_stats.csv"), "w") as o:
                o.write(i.read())
        for f in glob.glob(os.path.join(d, "*counter_collection.csv")):
            vals = {}
            with open(f) as i:
                for r in csv.DictReader(i):
                    k = r["Kernel_Name"]
                    if "q3a" in k or "q3p" in k or "copyBuffer" in k:
                        vals.setdefault((k, r["Counter_Name"]), []).append(float(r["Counter_Value"]))
            with open(os.path.join(dst, f"{name}_pmc.csv"), "w", newline="") as o:
                w = csv.writer(o)
                w.writerow(["kernel", "counter", "dispatches", "median", "mean"])
                for (k, c), v in sorted(vals.items()):
                    w.writerow([k, c, len(v), statistics.median(v), statistics.mean(v)])
    print(json.dumps({"rocprof_summary": sorted(os.listdir(dst))}), flush=True)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="decode576",
                    choices=["decode576", "decode256", "decode1x64", "decode-small", "decode-scaling",
                             "decode-plan-sweep", "cp512",
                             "prefill32", "admit", "probe"],
                    help="c5 (default, the headline metric), c3 decode, c1 decode, decode at small batches (each "
                         "decode kernel by path code and the library's choice), c5 with its contexts scaled by 1/2, "
                         "1, 2 (marginal read rate and fixed cost per call), c2 code predictor, c4 prefill, admit "
                         "fast-admission prefill, probe (HBM read ceilings of the decode's access pattern)")
    ap.add_argument("--split", type=int, default=0,
                    help="decode split_tokens: 0 = the library's choice (stream-K at 576 rows), -1 row-parallel, "
                         "-2 chunked, -3 stream-K, > 0 fixed split of that many tokens")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-plan", action="store_true",
                    help="decode frames without the per-frame plan (q3attn.decode_plan): every call scans the lengths "
                         "and looks its pages up itself")
    ap.add_argument("--no-append", action="store_true",
                    help="skip the KV-append comparisons (decode: fused append; prefill: the prompt step)")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-extra", action="store_true",
                    help="576-row decode only: skip the short runs of the other workloads and their CPU baselines "
                         "(other_workloads field)")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="only run a plain device copy of this many MiB (calibrates rocprof byte counters)")
    ap.add_argument("--rocprof-summary", nargs=2, metavar=("SRC", "DST"),
                    help="no GPU work: condense the rocprofv3 CSV runs under SRC into per-kernel summaries under DST")
    args = ap.parse_args()
    if args.rocprof_summary:
        rocprof_summary(*args.rocprof_summary)
        return 0

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the decode attention shards by seat with no exchange). Run with --gpus 1.", file=sys.stderr)
        return 2

    import torch

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.copy_probe_mib:
        n = args.copy_probe_mib << 20
        src = torch.randint(0, 255, (n,), dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": n, "launches": 3}), flush=True)
        return 0
    if args.workload in ("decode576", "decode256", "decode1x64"):
        rec = bench_decode(args, dev, args.workload)
        if args.workload == "decode576" and not args.no_extra:
            rec["other_workloads"] = other_workloads(args, dev)
            if rec.get("cpu_baseline"):
                per = {"decode576": {k: rec["cpu_baseline"][k] for k in ("us_per_layer_call", "gbps", "cores")}}
                for k in ("decode256", "decode1x64"):
                    if "cpu_baseline" in rec["other_workloads"].get(k, {}):
                        per[k] = rec["other_workloads"][k]["cpu_baseline"]
                rec["cpu_baseline"]["per_config"] = per
    elif args.workload == "decode-small":
        rec = bench_decode_small(args, dev)
    elif args.workload == "decode-scaling":
        rec = bench_decode_scaling(args, dev)
    elif args.workload == "decode-plan-sweep":
        rec = bench_decode_plan_sweep(args, dev)
    elif args.workload == "probe":
        rec = bench_probe(args, dev)
    elif args.workload == "cp512":
        rec = bench_cp(args, dev)
    elif args.workload == "admit":
        rec = bench_admit(args, dev)
    else:
        rec = bench_prefill(args, dev)
    print(json.dumps(rec), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
