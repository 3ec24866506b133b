"""Benchmark: talker paged decode attention at 576 rows on one MI355X.

One step = one frame of the talker = 28 decode-attention layer calls (engine/talker.py:66-77) over
the 576-row workload: 518 live rows with ctx = round(exp(U[ln 64, ln 1800])), 58 padded rows with
ctx = 0, GQA 16/8, head_dim 128, bf16, 16-token pages, every layer with its own seeded random
page table over one 131,072-page pool (8.59 GB of K+V).  Inputs are resident in HBM before the
timed region.  Prints one JSON line.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import json
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


def cpu_model() -> str:
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for ln in out.splitlines():
            if ln.startswith("Model name:"):
                return ln.split(":", 1)[1].strip()
    except Exception:
        pass
    return "unknown"


def cpu_baseline(wl, reps_min: int = 3, budget_s: float = 12.0):
    """The reference's per-row fp32 torch attention (engine/talker.py:82-88 with the page gather),
    on the host cores, over layer 0 of the same workload (all 576 rows).  Reported per frame (x28)."""
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
    threads = torch.get_num_threads()
    paged_decode_rows(q, k, v, sl, tb, wl.scale)                # warm-up
    times = []
    t_start = time.perf_counter()
    while len(times) < reps_min or (time.perf_counter() - t_start < budget_s and len(times) < 50):
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
                   f"{threads} threads on {cpu_model()}"),
        "us_per_layer_call": round(per_call_us, 1),
        "gbps": round(wl.algorithmic_bytes() / (per_call_us * 1e-6) / 1e9, 2),
    }


def measured_traffic():
    """HBM bytes per decode-kernel launch from the committed rocprofv3 --pmc summary (FETCH_SIZE and
    WRITE_SIZE scaled by a plain-copy calibration), or None when the summary is absent."""
    path = os.path.join(ROOT, "profiles", "paged_decode_c5.md")
    try:
        for ln in open(path):
            if ln.startswith("traffic_bytes_per_launch"):
                return int(ln.split("=")[1])
    except OSError:
        pass
    return None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--split", type=int, default=0, help="split_tokens (0 = library default)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="only run a plain device copy of this many MiB (calibrates rocprof byte counters)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the decode attention shards by seat with no exchange; see the design notes). "
              "Run with --gpus 1.", file=sys.stderr)
        return 2

    import torch

    import q3attn
    from q3attn import workloads as W

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
    t0 = time.time()
    wl = W.make_decode("c5", dev, layers=LAYERS, seed=args.seed)
    torch.cuda.synchronize()
    log(f"[bench] workload c5 built in {time.time() - t0:.1f} s: rows={wl.batch} live={(wl.ctx > 0).sum()} "
        f"sum_ctx={int(wl.ctx.sum())} pool={tuple(wl.k_cache.shape)}")
    nbytes = wl.algorithmic_bytes()

    def layer_call(L):
        return q3attn.paged_decode(L.q, wl.k_cache, wl.v_cache, wl.cache_seqlens, L.block_table,
                                   wl.scale, args.split)

    def frame():
        return [layer_call(L) for L in wl.layers]

    # The engine replays its 28-layer frame as one captured graph (engine/talker.py:115-137);
    # the step here is the same: one replay of a graph holding the 28 decode-attention calls.
    stream = torch.cuda.Stream(dev)
    stream.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(stream):
        eager = [o.clone() for o in frame()]
    torch.cuda.current_stream(dev).wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        static_out = frame()
    graph.replay()
    torch.cuda.synchronize()
    if not all(torch.equal(a, b) for a, b in zip(static_out, eager)):
        raise RuntimeError("graph replay differs from the eager frame")

    cur = torch.cuda.current_stream(dev)
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()

    K = args.steps
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(K)]
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    for i in range(K):
        ev[i][0].record(cur)
        graph.replay()
        ev[i][1].record(cur)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_start
    frame_ms = [a.elapsed_time(b) for a, b in ev]
    avg_call_us = statistics.mean(frame_ms) * 1e3 / LAYERS
    ms_per_step = wall * 1e3 / K
    us_per_step = ms_per_step * 1e3
    achieved = nbytes / (avg_call_us * 1e-6) / 1e9
    log(f"[bench] {K} graph replays of {LAYERS} calls: wall {ms_per_step:.3f} ms/step; events "
        f"{statistics.mean(frame_ms):.3f} ms/frame (min {min(frame_ms):.3f}) = {avg_call_us:.1f} us/call; "
        f"{achieved:.0f} GB/s = {achieved / HBM_PEAK_GBPS:.1%} of peak")

    # Eager calls with an event pair around each (host launch gaps excluded): extra information.
    eg = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(LAYERS * 2)]
    i = 0
    for _ in range(2):
        for L in wl.layers:
            eg[i][0].record(cur)
            layer_call(L)
            eg[i][1].record(cur)
            i += 1
    torch.cuda.synchronize()
    eager_call_us = statistics.mean(a.elapsed_time(b) for a, b in eg) * 1e3

    cpu = None
    if not args.no_cpu_baseline:
        t0 = time.time()
        cpu = cpu_baseline(wl)
        log(f"[bench] cpu baseline {cpu['us_per_layer_call']:.0f} us/call in {time.time() - t0:.1f} s")

    split = args.split or "stream-K"
    rec = {
        "metric": METRIC,
        "value": round(us_per_step, 2),
        "unit": "us/step",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": ("talker paged decode attention, 576 rows (518 live, ctx log-uniform [64,1800]; "
                         "58 padded ctx=0), GQA 16/8, head_dim 128, bf16 K/V, fp32 softmax/accumulate, "
                         "16-token pages, 131072-page pool, 28 layer calls per step with per-layer random tables"),
            "rows": wl.batch,
            "sum_ctx": int(wl.ctx.sum()),
            "layers_per_step": LAYERS,
            "split_tokens": split,
            "parallelism": "single GPU",
        },
        "us_per_layer_call": round(avg_call_us, 2),
        "us_per_layer_call_eager": round(eager_call_us, 2),
        "hbm_gbps": round(achieved, 1),
        "pct_hbm_peak": round(100 * achieved / HBM_PEAK_GBPS, 2),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": measured_traffic(),
            "kernel": "paged decode call (stream-K decode kernel + combine kernel), per call inside the graph",
            "bytes_per_call": nbytes,
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(rec), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
