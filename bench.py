#!/usr/bin/env python3
"""Benchmark of libllmk's non-GEMM layer kernels on one MI355X.

Headline (the JSON line's `value`): the fused residual add + RMSNorm over [8192, 2048] fp16
-- whole-job throughput in GB/s of algorithmic bytes (inputs read once,
outputs written once), inputs resident in HBM before the timed region. One step = one launch
over the full batch. The other BASELINE configurations (RMSNorm [16,2048], RoPE, SwiGLU,
embedding gather, the 16-layer decode-step pass captured in a HIP graph) and a copy probe are
measured the same way and reported under "kernels".

Caches: MI355X has a 256 MB Infinity Cache (MALL) in front of HBM and 4 MB of L2 per XCD. Each
kernel cycles through enough independent input sets that the data of a launch was last
touched more than 1 GB of traffic earlier, so it cannot be served from the MALL.

Timing: `ms_per_step` = host wall time of K back-to-back steps, synchronised on both sides, / K;
`value` = algorithmic bytes per step / ms_per_step. Then K more launches are enqueued behind a
short spin kernel with a HIP event right before the first and right after the last, recorded on
the stream they are launched on (torch's current stream); the mean launch duration is the event
interval / K, and `roofline.achieved` = algorithmic bytes / that mean.

CPU baseline: the scalar C oracle of the same op (oracle/, test infrastructure) on the host's
cores, over a bounded sample of the same workload.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--kernels all|headline] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
METRIC = ("achieved HBM GB/s (% of ~8 TB/s) per fused kernel; "
          "µs per 16-layer non-GEMM pass")
PEAK_GBS = 8000.0
WARM_S = 0.25
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "llmk_kernels_bench_configs.txt")


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--kernels", choices=["all", "headline", "step", "step8", "sched"],
                    default="all",
                    help="all: every configuration; headline: config 2 only; step / step8: "
                         "config 2 and the engine's decode step of 256 / 8 sequences; sched: "
                         "config 2 and the reference's scheduler workload")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--summarize-profiles", nargs=3, metavar=("TRACE_DIR", "FETCH_DIR", "WRITE_DIR"),
                    help="summarise rocprofv3 csv output of this bench instead of running it")
    ap.add_argument("--summarize-sched", metavar="TRACE_DIR",
                    help="summarize a rocprofv3 kernel trace of --kernels sched by row count")
    ap.add_argument("--summarize-step", nargs="+", metavar="TRACE_DIR [ROWS]",
                    help="per-kernel time of one engine decode step of ROWS (256) sequences from "
                         "a rocprofv3 kernel trace of `bench.py --kernels step` (or step8, 8)")
    return ap.parse_args()


def read_traffic() -> dict:
    """Counter-based HBM bytes per launch, from the committed rocprofv3 summary (one line per
    kernel: `<name> traffic_bytes=<int> ...`)."""
    out = {}
    if os.path.exists(TRAFFIC_FILE):
        for line in open(TRAFFIC_FILE):
            parts = line.split()
            if len(parts) >= 2 and not line.startswith("#"):
                kv = dict(p.split("=", 1) for p in parts[1:] if "=" in p)
                if "traffic_bytes" in kv:
                    out[parts[0]] = int(float(kv["traffic_bytes"]))
    return out



# (label, kernel-name substring, grid size in work-items, algorithmic bytes) of each measured
# launch shape; grid sizes follow from the launchers' grid choices at the benchmark shapes.
# Decode attention over 256 sequences with lengths uniform in [1, 2048] (seed 0x5EED0006):
# the bytes of bytes_attention(attention_lens()) in cuda-llm-engine_amd/workloads.py.
ATTN_BYTES_256 = 546_019_628
ATTN_BYTES_16x2048 = 67_248_192  # 16 sequences x 2048 positions

PROFILE_SHAPES = [
    ("add_rmsnorm_8192x2048", "k_rmsnorm_waveILi4ELb1ELb1E", 8192 * 64, 134221824),
    ("rmsnorm_16x2048", "k_rmsnorm_waveILi4ELb0ELb1E", 16 * 64, 135168),
    # 8 tokens per block, 10 vector tasks per thread (40 heads x 8 vectors x 8 tokens / 256)
    ("rope_8192", "k_rope_vecILi4ELi10ELb0E", 1024 * 256, 83918976),
    ("swiglu_8192x8192", "k_swiglu_vecILi2E", 16384 * 256, 402653184),
    ("embedding_8192", "k_embedding_rowsILi8E", 256 * 256, 67141632),
    ("copy_1GiB", "k_copy", 8192 * 256, 2 * (1 << 30)),
    # 512 blocks: two resident blocks of 256 threads on each of the 256 CUs (191 VGPRs).
    ("attention_decode_256", "k_attn_balancedILi8E", 512 * 256, ATTN_BYTES_256,
     ("k_attn_merge", 256 * 256)),
    # 16 sequences take the sequence-split grid (32 splits of 4 pages, 16 blocks per split).
    ("attention_decode_16x2048", "k_attn_splitILi8ELi0E", 32 * 256 * 16, ATTN_BYTES_16x2048,
     ("k_attn_merge_many", 8 * 256 * 16)),
    ("argmax_256x128256", "k_argmax_vec", 256 * 1024, 256 * 128256 * 2 + 256 * 4),
    ("decode:embedding_256", "k_embeddingILi0E", 256 * 64, 2098176),
    ("decode:add_rmsnorm_256x2048", "k_rmsnorm_waveILi4ELb1ELb1E", 256 * 64, 4198400),
    ("decode:rope_kv_scatter_256", "k_rope_vecILi4ELi2ELb1E", 256 * 256, 3147904),
    ("decode:swiglu_256x8192", "k_swiglu_vecILi2E", 512 * 256, 12582912),
]


def summarize_profiles(trace_dir, fetch_dir, write_dir):
    """Per launch shape: mean kernel duration from the kernel trace, FETCH_SIZE and WRITE_SIZE per
    dispatch, and HBM traffic per launch with each counter scaled by what it reads for the
    1 GiB copy probe (1 GiB read, 1 GiB written)."""
    import csv
    import glob

    def rows(d, suffix):
        out = []
        for f in glob.glob(os.path.join(d, "**", f"*{suffix}"), recursive=True):
            out += list(csv.DictReader(open(f)))
        return out

    def grid(r):
        if "Grid_Size_X" in r:
            return int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
        return int(r["Grid_Size"])

    def matches(table):
        """(label, row) for every row of a launch shape; a shape with a 5th field also needs
        the next dispatch to be that (kernel, grid) -- the attention kernel is told apart by
        the merge launch that follows it."""
        by_id = {int(r["Dispatch_Id"]): r for r in table}
        for r in table:
            for shape in PROFILE_SHAPES:
                label, name, g = shape[:3]
                if name not in r["Kernel_Name"] or grid(r) != g:
                    continue
                if len(shape) > 4:
                    nxt = by_id.get(int(r["Dispatch_Id"]) + 1)
                    if nxt is None or shape[4][0] not in nxt["Kernel_Name"] \
                            or grid(nxt) != shape[4][1]:
                        continue
                yield label, r

    dur, cnt = {}, {}
    for label, r in matches(rows(trace_dir, "kernel_trace.csv")):
        dur.setdefault(label, []).append(
            (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-3)
    for d, cname in ((fetch_dir, "FETCH_SIZE"), (write_dir, "WRITE_SIZE")):
        table = [r for r in rows(d, "counter_collection.csv") if r["Counter_Name"] == cname]
        for label, r in matches(table):
            cnt.setdefault((label, cname), []).append(float(r["Counter_Value"]))
    avg = {k: sum(v) / len(v) for k, v in cnt.items() if v}
    print("# rocprofv3 summaries of bench.py on one MI355X (gfx950), made by:")
    print(f"#   rocprofv3 --kernel-trace --stats -f csv -d {trace_dir} -o bench -- "
          "python3 bench.py --no-cpu")
    print(f"#   rocprofv3 --pmc FETCH_SIZE -f csv -d {fetch_dir} -o fetch -- "
          "python3 bench.py --no-cpu --steps 20 --warmup 2")
    print(f"#   rocprofv3 --pmc WRITE_SIZE -f csv -d {write_dir} -o write -- "
          "python3 bench.py --no-cpu --steps 20 --warmup 2")
    print(f"#   python3 bench.py --summarize-profiles {trace_dir} {fetch_dir} {write_dir}")
    print("#")
    print("# rocprofv3 --stats, libllmk kernels (all launch shapes of the run together):")
    print("#   calls  avg_us  min_us  max_us  kernel")
    for r in rows(trace_dir, "kernel_stats.csv"):
        if "llmk" in r["Name"]:
            print(f"#   {int(r['Calls']):6d} {float(r['AverageNs']) / 1e3:8.3f} "
                  f"{float(r['MinNs']) / 1e3:8.3f} {float(r['MaxNs']) / 1e3:8.3f}  {r['Name'][:90]}")
    print("#")
    copy_b = 1 << 30
    sf = copy_b / (avg[("copy_1GiB", "FETCH_SIZE")] * 1024)
    sw = copy_b / (avg[("copy_1GiB", "WRITE_SIZE")] * 1024)
    print(f"# Per launch shape. us_mean: mean kernel duration in the kernel trace. fetch_kib and")
    print(f"# write_kib: FETCH_SIZE and WRITE_SIZE per dispatch. traffic_bytes = fetch_kib*1024*"
          f"{sf:.4f} + write_kib*1024*{sw:.4f}, the factors being 1 GiB over what each counter")
    print("# reads for the 1 GiB copy probe (1 GiB read and 1 GiB written per launch).")
    missing = []
    for label, _, _, alg, *_ in PROFILE_SHAPES:
        d = dur.get(label, [])
        f, w = avg.get((label, "FETCH_SIZE")), avg.get((label, "WRITE_SIZE"))
        us = f"{sum(d) / len(d):.3f}" if d else "-"
        if f is None or w is None or not d:
            print(f"{label} us_mean={us} calls={len(d)} MISSING (kernel name or grid not found)")
            missing.append(label)
            continue
        traffic = f * 1024 * sf + w * 1024 * sw
        print(f"{label} us_mean={us} calls={len(d)} fetch_kib={f:.1f} write_kib={w:.1f} "
              f"traffic_bytes={traffic:.0f} algorithmic_bytes={alg} ratio={traffic / alg:.4f}")
    return 1 if missing else 0


def summarize_step(trace_dir, n_rows=256):
    """Kernels of the engine's decode step (the dispatches between the first and the last
    embedding gather of n_rows rows, i.e. the graph replays), grouped by kernel name and grid
    size: launches per step, mean duration, and time per step."""
    import csv
    import glob
    rows = []
    for f in glob.glob(os.path.join(trace_dir, "**", "*kernel_trace.csv"), recursive=True):
        rows += list(csv.DictReader(open(f)))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))

    def grid(r):
        return int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])

    starts = [i for i, r in enumerate(rows) if "k_embedding" in r["Kernel_Name"]
              and grid(r) == n_rows * 64]
    if len(starts) < 3:
        print("no decode steps found")
        return
    # whole steps, skipping the eager first pass; only the step's own kernels (libllmk and
    # hipBLASLt), not the bench's spin or fill kernels in between
    steps = [r for r in rows[starts[1]:starts[-1]]
             if "llmk" in r["Kernel_Name"] or r["Kernel_Name"].startswith("Cijk")]
    n_steps = len(starts) - 2
    agg = {}
    for r in steps:
        key = (r["Kernel_Name"], grid(r))
        agg.setdefault(key, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    print(f"# engine decode step (Llama-3.2-1B shape, {n_rows} rows), {n_steps} graph replays")
    print("# launches/step  mean_us  us/step  grid  kernel")
    total = 0.0
    for (name, g), d in sorted(agg.items(), key=lambda kv: -sum(kv[1])):
        per = sum(d) / n_steps
        total += per
        print(f"{len(d) / n_steps:8.2f} {sum(d) / len(d):9.2f} {per:9.1f} {g:9d}  {name[:100]}")
    print(f"# sum of kernel time per step: {total:.1f} us")


def summarize_sched(trace_dir, min_passes=20, top=10):
    """Forward passes of the scheduler workload, grouped by row count: a pass runs from an
    embedding gather to the next argmax (a gather of logit rows inside the pass is part of it).
    For every row count with at least min_passes passes: passes, kernel time per pass, and the
    top kernels (launches per pass, mean duration, time per pass, grid)."""
    import csv
    import glob
    rows = []
    for f in glob.glob(os.path.join(trace_dir, "**", "*kernel_trace.csv"), recursive=True):
        rows += list(csv.DictReader(open(f)))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))

    def grid(r):
        return int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])

    passes, cur = {}, None
    for r in rows:
        name = r["Kernel_Name"]
        if "llmk" not in name and not name.startswith("Cijk"):
            continue
        if cur is None:
            if "k_embedding" not in name:
                continue
            cur = {"n": grid(r) // 64, "k": []}
        cur["k"].append((name, grid(r), (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3))
        if "k_argmax" in name:
            passes.setdefault(cur["n"], []).append(cur["k"])
            cur = None
    print("# engine forward passes of the scheduler workload, by row count")
    for n in sorted(passes):
        ps = passes[n]
        if len(ps) < min_passes:
            continue
        agg = {}
        for p_ in ps:
            for name, g, d in p_:
                agg.setdefault((name, g), []).append(d)
        total = sum(sum(d) for d in agg.values()) / len(ps)
        print(f"# {n} rows: {len(ps)} passes, kernel time {total:.1f} us per pass")
        print("# launches/pass  mean_us  us/pass  grid  kernel")
        for (name, g), d in sorted(agg.items(), key=lambda kv: -sum(kv[1]))[:top]:
            print(f"{len(d) / len(ps):8.2f} {sum(d) / len(d):9.2f} {sum(d) / len(ps):9.1f} "
                  f"{g:9d}  {name[:100]}")


class Timer:
    """Two timed passes of `steps` launches each.

    1. Host wall clock: `steps` back-to-back launches, torch.cuda.synchronize() on both sides.
    2. HIP events: filler launches (3 ms of GPU time) and then the `steps` timed launches are
       enqueued back to back, with one event recorded right before the first timed launch and one
       right after the last, on the launching stream. Where the host enqueues more slowly than
       the GPU executes, a spin kernel holds the stream until all of it is enqueued. The mean
       launch duration is the event interval / steps: the launches run back to back on the GPU.
    """

    def __init__(self, torch):
        self.torch = torch
        self.cycles_per_s = None

    def _calibrate(self):
        torch = self.torch
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        n = 1 << 22
        torch.cuda._sleep(n)  # warm the spin kernel
        a.record()
        torch.cuda._sleep(n)
        b.record()
        torch.cuda.synchronize()
        self.cycles_per_s = n / max(a.elapsed_time(b) * 1e-3, 1e-9)

    def run(self, launch, n_sets: int, steps: int, warmup: int):
        torch = self.torch
        if self.cycles_per_s is None:
            self._calibrate()
        # Warm-up: at least `warmup` launches and at least WARM_S seconds of back-to-back
        # launches, so that clocks have ramped up from the idle state before timing starts
        # (the first milliseconds after idle measured up to 15% slow).
        t_w = time.perf_counter()
        i = 0
        while i < warmup or time.perf_counter() - t_w < WARM_S:
            launch(i % n_sets)
            i += 1
            if i % 64 == 0:
                torch.cuda.synchronize()
        torch.cuda.synchronize()
        warmup = i
        t0 = time.perf_counter()
        for i in range(steps):
            launch((warmup + i) % n_sets)
        enq = (time.perf_counter() - t0) / steps  # host time to enqueue one launch
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0

        # Event pass: `fill` launches of the same kernel (at least 3 ms of GPU time) run ahead of
        # the start event, so the queue is full and the clocks are up when timing starts. When
        # the host enqueues more slowly than the GPU executes (short kernels), the stream is
        # first held by a spin kernel until everything is enqueued.
        stream = torch.cuda.current_stream()
        fill = min(4000, max(8, int(3e-3 / max(wall / steps, 1e-7))))
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        host_bound = enq > 0.5 * wall / steps
        hold = 3 * enq * (fill + steps) if host_bound else 0.0
        if host_bound:
            torch.cuda._sleep(int(hold * self.cycles_per_s))
        t1 = time.perf_counter()
        for i in range(fill):
            launch(i % n_sets)
        a.record(stream)
        for i in range(steps):
            launch((warmup + steps + i) % n_sets)
        b.record(stream)
        enqueue = time.perf_counter() - t1
        torch.cuda.synchronize()
        ev = a.elapsed_time(b) * 1e-3
        return {"wall_s": wall, "mean_s": ev / steps, "event_s": ev, "enqueue_s": enqueue,
                "hold_s": hold, "host_bound": host_bound,
                "queue_prefilled": (enqueue < hold) if host_bound else True, "steps": steps}


def kernel_entry(name, nbytes, t, traffic=None, extra=None):
    achieved = nbytes / t["mean_s"] / 1e9
    e = {"bytes": nbytes, "us_mean": round(t["mean_s"] * 1e6, 3),
         "us_wall_per_step": round(t["wall_s"] / max(1, t.get("steps", 1)) * 1e6, 3),
         "GBps": round(achieved, 1), "frac_of_peak": round(achieved / PEAK_GBS, 4),
         "queue_prefilled": t["queue_prefilled"]}
    if traffic is not None:
        e["traffic_bytes"] = traffic
    if extra:
        e.update(extra)
    log(f"  {name:34s} {e['us_mean']:9.2f} us  {e['GBps']:8.1f} GB/s  "
        f"{100 * e['frac_of_peak']:5.1f}% of 8 TB/s  (wall {e['us_wall_per_step']:.2f} us/step)")
    return e


def sets_for(bytes_per_set: int, floor: int = 1 << 30, most: int = 64) -> int:
    return max(2, min(most, -(-floor // max(1, bytes_per_set)) + 1))


def main() -> int:
    args = parse_args()
    if args.summarize_profiles:
        return summarize_profiles(*args.summarize_profiles)  # 1 when a launch shape is missing
    if args.summarize_sched:
        summarize_sched(args.summarize_sched)
        return 0
    if args.summarize_step:
        summarize_step(args.summarize_step[0],
                       int(args.summarize_step[1]) if len(args.summarize_step) > 1 else 256)
        return 0
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (the kernels are single-GPU; this build has no "
              f"multi-GPU path): --gpus {args.gpus} is not supported", file=sys.stderr)
        return 2
    import numpy as np
    import torch

    sys.path.insert(0, ROOT)
    from __graft_entry__ import load_llmk
    llmk = load_llmk()
    import llmk.workloads as wl

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    timer = Timer(torch)
    traffic = read_traffic()
    K, W = args.steps, args.warmup
    log(f"device: {torch.cuda.get_device_name(dev)}  steps={K} warmup={W}")
    kernels = {}

    # ---------------- headline: fused residual add + RMSNorm [8192, 2048] ----------------
    rows, hidden = 8192, wl.HIDDEN
    nbytes = wl.bytes_add_rmsnorm(rows, hidden)
    R = sets_for(3 * rows * hidden * 2)
    sets = [wl.add_rmsnorm_inputs(rows, hidden, seed=wl.SEED_BASE + 2 + 100 * i) for i in range(R)]
    w = sets[0]["w"]

    def launch_add_rmsnorm(i):
        s = sets[i]
        llmk.add_rmsnorm(s["residual"], s["x"], w, s["out"], rows, hidden, wl.EPS)

    t = timer.run(launch_add_rmsnorm, R, K, W)
    head = kernel_entry("add_rmsnorm [8192,2048]", nbytes, t, traffic.get("add_rmsnorm_8192x2048"),
                        {"sets": R})
    kernels["add_rmsnorm_8192x2048"] = head
    headline_wall = t["wall_s"]
    cpu_inputs = {k: sets[0][k].cpu().contiguous() for k in ("residual", "x", "w")}
    del sets
    torch.cuda.empty_cache()

    if args.kernels == "step":
        kernels.update(bench_decode_step(llmk, wl, timer, torch, np, dev, K, W))
    if args.kernels == "step8":
        kernels.update(bench_decode_step(llmk, wl, timer, torch, np, dev, K, W, n_seqs=8))
    if args.kernels == "sched":
        kernels.update(bench_scheduler(llmk, wl, torch, np, dev))

    if args.kernels == "all":
        # config 1: RMSNorm [16, 2048] (the reference's CPU-plumbing case, on the GPU)
        sets1 = [wl.add_rmsnorm_inputs(16, hidden, seed=wl.SEED_BASE + 1 + 100 * i)
                 for i in range(8)]
        t = timer.run(lambda i: llmk.rmsnorm(sets1[i]["x"], sets1[i]["w"], sets1[i]["out"], 16,
                                             hidden, wl.EPS), 8, K, W)
        kernels["rmsnorm_16x2048"] = kernel_entry("rmsnorm [16,2048]",
                                                  wl.bytes_rmsnorm(16, hidden), t,
                                                  traffic.get("rmsnorm_16x2048"))
        del sets1

        # config 3: RoPE, Q [8192,32,64] + K [8192,8,64], positions < 131072
        inv = torch.tensor(llmk.compute_rope_inv_freq(wl.HEAD_DIM, *wl.ROPE_ARGS),
                           dtype=torch.float32, device=dev)
        T = 8192
        R3 = sets_for(wl.bytes_rope(T, wl.N_HEADS, wl.N_KV, wl.HEAD_DIM) // 2)
        sets3 = [wl.rope_inputs(T, seed=wl.SEED_BASE + 3 + 100 * i, inv_freq=inv)
                 for i in range(R3)]
        t = timer.run(lambda i: llmk.rope_apply(sets3[i]["q"], sets3[i]["k"],
                                                sets3[i]["positions"], inv, T, wl.N_HEADS,
                                                wl.N_KV, wl.HEAD_DIM), R3, K, W)
        kernels["rope_8192"] = kernel_entry(
            "rope_apply Q+K [8192 tokens]", wl.bytes_rope(T, wl.N_HEADS, wl.N_KV, wl.HEAD_DIM),
            t, traffic.get("rope_8192"), {"sets": R3})
        del sets3

        # config 4a: SwiGLU [8192, 8192]
        n = 8192 * wl.INTER
        R4 = sets_for(wl.bytes_swiglu(n))
        sets4 = [wl.swiglu_inputs(seed=wl.SEED_BASE + 4 + 100 * i) for i in range(R4)]
        t = timer.run(lambda i: llmk.swiglu(sets4[i]["gate"], sets4[i]["up"], sets4[i]["out"], n),
                      R4, K, W)
        kernels["swiglu_8192x8192"] = kernel_entry("swiglu [8192,8192]", wl.bytes_swiglu(n), t,
                                                   traffic.get("swiglu_8192x8192"), {"sets": R4})
        del sets4
        torch.cuda.empty_cache()

        # config 4b: embedding gather of 8192 ids from [128256, 2048]. Four tables (2.1 GB)
        # so a row read by one launch is rarely still cached when its table comes round again.
        tables = [wl.embedding_table(seed=wl.SEED_BASE + 40 + 100 * i) for i in range(4)]
        R5 = 16
        sets5 = [wl.embedding_inputs(8192, tables[i % 4], seed=wl.SEED_BASE + 41 + 100 * i)
                 for i in range(R5)]
        t = timer.run(lambda i: llmk.embedding_lookup(sets5[i]["table"], sets5[i]["ids"],
                                                      sets5[i]["out"], 8192, hidden,
                                                      check_indices=False), R5, K, W)
        kernels["embedding_8192"] = kernel_entry(
            "embedding_lookup 8192 of 128256", wl.bytes_embedding(8192, hidden), t,
            traffic.get("embedding_8192"), {"sets": R5, "tables": 4,
                                       "note": "ids uniform; ~3% duplicate rows per launch"})
        table = tables[0]
        del sets5, tables

        # config 5: decode-step non-GEMM pass, 16 layers x 256 sequences, in a HIP graph
        p = wl.decode_pass_inputs(inv, table=table)
        dp = llmk.DecodeNonGemmPass(p.table, p.token_ids, p.residual, p.block_tables,
                                    p.positions, p.inv_freq, p.per_layer, n_heads=wl.N_HEADS,
                                    n_kv_heads=wl.N_KV, head_dim=wl.HEAD_DIM, inter=wl.INTER,
                                    page_size=wl.PAGE, max_pages=p.max_pages, eps=wl.EPS)
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            dp.run()
        torch.cuda.current_stream().wait_stream(s)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            dp.run()
        t = timer.run(lambda i: graph.replay(), 1, max(20, K // 4), max(5, W // 4))
        kernels["decode_pass_16x256"] = kernel_entry(
            "decode pass 16 layers x 256 (graph)", wl.bytes_decode_pass(256, 16), t, None,
            {"launches": 1 + 3 * 16, "layers": 16, "seqs": 256,
             "note": "footprint 321 MB (> 256 MB MALL); one HIP graph of 49 kernels"})
        t = timer.run(lambda i: dp.run(), 1, max(20, K // 4), max(5, W // 4))
        kernels["decode_pass_16x256_eager"] = kernel_entry(
            "decode pass 16 layers x 256 (eager)", wl.bytes_decode_pass(256, 16), t)
        del p, dp, graph, table
        torch.cuda.empty_cache()

        # decode attention over the paged pool (the pool's consumer): 256 sequences with
        # lengths uniform in [1, 2048], and the reference's bench shape, 16 sequences x 2048
        # (ref: bench/bench_attention_compare.cu). Split count: choose_num_splits' default.
        lens = wl.attention_lens()
        nb_attn = wl.bytes_attention(lens)
        if nb_attn != ATTN_BYTES_256:
            raise RuntimeError(f"attention workload bytes {nb_attn} != {ATTN_BYTES_256}")
        for label, lens_b, R6 in (("attention_decode_256", lens, 2),
                                  ("attention_decode_16x2048", np.full(16, 2048), 17)):
            splits = llmk.choose_num_splits(lens_b.size, wl.N_KV, int(lens_b.max()))
            sets6 = [wl.attention_inputs(lens_b, num_splits=splits,
                                         seed=wl.SEED_BASE + 6 + 100 * i) for i in range(R6)]

            def launch_attn(i, sets6=sets6, splits=splits):
                a = sets6[i]
                llmk.attention_decode_fast(a["q"], a["k_pool"], a["v_pool"], a["block_tables"],
                                           a["seq_lens"], a["out"], a["workspace"], a["n"],
                                           a["max_pages"], wl.PAGE, wl.N_HEADS, wl.N_KV,
                                           wl.HEAD_DIM, splits, check_indices=False)

            t = timer.run(launch_attn, R6, K, W)
            kernels[label] = kernel_entry(
                f"attention_decode_fast {label.split('_')[-1]}", wl.bytes_attention(lens_b), t,
                traffic.get(label), {"sets": R6, "num_splits": splits, "seqs": int(lens_b.size),
                                     "context_tokens": int(lens_b.sum()),
                                     "launches": 2, "note": "page-balanced split + merge"})
            del sets6
            torch.cuda.empty_cache()

        # argmax over the logits of a decode batch: [256, 128256] (ref: kernels/argmax.cu,
        # engine/batched.cu:150). 17 sets of 65.7 MB rotate through more than 1 GB.
        R7, n7 = 17, 256
        g7 = torch.Generator(device=dev)
        g7.manual_seed(wl.SEED_BASE + 7)
        logits = [torch.randn((n7, wl.VOCAB), generator=g7, device=dev).half()
                  for _ in range(R7)]
        am_out = torch.empty(n7, dtype=torch.int32, device=dev)
        t = timer.run(lambda i: llmk.argmax_rows(logits[i], am_out, n7, wl.VOCAB), R7, K, W)
        kernels["argmax_256x128256"] = kernel_entry(
            "argmax_rows [256,128256]", wl.bytes_argmax(n7, wl.VOCAB), t,
            traffic.get("argmax_256x128256"), {"sets": R7})
        del logits
        torch.cuda.empty_cache()

        # the whole decode step of the engine (Llama-3.2-1B shape, seeded random weights):
        # 256 sequences with context lengths uniform in [1, 2048] (the attention workload), one
        # new token each, every layer's K/V pool pre-filled for the cached positions; one HIP
        # graph per step (ref: engine/batched.cu:81-120, model_decode_batch_greedy :146-150)
        kernels.update(bench_decode_step(llmk, wl, timer, torch, np, dev, K, W))
        # the same with 8 sequences: the fused few-rows pass (projections streaming the weights
        # with the norms, RoPE + scatter, SwiGLU and residual adds inside them)
        kernels.update(bench_decode_step(llmk, wl, timer, torch, np, dev, K, W, n_seqs=8))

        # continuous batching on the engine: the reference's scheduler workload, one request
        # at a time and up to 8 at once (ref: tests/test_scheduler.cu, engine/scheduler.cu)
        kernels.update(bench_scheduler(llmk, wl, torch, np, dev))

        # copy probe: practical HBM ceiling (ref: bench/bandwidth.cu)
        nb = 1 << 30
        bufs = [torch.empty(nb, dtype=torch.uint8, device=dev) for _ in range(4)]
        t = timer.run(lambda i: llmk.copy_bytes(bufs[2 * (i % 2)], bufs[2 * (i % 2) + 1], nb),
                      2, max(20, K // 4), 5)
        kernels["copy_1GiB"] = kernel_entry("copy probe 1 GiB", 2 * nb, t,
                                            traffic.get("copy_1GiB"))
        del bufs

    # ---------------- CPU baseline: the scalar oracle on the host cores ----------------
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(cpu_inputs, rows, hidden, nbytes, args.cpu_seconds, wl.EPS)

    value = nbytes * K / headline_wall / 1e9
    rec = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": K,
        "warmup": W, "ms_per_step": round(headline_wall / K * 1e3, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16", "data": "synthetic",
        "config": {"workload": "fused residual add + RMSNorm fp16 [8192,2048] (configs[1])",
                   "rows": rows, "hidden": hidden, "eps": wl.EPS, "accumulate": "f32",
                   "input_sets": head["sets"], "algorithmic_bytes_per_step": nbytes},
        "roofline": {"bound": "hbm", "achieved": head["GBps"], "peak": PEAK_GBS,
                     "unit": "GB/s", "frac": round(head["GBps"] / PEAK_GBS, 4),
                     "traffic": traffic.get("add_rmsnorm_8192x2048")},
        "cpu_baseline": cpu,
        "kernels": kernels,
    }
    print(json.dumps(rec), flush=True)
    return 0


def bench_decode_step(llmk, wl, timer, torch, np, dev, K, W, n_seqs=256) -> dict:
    import importlib
    weights = importlib.import_module("llmk.weights")
    cfg = llmk.ModelConfig()
    lens = wl.attention_lens(n_seqs)
    tokens, pos, tables, used = wl.decode_step_rows(lens)
    n = lens.size
    eng = llmk.Engine(cfg, max_rows=n, max_pages=128, num_pages=used)
    w = weights.random_weights(cfg, wl.SEED_BASE + 9, device=dev)
    eng.set_weights(*weights.engine_layers(w, cfg))
    del w
    g = torch.Generator(device=dev)
    g.manual_seed(wl.SEED_BASE + 10)
    fill = torch.randn(used * wl.PAGE * wl.N_KV * wl.HEAD_DIM, generator=g, device=dev).half()
    for l in range(cfg.n_layers):
        for which in (llmk.BUF_K_POOL, llmk.BUF_V_POOL):
            eng.write_pool(which, l, fill)
    del fill
    torch.cuda.empty_cache()
    eng.tune(n)     # time hipBLASLt's candidates for this batch's projection shapes
    eng.set_rows(tokens, pos, tables)
    eng.forward(n)  # eager once before capture
    torch.cuda.synchronize()
    if not torch.isfinite(eng.logits(n).float()).all():
        raise RuntimeError("decode step produced non-finite logits")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        eng.forward(n, stream=s)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        eng.forward(n)
    steps = max(20, K // 4)
    t = timer.run(lambda i: graph.replay(), 1, steps, max(5, W // 4))
    nbytes = wl.bytes_decode_step(lens)
    path = ("fused few-rows projections (libllmk) with the norms, RoPE + scatter, SwiGLU and "
            "residual adds inside them" if n <= llmk.LINEAR_ROWS_MAX else
            "hipBLASLt projections + libllmk kernels")
    e = kernel_entry(f"decode step 1B, {n} seqs (graph)", nbytes, t, None, {
        "tokens_per_s": round(n / t["mean_s"], 1), "seqs": int(n),
        "context_tokens": int(lens.sum()), "layers": cfg.n_layers,
        "note": f"engine forward pass: {path}, one HIP graph; bytes = sum of the step's "
                "kernels' algorithmic bytes (weights 2.47 GB, KV cache reads, activations "
                "between kernels)"})
    log(f"    -> {e['tokens_per_s']:.0f} tokens/s")
    eng.close()
    del graph
    torch.cuda.empty_cache()
    return {f"decode_step_1b_{n}": e}


def bench_scheduler(llmk, wl, torch, np, dev) -> dict:
    """The reference's scheduler benchmark on the engine (Llama-3.2-1B shape, seeded random
    weights): 24 requests (prompts of 5 to 402 tokens, 32 new tokens each, one eligible every 2
    iterations), 256 pages of 16, one request at a time and up to 8 at once, two rounds each as
    the reference runs them (ref: tests/test_scheduler.cu:14-76). words/s = new tokens over the
    scheduler's own wall clock (first iteration to last retirement), as the reference reports
    it. Decode steps of each batch size run from the engine's HIP graph cache."""
    import importlib
    weights = importlib.import_module("llmk.weights")
    cfg = llmk.ModelConfig()
    max_len = max(wl.SCHED_PROMPT_LENS) + wl.SCHED_NEW
    max_pages = (max_len + wl.PAGE - 1) // wl.PAGE
    max_rows = 512  # the longest prompt (402 tokens) prefills in one pass
    eng = llmk.Engine(cfg, max_rows=max_rows, max_pages=max_pages, num_pages=wl.SCHED_PAGES)
    # A wide embedding (std 0.5) makes the logits peaked, so that the greedy tokens do not hinge
    # on last-bit differences: a sequence's bits depend on its batch (the attention's split
    # count follows the batch size), as cuBLAS results do in the reference.
    w = weights.random_weights(cfg, wl.SEED_BASE + 9, device=dev, embed_std=0.5)
    eng.set_weights(*weights.engine_layers(w, cfg))
    del w
    torch.cuda.empty_cache()
    stream = torch.cuda.Stream()
    model = eng.sched_model(stream)
    reqs = wl.scheduler_requests()
    order = np.random.default_rng(wl.SEED_BASE + 12).permutation(wl.SCHED_PAGES).astype(np.int32)

    def run(rs, max_running):
        pages = llmk.PageAllocator(wl.SCHED_PAGES)
        pages.set_free_list(order)
        outs, stats, _ = llmk.run_scheduler(rs, max_running, max_pages, wl.PAGE, pages, model)
        if pages.num_free() != wl.SCHED_PAGES:
            raise RuntimeError("scheduler run leaked pages")
        return outs, stats

    run(reqs[:2], wl.SCHED_MAX_RUNNING)  # warm-up, as the reference does
    run(reqs[:wl.SCHED_MAX_RUNNING], wl.SCHED_MAX_RUNNING)  # captures the decode graphs
    rounds = []
    outputs = {}
    for rnd in (1, 2):
        for mr in (1, wl.SCHED_MAX_RUNNING):
            outs, st = run(reqs, mr)
            if mr in outputs and outputs[mr] != outs:
                raise RuntimeError("scheduler outputs changed between rounds")
            outputs[mr] = outs
            wps = st["total_words"] / (st["total_ms"] * 1e-3)
            rounds.append({"round": rnd, "max_running": mr, "decode_steps": st["decode_steps"],
                           "mean_batch": round(st["mean_batch"], 2),
                           "total_ms": round(st["total_ms"], 2),
                           "prefill_ms": round(st["prefill_ms"], 2),
                           "decode_ms": round(st["decode_ms"], 2),
                           "words_per_s": round(wps, 1)})
            log(f"  scheduler round {rnd}, up to {mr} at once: {st['decode_steps']} decode "
                f"steps, mean batch {st['mean_batch']:.1f}, {st['total_ms']:.1f} ms, "
                f"{wps:.0f} words/s")
    if outputs[1] != outputs[wl.SCHED_MAX_RUNNING]:
        raise RuntimeError("batched and one-at-a-time scheduler outputs differ")
    best = {mr: max(r["words_per_s"] for r in rounds if r["max_running"] == mr)
            for mr in (1, wl.SCHED_MAX_RUNNING)}
    eng.close()
    torch.cuda.empty_cache()
    return {"scheduler_24x32_1b": {
        "label": "continuous batching, 24 requests x 32 new tokens (Llama-3.2-1B shape)",
        "words_per_s": best[wl.SCHED_MAX_RUNNING], "words_per_s_one_at_a_time": best[1],
        "gain": round(best[wl.SCHED_MAX_RUNNING] / best[1], 2), "rounds": rounds,
        "note": "reference on an RTX 4050 Laptop: 249 words/s up to 8 at once, 60 one at a "
                "time (docs/scheduler_results.md); outputs identical in both modes"}}


def cpu_baseline(inp, rows, hidden, nbytes, seconds, eps):
    """Times the oracle's add_rmsnorm on host copies of the first input set: all usable cores
    (threads split by rows), then one core, over a bounded number of full [8192, 2048] passes."""
    import numpy as np
    sys.path.insert(0, ROOT)
    import oracle
    oracle.lib()
    r0 = inp["residual"].numpy().view(np.uint16).copy()
    x = inp["x"].numpy().view(np.uint16)
    w = inp["w"].numpy().view(np.uint16)
    threads = max(1, min(16, len(os.sched_getaffinity(0))))

    def timed(nthreads, budget):
        reps, t0 = 0, time.perf_counter()
        while True:
            r = r0.copy()
            oracle.add_rmsnorm(r, x, w, rows, hidden, eps, threads=nthreads)
            reps += 1
            el = time.perf_counter() - t0
            if el >= budget:
                return reps, el

    reps, el = timed(threads, seconds * 0.7)
    reps1, el1 = timed(1, seconds * 0.3)
    v = nbytes * reps / el / 1e9
    v1 = nbytes * reps1 / el1 / 1e9
    log(f"  CPU oracle add_rmsnorm: {v:.2f} GB/s on {threads} threads, {v1:.2f} GB/s on 1")
    return {"value": round(v, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{reps} full [8192,2048] add_rmsnorm passes ({el:.1f} s) of the scalar C "
                      f"oracle, rows split over {threads} threads",
            "one_core": {"value": round(v1, 3), "unit": "GB/s", "cores": 1,
                         "sample": f"{reps1} passes ({el1:.1f} s)"}}


if __name__ == "__main__":
    sys.exit(main())
