#!/usr/bin/env python3
"""Benchmark of libllmk's non-GEMM layer kernels on one MI355X.

Headline (the JSON line's `value`): the fused residual add + RMSNorm over [8192, 2048] fp16
-- whole-job throughput in GB/s of algorithmic bytes (inputs read once,
outputs written once), inputs resident in HBM before the timed region. One step = one launch
over the full batch. The other BASELINE configurations (RMSNorm [16,2048], RoPE, SwiGLU,
embedding gather, the 16-layer decode-step pass captured in HIP graphs) are measured the same
way and reported under "kernels", each with the scalar CPU oracle of the same work timed on the
host's cores in the same run ("cpu") and the bandwidth ceiling of its traffic mix ("ceiling").
The pass is also broken down by stage: one HIP graph per op type (16 launches each) and a graph
of empty kernels in the pass's 49 launch shapes, its launch floor (ref:
bench/bench_breakdown.cu:18-26,58-104 times each stage of a layer with its own events).

Caches: MI355X has a 256 MB Infinity Cache (MALL) in front of HBM and 4 MB of L2 per XCD. Each
kernel cycles through enough independent input sets that the data of a launch was last
touched more than 1 GB of traffic earlier, so it cannot be served from the MALL.

Timing: `ms_per_step` = host wall time of K back-to-back steps, synchronised on both sides, / K;
`value` = algorithmic bytes per step / ms_per_step. Then K more launches are enqueued behind a
short spin kernel with a HIP event right before the first and right after the last, recorded on
the stream they are launched on (torch's current stream); the mean launch duration is the event
interval / K, and `roofline.achieved` = algorithmic bytes / that mean.

Ceilings (ref: bench/bandwidth.cu:11-62, a copy kernel swept over block and grid sizes): the
bandwidth probes of llmk_bw_probe -- read-only, 1:1 copy, 2:1 read:write, in-place rewrite,
write-only -- swept over grid and unroll at 1 GiB, and run again at each kernel's own byte
count and traffic mix.

Profiles: every measurement is preceded by a marker launch (an empty kernel whose grid names the
section, SECTIONS below), so `--summarize-profiles` can group a rocprofv3 trace by section.

CPU baseline: the scalar C oracle of the same op (oracle/, test infrastructure) on the host's
cores, over a bounded sample of the same workload.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--kernels all|headline|...] [--no-cpu]
"""
from __future__ import annotations

import argparse
import ctypes
import glob
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
METRIC = ("achieved HBM GB/s (% of ~8 TB/s) per fused kernel; "
          "µs per 16-layer non-GEMM pass")
PEAK_GBS = 8000.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "llmk_kernels_bench_configs.txt")

# Marker launches: llmk_empty_launch(MARK_BASE + index, 64) before each measurement.
MARK_BASE = 50000
SECTIONS = ["headline", "rmsnorm_16", "rope_8192", "swiglu_8192", "embedding_8192",
            "pass_graph", "pass_eager", "pass_layers", "pass_floor", "pass_stage_embedding",
            "pass_stage_add_rmsnorm", "pass_stage_rope_kv_scatter", "pass_stage_swiglu",
            "pass_floor_stages", "attention_256", "attention_16x2048", "attention_sweep",
            "argmax", "step_256", "step_8", "sched", "probe_sweep", "probe_kernels", "copy_1GiB",
            "residual_add", "rmsnorm_8192", "kv_scatter_8192", "kv_scatter_batch_256",
            "pass2_graph", "pass2_layers", "pass_fused", "pass2_fused", "calib", "calib_resident",
            "calib_hbm", "end", "setup", "sched_ab", "pass_fused_eager", "pass2_fused_eager",
            "pass_layers_eager"]

# Launch shapes (blocks, threads) of the 16-layer pass at 256 sequences, from the launchers'
# grid rules: the embedding and add+RMSNorm take one 64-thread wave per row below 4096 rows
# (gather_scatter.hip rows_grid, norm.hip rmsnorm_launch); the fused RoPE + scatter one token
# per 256-thread block below 2048 tokens (rope.hip tokens_per_block: 48 vectors of 16 B per
# token, 2 per thread); SwiGLU one 16-byte vector of each input per lane in one-wave blocks
# (swiglu.hip) over 256 x 8192 values.
PASS_SHAPES = {"embedding": (256, 64), "add_rmsnorm": (256, 64),
               "rope_kv_scatter": (256, 256), "swiglu": (4096, 64)}


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--kernels", default="all",
                    choices=["all", "kernels", "headline", "configs", "pass", "attn", "probe",
                             "step", "step8", "sched", "rows", "calib"],
                    help="all: everything; kernels: all but the engine step and the scheduler "
                         "(for counter runs); headline: config 2 only; configs: configs 1-4, the "
                         "pass and the probes; pass: the decode pass and its breakdown; attn: decode "
                         "attention and its batch sweep; probe: bandwidth probes; step / step8: "
                         "the engine's decode step of 256 / 8 sequences; sched: the reference's "
                         "scheduler workload; rows: residual_add, RMSNorm [8192,2048] and the "
                         "two scatters; calib: the probes that calibrate the HBM counters "
                         "(config 2 is always measured)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--cpu-seconds", type=float, default=3.0,
                    help="CPU time per configuration (all cores 70%%, one core 30%%)")
    ap.add_argument("--warm-seconds", type=float, default=0.25,
                    help="minimum back-to-back warm-up per measurement")
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


# ---------------------------------------------------------------------------------------------
# rocprofv3 summaries
# ---------------------------------------------------------------------------------------------
# Decode attention over 256 sequences with lengths uniform in [1, 2048] (seed 0x5EED0006):
# the bytes of bytes_attention(attention_lens()) in cuda-llm-engine_amd/workloads.py.
ATTN_BYTES_256 = 546_019_628
ATTN_BYTES_16x2048 = 67_248_192  # 16 sequences x 2048 positions

# Kernel rows listed per section in the profile summary.
SECTION_ROWS = 12

# (label, section, kernel-name substring, grid size in work-items, algorithmic bytes) of each
# measured launch shape whose counters are reported; grid sizes follow from the launchers'
# grid choices at the benchmark shapes.
PROFILE_SHAPES = [
    # 8192 rows of 2048 fill one resident round at 8 rows per wave: 256 blocks of 4 waves
    ("add_rmsnorm_8192x2048", "headline", "k_rmsnorm_rowsILi8ELb1EE", 256 * 256, 134221824),
    # 8192 blocks of 256 threads over 2,097,152 vectors; the scatters: one row per wave, 4 waves
    # per block from 4096 rows
    ("residual_add_8192x2048", "residual_add", "k_residual_add_vec", 8192 * 256, 100663296),
    ("rmsnorm_8192x2048", "rmsnorm_8192", "k_rmsnorm_rowsILi8ELb0EE", 256 * 256, 67112960),
    ("kv_scatter_8192", "kv_scatter_8192", "k_kv_scatterILb0ELi1E", 2048 * 256, 16779264),
    ("kv_scatter_batch_256", "kv_scatter_batch_256", "k_kv_scatterILb1ELi1E", 256 * 64, 526336),
    ("rmsnorm_16x2048", "rmsnorm_16", "k_rmsnorm_waveILi4ELb0ELb1E", 16 * 64, 135168),
    # 16 tokens per 512-thread block, 10 vector tasks per thread (40 heads x 8 vectors x 16
    # tokens / 512)
    ("rope_8192", "rope_8192", "k_rope_vecILi4ELi10ELb0ELb0ELi512E", 512 * 512, 83918976),
    ("swiglu_8192x8192", "swiglu_8192", "k_swiglu_vecILi1E", 131072 * 64, 402653184),
    ("embedding_8192", "embedding_8192", "k_embedding_rowsILi8E", 256 * 256, 67141632),
    ("copy_1GiB", "copy_1GiB", "k_copy", 8192 * 256, 2 * (1 << 30)),
    # 256 blocks: one block of 256 threads on each of the 256 CUs.
    ("attention_decode_256", "attention_256", "k_attn_balancedILi8E", 256 * 256,
     ATTN_BYTES_256),
    ("attention_merge_256", "attention_256", "k_attn_mergeE|k_attn_merge(", 256 * 256, None),
    # 16 sequences take the sequence-split grid (32 splits of 4 pages, 16 blocks per split).
    ("attention_decode_16x2048", "attention_16x2048", "k_attn_splitILi8ELi0E", 32 * 256 * 16,
     ATTN_BYTES_16x2048),
    ("attention_merge_16x2048", "attention_16x2048", "k_attn_merge_many", 8 * 256 * 16, None),
    ("argmax_256x128256", "argmax", "k_argmax_vec", 256 * 1024, 256 * 128256 * 2 + 256 * 4),
    ("decode:embedding_256", "pass_graph", "k_embeddingILi0E", 256 * 64, 2098176),
    ("decode:add_rmsnorm_256x2048", "pass_graph", "k_rmsnorm_waveILi4ELb1ELb1E", 256 * 64,
     4198400),
    ("decode:rope_kv_scatter_256", "pass_graph", "k_rope_vecILi4ELi2ELb1ELb0E", 256 * 256,
     3147904),
    ("decode:swiglu_256x8192", "pass_graph", "k_swiglu_vecILi1E", 4096 * 64, 12582912),
    # the pass with one launch per layer: 256 norm rows, 256 RoPE tokens, 4096 SwiGLU chunks
    ("decode_layers:layer_256", "pass_layers", "k_layer_passILi4ELb0ELi6ELb0E|k_layer_pass<4, false, 6, false>",
     4608 * 64, 4198400 + 3147904 + 12582912),
    # the whole pass in one launch: 256 residual chains, 16 x 256 RoPE tokens, 16 x 2048 SwiGLU
    # chunks of two vectors per lane; bytes: what it must move (config 5's count less the
    # residual rows it keeps in registers, workloads.bytes_decode_pass_fused)
    ("decode_fused:pass_256", "pass_fused", "k_layers_fusedILi4ELi6ELb0ELb1E|k_layers_fused<4, 6, false, true>",
     (256 + 16 * 256 + 16 * 2048) * 64, 303139840),
]


# Counter calibration: for each launch shape of PROFILE_SHAPES, a bandwidth probe of the same
# traffic mix at the same byte count and the same input rotation (so the same share of its data
# can sit in the 256 MB MALL), run once per counter pass. FETCH_SIZE does not count the bytes
# read at a fixed ratio: it reads about half of them for data streamed from HBM and about all of
# them for data the caches hold, so each shape's counters are scaled by what they read for its
# own probe. (label, probe mode, unit bytes, sets); probe modes as llmk_bw_probe: 0 read,
# 1 copy (unit read, unit written), 2 read2 (2 units read, one written), 3 in place, 4 write.
CALIB_PROBES = [
    ("add_rmsnorm_8192x2048", 1, 67110912, 12),
    ("residual_add_8192x2048", 2, 33554432, 11),
    ("rmsnorm_8192x2048", 1, 33556480, 11),
    ("kv_scatter_8192", 1, 8390656, 64),
    ("kv_scatter_batch_256", 1, 263168, 16),
    ("rmsnorm_16x2048", 1, 67584, 8),
    ("rope_8192", 3, 41959488, 27),
    ("swiglu_8192x8192", 2, 134217728, 4),
    ("embedding_8192", 1, 33570816, 16),
    ("argmax_256x128256", 0, 65668096, 17),
    ("attention_decode_256", 0, ATTN_BYTES_256, 2),
    ("attention_decode_16x2048", 0, ATTN_BYTES_16x2048, 17),
    ("decode:embedding_256", 1, 1049088, 2),
    ("decode:add_rmsnorm_256x2048", 1, 2099200, 32),
    ("decode:rope_kv_scatter_256", 1, 1573952, 32),
    ("decode:swiglu_256x8192", 2, 4194304, 32),
    ("decode_layers:layer_256", 1, 9964608, 32),
    ("decode_fused:pass_256", 1, 151569920, 2),
]
CALIB_UNROLL = 4
CALIB_SWEEP_SIZES = (65536, 262144, 1048576, 2097152, 8388608, 33554432)
PROBE_READS = (1, 1, 2, 1, 0)   # units read per unit of buffer, by probe mode
PROBE_WRITES = (0, 1, 1, 1, 1)  # units written


def _probe_grid(unit: int, unroll: int = CALIB_UNROLL) -> int:
    """Work-items of a one-pass llmk_bw_probe launch over `unit` bytes."""
    nvec = unit // 16
    return -(-nvec // (256 * unroll)) * 256


def _name_matches(pattern: str, name: str) -> bool:
    """`pattern`: substrings separated by '|', any of which may occur in the kernel name
    (rocprofv3 prints some names mangled and some demangled)."""
    return any(p in name for p in pattern.split("|"))


def _grid(r) -> int:
    if "Grid_Size_X" in r:
        return int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
    return int(r["Grid_Size"])


def _csv_rows(d, suffix):
    import csv
    import glob
    out = []
    for f in glob.glob(os.path.join(d, "**", f"*{suffix}"), recursive=True):
        out += list(csv.DictReader(open(f)))
    return out


def _by_section(table):
    """Rows in dispatch order, each tagged with the section of the last marker before it;
    marker dispatches themselves are dropped."""
    table = sorted(table, key=lambda r: int(r["Dispatch_Id"]))
    cur, out = None, []
    for r in table:
        g = _grid(r)
        if "k_empty" in r["Kernel_Name"] and g % 64 == 0 and g // 64 >= MARK_BASE:
            i = g // 64 - MARK_BASE
            cur = SECTIONS[i] if i < len(SECTIONS) else None
            continue
        out.append((cur, r))
    return out


def summarize_profiles(trace_dir, fetch_dir, write_dir):
    """Per section of the run: every (kernel, grid) with its mean, min and max duration from the
    kernel trace; FETCH_SIZE and WRITE_SIZE per dispatch; and for the launch shapes of
    PROFILE_SHAPES the HBM traffic per launch, each counter scaled by what it reads for the
    1 GiB copy probe (1 GiB read, 1 GiB written). For the decode pass: kernel time per pass."""
    dur = {}
    for sec, r in _by_section(_csv_rows(trace_dir, "kernel_trace.csv")):
        key = (sec, r["Kernel_Name"], _grid(r))
        dur.setdefault(key, []).append(
            (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-3)
    cnt = {}
    for d, cname in ((fetch_dir, "FETCH_SIZE"), (write_dir, "WRITE_SIZE")):
        table = [r for r in _csv_rows(d, "counter_collection.csv") if r["Counter_Name"] == cname]
        for sec, r in _by_section(table):
            cnt.setdefault((sec, r["Kernel_Name"], _grid(r), cname), []).append(
                float(r["Counter_Value"]))
    avg = {k: sum(v) / len(v) for k, v in cnt.items() if v}

    def find(section, name, grid):
        keys = [k for k in dur if k[0] == section and _name_matches(name, k[1]) and k[2] == grid]
        return keys[0] if keys else None

    print("# rocprofv3 summaries of bench.py on one MI355X (gfx950), made by:")
    print(f"#   rocprofv3 --kernel-trace --stats -f csv -d {trace_dir} -o bench -- "
          "python3 bench.py --no-cpu")
    print(f"#   rocprofv3 --pmc FETCH_SIZE -f csv -d {fetch_dir} -o fetch -- "
          "python3 bench.py --no-cpu --kernels kernels --steps 20 --warmup 2 --warm-seconds 0")
    print(f"#   rocprofv3 --pmc WRITE_SIZE -f csv -d {write_dir} -o write -- "
          "python3 bench.py --no-cpu --kernels kernels --steps 20 --warmup 2 --warm-seconds 0")
    print(f"#   python3 bench.py --summarize-profiles {trace_dir} {fetch_dir} {write_dir}")
    print("#")
    ck = find("copy_1GiB", "k_copy", 8192 * 256)
    if ck is None or (ck + ("FETCH_SIZE",)) not in avg or (ck + ("WRITE_SIZE",)) not in avg:
        print("copy_1GiB MISSING (kernel name or grid not found)")
        return 1
    copy_b = 1 << 30
    sf = copy_b / (avg[ck + ("FETCH_SIZE",)] * 1024)
    sw = copy_b / (avg[ck + ("WRITE_SIZE",)] * 1024)

    def probe_counts(section, mode, unit):
        pat = f"k_bw_probeILi{mode}ELi{CALIB_UNROLL}E|k_bw_probe<{mode}, {CALIB_UNROLL}>"
        pk = [k for k in avg if k[0] == section and k[3] == "FETCH_SIZE"
              and _name_matches(pat, k[1]) and k[2] == _probe_grid(unit)]
        if not pk:
            return None
        base = pk[0][:3]
        return avg.get(base + ("FETCH_SIZE",)), avg.get(base + ("WRITE_SIZE",))

    print("# Counter calibration: FETCH_SIZE and WRITE_SIZE of a one-pass copy probe (16-byte")
    print("# non-temporal accesses, 4 per thread) over the bytes read / written, by size; 'resident':")
    print("# 4 buffers rotated (they stay in the caches between launches), 'hbm': the launches walk")
    print("# 1 GiB of buffers (every launch reads from HBM). size_kib fetch_ratio write_ratio")
    for sec in ("calib_resident", "calib_hbm"):
        for size in CALIB_SWEEP_SIZES:
            c = probe_counts(sec, 1, size)
            if c is None or c[0] is None or c[1] is None:
                print(f"#   {sec:15s} {size >> 10:7d} MISSING")
                continue
            print(f"#   {sec:15s} {size >> 10:7d} {c[0] * 1024 / size:7.4f} {c[1] * 1024 / size:7.4f}")
    print("#")
    # Per launch shape: the factors of its own probe (same mix, bytes and rotation); the 1 GiB
    # copy probe's where a shape has none.
    own = {}
    for label, mode, unit, _sets in CALIB_PROBES:
        unit -= unit % 16
        c = probe_counts("calib", mode, unit)
        if c is None or not c[0] or not c[1]:
            continue
        f_ = PROBE_READS[mode] * unit / (c[0] * 1024) if PROBE_READS[mode] else sf
        w_ = PROBE_WRITES[mode] * unit / (c[1] * 1024) if PROBE_WRITES[mode] else sw
        own[label] = (f_, w_)
    print("# Launch shapes. us_mean: mean kernel duration in the kernel trace (all launches of the")
    print("# shape in its section). fetch_kib, write_kib: FETCH_SIZE and WRITE_SIZE per dispatch.")
    print("# traffic_bytes = fetch_kib*1024*f + write_kib*1024*w with (f, w) = factor_fetch,")
    print("# factor_write: bytes read (written) by the shape's own calibration probe over what the")
    print("# counter reads for it (CALIB_PROBES: same traffic mix, byte count and rotation).")
    print(f"# traffic_1gib: the same with the 1 GiB copy probe's factors ({sf:.4f}, {sw:.4f}).")
    missing = []
    for label, sec, name, g, alg in PROFILE_SHAPES:
        k = find(sec, name, g)
        if k is None:
            print(f"{label} MISSING (kernel name or grid not found in section {sec})")
            missing.append(label)
            continue
        d = dur[k]
        f, w = avg.get(k + ("FETCH_SIZE",)), avg.get(k + ("WRITE_SIZE",))
        line = (f"{label} us_mean={sum(d) / len(d):.3f} us_min={min(d):.3f} "
                f"us_max={max(d):.3f} calls={len(d)}")
        if f is not None and w is not None:
            fs, ws = own.get(label, (sf, sw))
            traffic = f * 1024 * fs + w * 1024 * ws
            line += (f" fetch_kib={f:.1f} write_kib={w:.1f} factor_fetch={fs:.4f} "
                     f"factor_write={ws:.4f} traffic_bytes={traffic:.0f} "
                     f"traffic_1gib={f * 1024 * sf + w * 1024 * sw:.0f}")
            if alg:
                line += f" algorithmic_bytes={alg} ratio={traffic / alg:.4f}"
        print(line)
    print("#")
    print("# The libllmk and hipBLASLt kernels of every section (input generation and the timer's")
    print("# spin kernel left out): calls, mean / min / max duration (us), grid (work-items), kernel;")
    print(f"# the {SECTION_ROWS} (kernel, grid) pairs with the most time per section, the rest in one")
    print("# line (in the argmax section: the engine's start-up, whose GEMM plan search times every")
    print("# candidate hipBLASLt solution a few times).")
    sections = []
    for k in dur:
        if k[0] not in sections:
            sections.append(k[0])
    for sec in sections:
        ks = [k for k in dur if k[0] == sec and _own_kernel(k[1])]
        if not ks:
            continue
        print(f"## section {sec}")
        ks.sort(key=lambda k: -sum(dur[k]))
        for k in ks[:SECTION_ROWS]:
            d = dur[k]
            print(f"#   {len(d):6d} {sum(d) / len(d):9.3f} {min(d):9.3f} {max(d):9.3f} "
                  f"{k[2]:9d}  {k[1][:96]}")
        rest = ks[SECTION_ROWS:]
        if rest:
            print(f"#   ... {len(rest)} more pairs: {sum(len(dur[k]) for k in rest)} launches, "
                  f"{sum(sum(dur[k]) for k in rest):.1f} us in all")
    print("#")
    tagged = _by_section(_csv_rows(trace_dir, "kernel_trace.csv"))
    summarize_spread(tagged)
    print("#")
    summarize_pass(tagged, "pass_graph", "k_embedding", 49)
    summarize_pass(tagged, "pass_layers", "k_layer_passILi4ELb1E|k_layer_pass<4, true", 16)
    print("#")
    summarize_pass(tagged, "pass2_graph", "k_embedding", 65)
    print("#")
    summarize_pass(tagged, "pass2_layers", "k_layer_passILi4ELb1E|k_layer_pass<4, true", 16)
    print("#")
    summarize_pass(tagged, "pass_fused", "k_layers_fused", 1)
    print("#")
    summarize_pass(tagged, "pass2_fused", "k_layers_fused", 1)
    return 1 if missing else 0


def summarize_spread(tagged):
    """Duration spread of each configuration kernel in its section, by what precedes the
    launch on the GPU: back to back (the previous kernel ended < 1 us before it started), after
    a short gap (1-20 us: the host's enqueue or an event), or after idle (> 20 us: a
    synchronisation, between timing passes). Quantiles in us."""
    import statistics
    print("# Duration spread of the configuration kernels by the gap in front of each launch")
    print("# (back to back: < 1 us after the previous kernel's end; gap: 1-20 us; idle: > 20 us):")
    print("#   label  class  launches  mean  p1  p10  p50  p90  p99  max")
    by_sec = {}
    order = sorted((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), sec, r["Kernel_Name"],
                    _grid(r)) for sec, r in tagged)
    prev_end = None
    for st, en, sec, name, g in order:
        gap = None if prev_end is None else (st - prev_end) * 1e-3
        prev_end = en if prev_end is None else max(prev_end, en)
        by_sec.setdefault((sec, name, g), []).append(((en - st) * 1e-3, gap))
    for label, sec, name, g, alg in PROFILE_SHAPES:
        if sec.startswith("pass") or "merge" in label:
            continue
        keys = [k for k in by_sec if k[0] == sec and _name_matches(name, k[1]) and k[2] == g]
        if not keys:
            continue
        rows = by_sec[keys[0]]
        for cls, test in (("b2b", lambda x: x is not None and x < 1.0),
                          ("gap", lambda x: x is not None and 1.0 <= x <= 20.0),
                          ("idle", lambda x: x is None or x > 20.0)):
            d = sorted(v for v, gp in rows if test(gp))
            if not d:
                continue
            q = lambda f: d[min(len(d) - 1, int(f * len(d)))]
            print(f"#   {label:26s} {cls:4s} {len(d):6d} {statistics.fmean(d):7.3f} {q(0.01):7.3f} "
                  f"{q(0.1):7.3f} {q(0.5):7.3f} {q(0.9):7.3f} {q(0.99):7.3f} {d[-1]:7.3f}")


def _own_kernel(name: str) -> bool:
    return "llmk" in name or name.startswith("Cijk")


def summarize_pass(tagged, section, first, launches):
    """The 16-layer pass on the traced GPU timeline: each graph replay of the section is
    `launches` kernels from one whose name contains `first` on. Its span (first start to last
    end) is the pass as the GPU ran it under the profiler; the kernels' durations add up to the
    span less the gaps between them."""
    rows = [r for sec, r in tagged if sec == section and _own_kernel(r["Kernel_Name"])]
    passes, cur = [], None
    for r in rows:
        if _name_matches(first, r["Kernel_Name"]):
            cur = []
            passes.append(cur)
        if cur is not None:
            cur.append(r)
    passes = [p for p in passes if len(p) == launches]
    if not passes:
        print(f"# {section}: no complete passes found")
        return
    span = busy = 0.0
    per_kernel = {}
    for p in passes:
        st = [int(r["Start_Timestamp"]) for r in p]
        en = [int(r["End_Timestamp"]) for r in p]
        span += (max(en) - min(st)) * 1e-3
        for r in p:
            d = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-3
            busy += d
            per_kernel.setdefault(r["Kernel_Name"], []).append(d)
    n = len(passes)
    print(f"# {section}: {n} passes of {launches} kernels on the traced timeline: span "
          f"{span / n:.2f} us per pass = kernel durations {busy / n:.2f} us + gaps "
          f"{(span - busy) / n:.2f} us. Kernel tracing adds several us per dispatch of a graph "
          f"(the gaps), so the span is no measure of the unprofiled pass; a kernel's duration "
          f"includes its launch floor (an empty kernel's is 1.4-2.2 us).")
    for name, d in sorted(per_kernel.items(), key=lambda kv: -sum(kv[1])):
        print(f"#   {len(d) / n:6.2f} launches/pass x {sum(d) / len(d):7.3f} us = "
              f"{sum(d) / n:7.2f} us/pass  {name[:80]}")


def summarize_step(trace_dir, n_rows=256):
    """Kernels of the engine's decode step (the graph replays of the bench's step_256 or step_8
    section), grouped by kernel name and grid size: launches per step, mean duration, and time
    per step."""
    sec = "step_256" if n_rows == 256 else "step_8"
    rows = [r for s_, r in _by_section(_csv_rows(trace_dir, "kernel_trace.csv")) if s_ == sec]
    # only the step's own kernels (libllmk and hipBLASLt), not the bench's spin kernels
    steps = [r for r in rows if "llmk" in r["Kernel_Name"] or r["Kernel_Name"].startswith("Cijk")]
    n_steps = sum(1 for r in steps if "k_embedding" in r["Kernel_Name"]
                  and _grid(r) == n_rows * 64)
    if n_steps == 0:
        print(f"no decode steps found in section {sec}")
        return
    agg = {}
    for r in steps:
        key = (r["Kernel_Name"], _grid(r))
        agg.setdefault(key, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    print(f"# engine decode step (Llama-3.2-1B shape, {n_rows} rows), {n_steps} graph replays, "
          "made by:")
    print(f"#   rocprofv3 --kernel-trace --stats -f csv -d {trace_dir} -o bench -- "
          "python3 bench.py --no-cpu")
    print(f"#   python3 bench.py --summarize-step {trace_dir} {n_rows}")
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
    rows = [r for s_, r in _by_section(_csv_rows(trace_dir, "kernel_trace.csv"))
            if s_ == "sched"]
    passes, cur = {}, None
    for r in rows:
        name = r["Kernel_Name"]
        if "llmk" not in name and not name.startswith("Cijk"):
            continue
        if cur is None:
            if "k_embedding" not in name:
                continue
            cur = {"n": _grid(r) // 64, "k": []}
        cur["k"].append((name, _grid(r), (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3))
        if "k_argmax" in name:
            passes.setdefault(cur["n"], []).append(cur["k"])
            cur = None
    print("# engine forward passes of the scheduler workload, by row count, made by:")
    print(f"#   rocprofv3 --kernel-trace --stats -f csv -d {trace_dir} -o bench -- "
          "python3 bench.py --no-cpu")
    print(f"#   python3 bench.py --summarize-sched {trace_dir}")
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


# ---------------------------------------------------------------------------------------------
# timing
# ---------------------------------------------------------------------------------------------
class Timer:
    """Two timed passes of `steps` launches each.

    1. Host wall clock: `steps` back-to-back launches, torch.cuda.synchronize() on both sides.
    2. HIP events: filler launches (3 ms of GPU time) and then the `steps` timed launches are
       enqueued back to back, with one event recorded right before the first timed launch and one
       right after the last, on the launching stream. Where the host enqueues more slowly than
       the GPU executes, a spin kernel holds the stream until all of it is enqueued. The mean
       launch duration is the event interval / steps: the launches run back to back on the GPU.
    """

    def __init__(self, torch, warm_s: float):
        self.torch = torch
        self.warm_s = warm_s
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

    def run(self, launch, n_sets: int, steps: int, warmup: int, warm_s=None):
        torch = self.torch
        if self.cycles_per_s is None:
            self._calibrate()
        warm_s = self.warm_s if warm_s is None else warm_s
        # Warm-up: at least `warmup` launches and at least warm_s seconds of back-to-back
        # launches, so that clocks have ramped up from the idle state before timing starts
        # (the first milliseconds after idle measured up to 15% slow).
        t_w = time.perf_counter()
        i = 0
        while i < warmup or time.perf_counter() - t_w < warm_s:
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
    log(f"  {name:36s} {e['us_mean']:9.2f} us  {e['GBps']:8.1f} GB/s  "
        f"{100 * e['frac_of_peak']:5.1f}% of 8 TB/s  (wall {e['us_wall_per_step']:.2f} us/step)")
    return e


def write_step_rows(path, cfg, tokens, positions, tables, num_pages, max_pages) -> None:
    """The rows file llmk_step_bench reads (csrc/step_bench.hip): b"LLMKROWS", the
    llmk_model_config struct (`cfg`, a ctypes mirror of it), int32 n_rows, max_pages, num_pages,
    then int32 tokens[n], positions[n] and block_tables[n, max_pages] (zero-padded)."""
    import numpy as np
    tok = np.ascontiguousarray(tokens, np.int32).reshape(-1)
    n = tok.size
    pos = np.ascontiguousarray(positions, np.int32).reshape(-1)
    if pos.size != n:
        raise ValueError("tokens and positions differ in length")
    tab = np.asarray(tables, np.int32).reshape(n, -1)[:, :max_pages]
    tab = np.ascontiguousarray(np.pad(tab, ((0, 0), (0, max_pages - tab.shape[1]))))
    with open(path, "wb") as f:
        f.write(b"LLMKROWS")
        f.write(bytes(cfg))
        f.write(np.array([n, max_pages, num_pages], np.int32).tobytes())
        f.write(tok.tobytes())
        f.write(pos.tobytes())
        f.write(tab.tobytes())


def sets_for(bytes_per_set: int, floor: int = 1 << 30, most: int = 64) -> int:
    return max(2, min(most, -(-floor // max(1, bytes_per_set)) + 1))


class Bench:
    def __init__(self, args):
        import numpy as np
        import torch
        sys.path.insert(0, ROOT)
        from __graft_entry__ import load_llmk
        self.np, self.torch = np, torch
        self.llmk = load_llmk()
        import llmk.workloads as wl
        self.wl = wl
        self.args = args
        self.dev = torch.device("cuda:0")
        torch.cuda.set_device(self.dev)
        self.timer = Timer(torch, args.warm_seconds)
        self.traffic = read_traffic()
        self.K, self.W = args.steps, args.warmup
        self.kernels = {}
        self.cpu_inputs = {}  # host copies of one input set per configuration
        self.inv = torch.tensor(self.llmk.compute_rope_inv_freq(wl.HEAD_DIM, *wl.ROPE_ARGS),
                                dtype=torch.float32, device=self.dev)

    def mark(self, section: str) -> None:
        self.llmk.empty_launch(MARK_BASE + SECTIONS.index(section), 64)

    def run(self, launch, n_sets, steps=None, warmup=None):
        return self.timer.run(launch, n_sets, self.K if steps is None else steps,
                              self.W if warmup is None else warmup)

    def free(self):
        self.torch.cuda.synchronize()
        self.torch.cuda.empty_cache()

    # ------------------------------------------------------------------ configs 1-4
    def config2(self):
        wl, llmk = self.wl, self.llmk
        rows, hidden = 8192, wl.HIDDEN
        nbytes = wl.bytes_add_rmsnorm(rows, hidden)
        R = sets_for(3 * rows * hidden * 2)
        sets = [wl.add_rmsnorm_inputs(rows, hidden, seed=wl.SEED_BASE + 2 + 100 * i)
                for i in range(R)]
        w = sets[0]["w"]
        self.cpu_inputs["add_rmsnorm_8192x2048"] = {
            k: sets[0][k].cpu().numpy().view(self.np.uint16).copy() for k in ("residual", "x", "w")}

        def launch(i):
            s = sets[i]
            llmk.add_rmsnorm(s["residual"], s["x"], w, s["out"], rows, hidden, wl.EPS)

        self.mark("headline")
        t = self.run(launch, R)
        e = kernel_entry("add_rmsnorm [8192,2048]", nbytes, t,
                         self.traffic.get("add_rmsnorm_8192x2048"), {"sets": R})
        self.kernels["add_rmsnorm_8192x2048"] = e
        del sets
        self.free()
        return t, nbytes, R

    def config1(self):
        wl, llmk = self.wl, self.llmk
        hidden = wl.HIDDEN
        sets1 = [wl.add_rmsnorm_inputs(16, hidden, seed=wl.SEED_BASE + 1 + 100 * i)
                 for i in range(8)]
        self.cpu_inputs["rmsnorm_16x2048"] = {
            k: sets1[0][k].cpu().numpy().view(self.np.uint16).copy() for k in ("x", "w")}
        self.mark("rmsnorm_16")
        t = self.run(lambda i: llmk.rmsnorm(sets1[i]["x"], sets1[i]["w"], sets1[i]["out"], 16,
                                            hidden, wl.EPS), 8)
        self.kernels["rmsnorm_16x2048"] = kernel_entry(
            "rmsnorm [16,2048]", wl.bytes_rmsnorm(16, hidden), t,
            self.traffic.get("rmsnorm_16x2048"))
        del sets1

    def config3(self):
        wl, llmk = self.wl, self.llmk
        T = 8192
        nb = wl.bytes_rope(T, wl.N_HEADS, wl.N_KV, wl.HEAD_DIM)
        R3 = sets_for(nb // 2)
        sets3 = [wl.rope_inputs(T, seed=wl.SEED_BASE + 3 + 100 * i, inv_freq=self.inv)
                 for i in range(R3)]
        self.cpu_inputs["rope_8192"] = {
            "q": sets3[0]["q"].cpu().numpy().view(self.np.uint16).copy(),
            "k": sets3[0]["k"].cpu().numpy().view(self.np.uint16).copy(),
            "positions": sets3[0]["positions"].cpu().numpy().copy(),
            "inv": self.inv.cpu().numpy().copy()}
        self.mark("rope_8192")
        t = self.run(lambda i: llmk.rope_apply(sets3[i]["q"], sets3[i]["k"],
                                               sets3[i]["positions"], self.inv, T, wl.N_HEADS,
                                               wl.N_KV, wl.HEAD_DIM), R3)
        self.kernels["rope_8192"] = kernel_entry("rope_apply Q+K [8192 tokens]", nb, t,
                                                 self.traffic.get("rope_8192"), {"sets": R3})
        del sets3
        self.free()

    def config4a(self):
        wl, llmk = self.wl, self.llmk
        n = 8192 * wl.INTER
        R4 = sets_for(wl.bytes_swiglu(n))
        sets4 = [wl.swiglu_inputs(seed=wl.SEED_BASE + 4 + 100 * i) for i in range(R4)]
        self.cpu_inputs["swiglu_8192x8192"] = {
            k: sets4[0][k].cpu().numpy().view(self.np.uint16).copy() for k in ("gate", "up")}
        self.mark("swiglu_8192")
        t = self.run(lambda i: llmk.swiglu(sets4[i]["gate"], sets4[i]["up"], sets4[i]["out"], n),
                     R4)
        self.kernels["swiglu_8192x8192"] = kernel_entry(
            "swiglu [8192,8192]", wl.bytes_swiglu(n), t, self.traffic.get("swiglu_8192x8192"),
            {"sets": R4})
        del sets4
        self.free()

    def config4b(self):
        """Embedding gather of 8192 ids from [128256, 2048]. Four tables (2.1 GB) so a row read
        by one launch is rarely still cached when its table comes round again. Returns one
        table for the decode pass."""
        wl, llmk = self.wl, self.llmk
        hidden = wl.HIDDEN
        tables = [wl.embedding_table(seed=wl.SEED_BASE + 40 + 100 * i) for i in range(4)]
        R5 = 16
        sets5 = [wl.embedding_inputs(8192, tables[i % 4], seed=wl.SEED_BASE + 41 + 100 * i)
                 for i in range(R5)]
        # the CPU gathers cycle through the 16 id sets too (from one table): repeating one set
        # would serve its 33.5 MB of rows from the host's caches
        self.cpu_inputs["embedding_8192"] = {
            "table": tables[0].cpu().numpy().view(self.np.uint16),
            "ids": [s["ids"].cpu().numpy().copy() for s in sets5]}
        self.mark("embedding_8192")
        t = self.run(lambda i: llmk.embedding_lookup(sets5[i]["table"], sets5[i]["ids"],
                                                     sets5[i]["out"], 8192, hidden), R5)
        self.kernels["embedding_8192"] = kernel_entry(
            "embedding_lookup 8192 of 128256", wl.bytes_embedding(8192, hidden), t,
            self.traffic.get("embedding_8192"),
            {"sets": R5, "tables": 4, "note": "ids uniform; ~3% duplicate rows per launch"})
        table = tables[0]
        del sets5, tables
        self.free()
        return table

    # ------------------------------------------------------------------ rows a2, a3, a8, a9
    def other_rows(self):
        """The scope rows no configuration times on its own: residual_add (in place, as the
        reference's engine calls it) and RMSNorm at config 2's shape, the prefill scatter of
        8192 rows into a shuffled 512-page table, and the decode scatter of 256 sequences
        (lengths uniform in [1, 2048], pages shuffled over the batch's pool)."""
        wl, llmk, np, torch = self.wl, self.llmk, self.np, self.torch
        rows, H = 8192, wl.HIDDEN
        n = rows * H
        R = sets_for(3 * n * 2)
        sets = [wl.add_rmsnorm_inputs(rows, H, seed=wl.SEED_BASE + 60 + 100 * i)
                for i in range(R)]
        self.cpu_inputs["residual_add_8192x2048"] = {
            k: sets[0][k].cpu().numpy().view(np.uint16).copy() for k in ("residual", "x", "w")}
        self.cpu_inputs["rmsnorm_8192x2048"] = self.cpu_inputs["residual_add_8192x2048"]
        self.mark("residual_add")
        t = self.run(lambda i: llmk.residual_add(sets[i]["residual"], sets[i]["x"],
                                                 sets[i]["residual"], n), R)
        self.kernels["residual_add_8192x2048"] = kernel_entry(
            "residual_add [8192,2048] in place", wl.bytes_residual_add(n), t,
            self.traffic.get("residual_add_8192x2048"), {"sets": R})
        self.mark("rmsnorm_8192")
        t = self.run(lambda i: llmk.rmsnorm(sets[i]["x"], sets[i]["w"], sets[i]["out"], rows, H,
                                            wl.EPS), R)
        self.kernels["rmsnorm_8192x2048"] = kernel_entry(
            "rmsnorm [8192,2048]", wl.bytes_rmsnorm(rows, H), t,
            self.traffic.get("rmsnorm_8192x2048"), {"sets": R})
        del sets
        self.free()

        kvdim, ps = wl.N_KV * wl.HEAD_DIM, wl.PAGE
        T, pages = 8192, 8192 // wl.PAGE
        nb = wl.bytes_kv_scatter(T, kvdim, ps)
        R = sets_for(nb)
        rng = np.random.default_rng(wl.SEED_BASE + 70)
        g = torch.Generator(device=self.dev).manual_seed(wl.SEED_BASE + 71)
        sc = []
        for _ in range(R):
            sc.append(dict(src=wl.normal_f16((T, kvdim), g, self.dev),
                           pool=wl.poisoned(pages * ps * kvdim, self.dev),
                           table=torch.from_numpy(rng.permutation(pages).astype(np.int32))
                           .to(self.dev)))
        self.cpu_inputs["kv_scatter_8192"] = {
            "src": sc[0]["src"].cpu().numpy().view(np.uint16).copy(),
            "table": sc[0]["table"].cpu().numpy().copy(), "pages": pages}
        self.mark("kv_scatter_8192")
        t = self.run(lambda i: llmk.kv_scatter(sc[i]["src"], sc[i]["pool"], sc[i]["table"], 0, T,
                                               ps, kvdim), R)
        self.kernels["kv_scatter_8192"] = kernel_entry(
            "kv_scatter 8192 rows (prefill)", nb, t, self.traffic.get("kv_scatter_8192"),
            {"sets": R, "pages": pages})
        del sc
        self.free()

        n, max_pages = 256, 128
        lens = rng.integers(1, max_pages * ps + 1, n)
        npages = (lens + ps - 1) // ps
        total = int(npages.sum())
        perm = rng.permutation(total).astype(np.int32)
        tables = np.zeros((n, max_pages), np.int32)
        off = 0
        for b, pb in enumerate(npages):
            tables[b, :pb] = perm[off:off + pb]
            off += pb
        pool = wl.poisoned(total * ps * kvdim, self.dev)
        dtab = torch.from_numpy(tables).to(self.dev)
        dpos = torch.from_numpy((lens - 1).astype(np.int32)).to(self.dev)
        R = 16
        srcs = [wl.normal_f16((n, kvdim), g, self.dev) for _ in range(R)]
        self.cpu_inputs["kv_scatter_batch_256"] = {
            "src": srcs[0].cpu().numpy().view(np.uint16).copy(), "tables": tables,
            "pos": (lens - 1).astype(np.int32), "total": total}
        self.mark("kv_scatter_batch_256")
        t = self.run(lambda i: llmk.kv_scatter_batch(srcs[i], pool, dtab, dpos, n, max_pages, ps,
                                                     kvdim), R)
        self.kernels["kv_scatter_batch_256"] = kernel_entry(
            "kv_scatter_batch 256 sequences", wl.bytes_kv_scatter_batch(n, kvdim), t,
            self.traffic.get("kv_scatter_batch_256"),
            {"sets": R, "note": "one launch, 0.5 MB: bound by the launch, not the bytes"})
        del srcs, pool
        self.free()

    def config5_two_norms(self, table=None):
        """Config 5 with both of the real layer's add + RMSNorm pairs per layer (the second one
        between the RoPE + K/V scatter and the SwiGLU): 65 launches op by op, or 16 with one
        launch per layer; two input sets replayed alternately from HIP graphs."""
        wl, llmk, torch = self.wl, self.llmk, self.torch
        if table is None:
            table = wl.embedding_table(seed=wl.SEED_BASE + 40)
        L, n = wl.LAYERS, 256
        ps = [wl.decode_pass_inputs(self.inv, table=table, seed=wl.SEED_BASE + 62 + 100 * i,
                                    two_norms=True) for i in range(2)]
        dps = [llmk.DecodeNonGemmPass(p.table, p.token_ids, p.residual, p.block_tables,
                                      p.positions, p.inv_freq, p.per_layer, n_heads=wl.N_HEADS,
                                      n_kv_heads=wl.N_KV, head_dim=wl.HEAD_DIM, inter=wl.INTER,
                                      page_size=wl.PAGE, max_pages=p.max_pages, eps=wl.EPS)
               for p in ps]

        def capture(fn):
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                fn()
            torch.cuda.current_stream().wait_stream(s)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                fn()
            return g

        steps, warm = max(20, self.K // 4), max(5, self.W // 4)
        nb = wl.bytes_decode_pass(n, L, two_norms=True)
        graphs = [capture(dp.run) for dp in dps]
        self.mark("pass2_graph")
        t = self.run(lambda i: graphs[i].replay(), 2, steps, warm)
        self.kernels["decode_pass_16x256_two_norms"] = kernel_entry(
            "decode pass, both norms per layer (graph)", nb, t, None,
            {"launches": 1 + 4 * L, "layers": L, "seqs": n, "sets": 2,
             "note": "the real layer's two add + RMSNorm pairs per layer (config 5 lists one); "
                     "388 MB per pass"})
        del graphs
        lgraphs = [capture(dp.run_layers) for dp in dps]
        self.mark("pass2_layers")
        t = self.run(lambda i: lgraphs[i].replay(), 2, steps, warm)
        self.kernels["decode_pass_16x256_two_norms_layers"] = kernel_entry(
            "decode pass, both norms, one launch per layer", nb, t, None,
            {"launches": L, "layers": L, "seqs": n, "sets": 2})
        del lgraphs
        fgraphs = [capture(dp.run_fused) for dp in dps]
        self.mark("pass2_fused")
        t = self.run(lambda i: fgraphs[i].replay(), 2, steps, warm)
        moved = wl.bytes_decode_pass_fused(n, L, two_norms=True)
        self.kernels["decode_pass_16x256_two_norms_fused"] = kernel_entry(
            "decode pass, both norms, one launch", nb, t, None,
            {"launches": 1, "layers": L, "seqs": n, "sets": 2, "moved_bytes": moved,
             "moved_frac_of_peak": round(moved / t["mean_s"] / 1e9 / PEAK_GBS, 4)})
        del fgraphs
        # a single kernel needs no graph: launched directly, it skips the graph launch's own cost
        self.mark("pass2_fused_eager")
        t = self.run(lambda i: dps[i].run_fused(), 2, steps, warm)
        self.kernels["decode_pass_16x256_two_norms_fused_eager"] = kernel_entry(
            "decode pass, both norms, one launch (direct)", nb, t, None,
            {"launches": 1, "layers": L, "seqs": n, "sets": 2, "moved_bytes": moved,
             "moved_frac_of_peak": round(moved / t["mean_s"] / 1e9 / PEAK_GBS, 4)})
        del dps, ps
        self.free()

    # ------------------------------------------------------------------ config 5
    def config5(self, table=None):
        """The 16-layer non-GEMM decode pass over 256 sequences: two input sets (642 MB between
        reuses, past the 256 MB MALL), each captured in a HIP graph and replayed alternately;
        the same eagerly; then the breakdown: one graph per op type (the op's 16 launches of a
        pass, the embedding's one) and graphs of empty kernels in the same launch shapes (the
        launch floor), alternating between the two input sets likewise."""
        wl, llmk, torch = self.wl, self.llmk, self.torch
        if table is None:
            table = wl.embedding_table(seed=wl.SEED_BASE + 40)
        L, n = wl.LAYERS, 256
        ps = [wl.decode_pass_inputs(self.inv, table=table, seed=wl.SEED_BASE + 5 + 100 * i)
              for i in range(2)]
        dps = [llmk.DecodeNonGemmPass(p.table, p.token_ids, p.residual, p.block_tables,
                                      p.positions, p.inv_freq, p.per_layer, n_heads=wl.N_HEADS,
                                      n_kv_heads=wl.N_KV, head_dim=wl.HEAD_DIM, inter=wl.INTER,
                                      page_size=wl.PAGE, max_pages=p.max_pages, eps=wl.EPS)
               for p in ps]
        if not self.args.no_cpu:
            self.cpu_inputs["decode_pass_16x256"] = cpu_pass_inputs(ps[0], wl)

        def capture(fn):
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                fn()
            torch.cuda.current_stream().wait_stream(s)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                fn()
            return g

        graphs = [capture(dp.run) for dp in dps]
        steps, warm = max(20, self.K // 4), max(5, self.W // 4)
        nb = wl.bytes_decode_pass(n, L)
        self.mark("pass_graph")
        t = self.run(lambda i: graphs[i].replay(), 2, steps, warm)
        entry = kernel_entry("decode pass 16 layers x 256 (graph)", nb, t, None,
                             {"launches": 1 + 3 * L, "layers": L, "seqs": n, "sets": 2,
                              "note": "two input sets of 321 MB touched per pass, alternating "
                                      "(> 256 MB MALL between reuses); one HIP graph of 49 "
                                      "kernels per set"})
        self.kernels["decode_pass_16x256"] = entry
        self.mark("pass_eager")
        t = self.run(lambda i: dps[i].run(), 2, steps, warm)
        self.kernels["decode_pass_16x256_eager"] = kernel_entry(
            "decode pass 16 layers x 256 (eager)", nb, t, None, {"sets": 2})
        # the same pass with one launch per layer (llmk_decode_nongemm_pass_layers), possible
        # because the pass's per-layer inputs are independent; graphs of its 16 launches
        lgraphs = [capture(dp.run_layers) for dp in dps]
        self.mark("pass_layers")
        t = self.run(lambda i: lgraphs[i].replay(), 2, steps, warm)
        self.kernels["decode_pass_16x256_layers"] = kernel_entry(
            "decode pass, one launch per layer (graph)", nb, t, None,
            {"launches": L, "layers": L, "seqs": n, "sets": 2,
             "note": "each layer's add+RMSNorm rows, RoPE + K/V scatter tokens and SwiGLU "
                     "chunks as blocks of one launch, the embedding gather fused into the first "
                     "residual add (bytes counted as for the 49-launch pass, which also writes "
                     "and re-reads the 1 MB of embedding rows); valid for this pass, whose "
                     "per-layer inputs are independent, not for a decode step with GEMMs "
                     "between the ops"})
        del lgraphs
        self.mark("pass_layers_eager")
        t = self.run(lambda i: dps[i].run_layers(), 2, steps, warm)
        self.kernels["decode_pass_16x256_layers_eager"] = kernel_entry(
            "decode pass, one launch per layer (direct)", nb, t, None,
            {"launches": L, "layers": L, "seqs": n, "sets": 2})
        # the whole pass in one launch (llmk_decode_nongemm_pass_fused): the residual chains of
        # all 16 layers beside every layer's RoPE + scatter tokens and SwiGLU chunks
        fgraphs = [capture(dp.run_fused) for dp in dps]
        self.mark("pass_fused")
        t = self.run(lambda i: fgraphs[i].replay(), 2, steps, warm)
        moved = wl.bytes_decode_pass_fused(n, L)
        self.kernels["decode_pass_16x256_fused"] = kernel_entry(
            "decode pass, one launch (graph)", nb, t, None,
            {"launches": 1, "layers": L, "seqs": n, "sets": 2, "moved_bytes": moved,
             "moved_frac_of_peak": round(moved / t["mean_s"] / 1e9 / PEAK_GBS, 4),
             "note": "one wave per sequence carries the residual through all 16 layers' add + "
                     "RMSNorm (stored after every layer, never re-read) while the other blocks "
                     "run every layer's RoPE + K/V scatter and SwiGLU; `bytes` is config 5's "
                     "count, `moved_bytes` what this launch must move (no embedding rows "
                     "written and re-read, no residual re-read per layer)"})
        del fgraphs
        # the same launch made directly, back to back: a graph of one kernel adds the graph
        # launch's own cost to every pass and saves nothing
        self.mark("pass_fused_eager")
        t = self.run(lambda i: dps[i].run_fused(), 2, steps, warm)
        self.kernels["decode_pass_16x256_fused_eager"] = kernel_entry(
            "decode pass, one launch (direct)", nb, t, None,
            {"launches": 1, "layers": L, "seqs": n, "sets": 2, "moved_bytes": moved,
             "moved_frac_of_peak": round(moved / t["mean_s"] / 1e9 / PEAK_GBS, 4)})

        # ---- breakdown
        def stage_fn(op, p):
            def f():
                if op == "embedding":
                    llmk.embedding_lookup(p.table, p.token_ids, p.residual, n, wl.HIDDEN)
                for lay in (p.per_layer if op != "embedding" else ()):
                    if op == "add_rmsnorm":
                        llmk.add_rmsnorm(p.residual, lay["x"], lay["norm_w"], lay["normed"], n,
                                         wl.HIDDEN, wl.EPS)
                    elif op == "rope_kv_scatter":
                        llmk.rope_kv_scatter_batch(lay["q"], lay["k"], lay["v"], lay["k_pool"],
                                                   lay["v_pool"], p.block_tables, p.positions,
                                                   p.inv_freq, n, p.max_pages, wl.PAGE,
                                                   wl.N_HEADS, wl.N_KV, wl.HEAD_DIM)
                    elif op == "swiglu":
                        llmk.swiglu(lay["gate"], lay["up"], lay["act"], n * wl.INTER)
            return f

        def empty_fn(shapes):
            def f():
                for blocks, threads in shapes:
                    llmk.empty_launch(blocks, threads)
            return f

        pass_shapes = [PASS_SHAPES["embedding"]] + [
            PASS_SHAPES[op] for _ in range(L) for op in ("add_rmsnorm", "rope_kv_scatter",
                                                         "swiglu")]
        g_floor = capture(empty_fn(pass_shapes))
        self.mark("pass_floor")
        t_floor = self.run(lambda i: g_floor.replay(), 1, steps, warm)
        bd = {"pass_us": entry["us_mean"], "launch_floor_49_us": round(t_floor["mean_s"] * 1e6, 3)}
        log(f"    launch floor, 49 empty kernels in the pass's shapes: {bd['launch_floor_49_us']:.2f} us")
        stages = {}
        for op in ("embedding", "add_rmsnorm", "rope_kv_scatter", "swiglu"):
            cnt = 1 if op == "embedding" else L
            gs = [capture(stage_fn(op, p)) for p in ps]
            self.mark(f"pass_stage_{op}")
            t_op = self.run(lambda i: gs[i].replay(), 2, steps, warm)
            ge = capture(empty_fn([PASS_SHAPES[op]] * cnt))
            self.mark("pass_floor_stages")
            t_e = self.run(lambda i: ge.replay(), 1, steps, warm)
            us, us_e = t_op["mean_s"] * 1e6, t_e["mean_s"] * 1e6
            stages[op] = {"launches": cnt, "us": round(us, 3), "us_per_launch": round(us / cnt, 3),
                          "floor_us": round(us_e, 3), "floor_us_per_launch": round(us_e / cnt, 3),
                          "work_us_per_launch": round((us - us_e) / cnt, 3)}
            log(f"    stage {op:16s} {cnt:2d} launches {us:8.2f} us ({us / cnt:5.2f} per launch; "
                f"empty kernels of the same shapes {us_e / cnt:5.2f})")
            del gs, ge
        bd["stages"] = stages
        bd["sum_of_stages_us"] = round(sum(s["us"] for s in stages.values()), 3)
        bd["pass_minus_floor_us"] = round(bd["pass_us"] - bd["launch_floor_49_us"], 3)
        # A graph launch costs more than a launch inside a graph: from the 1- and 49-kernel
        # empty graphs, per launch = (floor_49 - floor_1) / 48, per graph = floor_1 - that. The
        # four stage graphs pay three graph launches more than the one pass graph.
        per_launch = (bd["launch_floor_49_us"] - stages["embedding"]["floor_us"]) / 48
        per_graph = stages["embedding"]["floor_us"] - per_launch
        bd["launch_us_in_graph"] = round(per_launch, 3)
        bd["graph_launch_us"] = round(per_graph, 3)
        bd["sum_of_stages_less_extra_graph_launches_us"] = round(
            bd["sum_of_stages_us"] - 3 * per_graph, 3)
        log(f"    sum of stages {bd['sum_of_stages_us']:.2f} us, less 3 extra graph launches of "
            f"{per_graph:.2f} us: {bd['sum_of_stages_less_extra_graph_launches_us']:.2f} us; pass "
            f"{bd['pass_us']:.2f} us = launch floor {bd['launch_floor_49_us']:.2f} "
            f"({per_launch:.2f} us per launch) + work {bd['pass_minus_floor_us']:.2f}")
        entry["breakdown"] = bd
        del graphs, g_floor, dps, ps
        self.free()

    # ------------------------------------------------------------------ attention
    def attention(self):
        wl, llmk, np, torch = self.wl, self.llmk, self.np, self.torch
        lens = wl.attention_lens()
        if wl.bytes_attention(lens) != ATTN_BYTES_256:
            raise RuntimeError(f"attention workload bytes {wl.bytes_attention(lens)} != "
                               f"{ATTN_BYTES_256}")

        def one(label, lens_b, R, section, quiet=False):
            splits = llmk.choose_num_splits(lens_b.size, wl.N_KV, int(lens_b.max()))
            sets6 = [wl.attention_inputs(lens_b, num_splits=splits,
                                         seed=wl.SEED_BASE + 6 + 100 * i) for i in range(R)]

            def launch_attn(i):
                a = sets6[i]
                llmk.attention_decode_fast(a["q"], a["k_pool"], a["v_pool"], a["block_tables"],
                                           a["seq_lens"], a["out"], a["workspace"], a["n"],
                                           a["max_pages"], wl.PAGE, wl.N_HEADS, wl.N_KV,
                                           wl.HEAD_DIM, splits)

            self.mark(section)
            t = self.run(launch_attn, R)
            e = kernel_entry(f"attention {label}", wl.bytes_attention(lens_b), t,
                             self.traffic.get(f"attention_decode_{label}"),
                             {"sets": R, "num_splits": splits, "seqs": int(lens_b.size),
                              "context_tokens": int(lens_b.sum()), "launches": 2})
            del sets6
            self.free()
            return e

        self.kernels["attention_decode_256"] = one("256", lens, 2, "attention_256")
        self.kernels["attention_decode_16x2048"] = one("16x2048", np.full(16, 2048), 17,
                                                       "attention_16x2048")
        # batch sweep at a full 2048-position context, batch 1 = the latency of one sequence
        # (ref: docs/attention_decode_batch_sweep.md:50-60, bench/bench_attention_compare.cu)
        sweep = {}
        for b in (1, 2, 4, 8, 16, 64, 256):
            lb = np.full(b, 2048)
            per_set = wl.bytes_attention(lb)
            sweep[str(b)] = one(f"{b}x2048", lb, sets_for(per_set, most=256), "attention_sweep")
        self.kernels["attention_decode_sweep_2048"] = sweep

    def argmax(self):
        wl, llmk, torch = self.wl, self.llmk, self.torch
        R7, n7 = 17, 256
        g7 = torch.Generator(device=self.dev)
        g7.manual_seed(wl.SEED_BASE + 7)
        logits = [torch.randn((n7, wl.VOCAB), generator=g7, device=self.dev).half()
                  for _ in range(R7)]
        am_out = torch.empty(n7, dtype=torch.int32, device=self.dev)
        self.mark("argmax")
        t = self.run(lambda i: llmk.argmax_rows(logits[i], am_out, n7, wl.VOCAB), R7)
        self.kernels["argmax_256x128256"] = kernel_entry(
            "argmax_rows [256,128256]", wl.bytes_argmax(n7, wl.VOCAB), t,
            self.traffic.get("argmax_256x128256"), {"sets": R7})
        del logits
        self.free()

    # ------------------------------------------------------------------ bandwidth ceilings
    PROBE_NAMES = ("read", "copy", "read2", "inplace", "write")
    PROBE_TRAFFIC = (1, 2, 3, 2, 1)  # bytes moved per byte of the probe's unit buffer

    def probes(self):
        """Sweep of every probe over grid and unroll at a 1 GiB unit buffer (two sets of
        buffers, alternating), then each kernel's own mix at its own byte count."""
        llmk, torch = self.llmk, self.torch
        nb = 1 << 30
        bufs = [[torch.empty(nb, dtype=torch.uint8, device=self.dev) for _ in range(3)]
                for _ in range(2)]
        for s in bufs:
            for t in s:
                t.random_(0, 256)
        sweep = {}
        self.mark("probe_sweep")
        for mode, name in enumerate(self.PROBE_NAMES):
            res = []
            for blocks in (0, 1024, 2048, 4096, 8192):
                for unroll in (1, 2, 4, 8):
                    def launch(i, mode=mode, blocks=blocks, unroll=unroll):
                        a, b, d = bufs[i]
                        llmk.bw_probe(mode, d if mode != 0 else a, nb, a=a, b=b, blocks=blocks,
                                      unroll=unroll)
                    t = self.timer.run(launch, 2, 10, 3, warm_s=0.02)
                    gbs = self.PROBE_TRAFFIC[mode] * nb / t["mean_s"] / 1e9
                    res.append({"blocks": blocks, "unroll": unroll, "GBps": round(gbs, 1)})
            best = max(res, key=lambda r: r["GBps"])
            sweep[name] = {"best": best, "one_pass_unroll4": next(
                r for r in res if r["blocks"] == 0 and r["unroll"] == 4)}
            log(f"  probe {name:8s} best {best['GBps']:7.1f} GB/s ({100 * best['GBps'] / PEAK_GBS:4.1f}%)"
                f" at blocks {best['blocks']} unroll {best['unroll']}; GB/s by blocks (0 = one "
                f"pass) x unroll 1/2/4/8: " + "; ".join(
                    f"{bl}: " + "/".join(f"{r['GBps']:.0f}" for r in res if r["blocks"] == bl)
                    for bl in (0, 1024, 2048, 4096, 8192)))
        del bufs
        self.free()
        self.kernels["probe_sweep_1GiB"] = sweep
        return sweep

    def kernel_ceilings(self, sweep):
        """Each kernel's traffic mix at its own byte count and rotation, with the best sweep
        setting of that mix and with one pass of unroll 4 (the kernels' launch style); the
        faster is the kernel's ceiling."""
        llmk, torch, wl = self.llmk, self.torch, self.wl
        # (kernel label, probe mode, bytes of the unit buffer, sets)
        mixes = [("add_rmsnorm_8192x2048", 1, 134221824 // 2, 12),
                 ("rope_8192", 3, 83918976 // 2, 27),
                 ("swiglu_8192x8192", 2, 402653184 // 3, 4),
                 ("embedding_8192", 1, 67141632 // 2, 16),
                 ("argmax_256x128256", 0, wl.bytes_argmax(256, wl.VOCAB), 17),
                 ("attention_decode_256", 0, ATTN_BYTES_256, 2)]
        self.mark("probe_kernels")
        out = {}
        for label, mode, unit, R in mixes:
            if label not in self.kernels:
                continue
            unit -= unit % 16
            bufs = [[torch.empty(unit, dtype=torch.uint8, device=self.dev)
                     for _ in range(3 if mode == 2 else (1 if mode in (0, 3) else 2))]
                    for _ in range(R)]
            name = self.PROBE_NAMES[mode]
            best = sweep[name]["best"]
            res = []
            for blocks, unroll in ((best["blocks"], best["unroll"]), (0, 4)):
                def launch(i, mode=mode, blocks=blocks, unroll=unroll):
                    s = bufs[i]
                    if mode == 0:
                        llmk.bw_probe(0, s[0], unit, a=s[0], blocks=blocks, unroll=unroll)
                    elif mode == 3:
                        llmk.bw_probe(3, s[0], unit, blocks=blocks, unroll=unroll)
                    elif mode == 1:
                        llmk.bw_probe(1, s[1], unit, a=s[0], blocks=blocks, unroll=unroll)
                    else:
                        llmk.bw_probe(2, s[2], unit, a=s[0], b=s[1], blocks=blocks,
                                      unroll=unroll)
                t = self.run(launch, R)
                res.append((self.PROBE_TRAFFIC[mode] * unit / t["mean_s"] / 1e9, blocks, unroll,
                            t["mean_s"] * 1e6))
            gbs, blocks, unroll, us = max(res)
            k = self.kernels[label]
            c = {"mix": name, "GBps": round(gbs, 1), "us": round(us, 3), "blocks": blocks,
                 "unroll": unroll, "frac_of_peak": round(gbs / PEAK_GBS, 4),
                 "kernel_frac_of_ceiling": round(k["GBps"] / gbs, 4)}
            k["ceiling"] = c
            out[label] = c
            log(f"  ceiling {label:24s} {name:8s} {gbs:7.1f} GB/s ({100 * gbs / PEAK_GBS:4.1f}%);"
                f" kernel at {100 * k['GBps'] / gbs:5.1f}% of it")
            del bufs
            self.free()
        return out

    def calibration(self):
        """Probes whose counters scale each launch shape's FETCH_SIZE / WRITE_SIZE: a copy probe
        swept over CALIB_SWEEP_SIZES with the buffers cache-resident and with every launch on
        fresh HBM, and one probe per CALIB_PROBES entry (the shape's mix, bytes and rotation).
        A few launches each: only their counters are used."""
        llmk, torch = self.llmk, self.torch
        big = 1 << 30
        src = torch.empty(big, dtype=torch.uint8, device=self.dev)
        dst = torch.empty(big, dtype=torch.uint8, device=self.dev)
        src.random_(0, 256)
        for sec, resident in (("calib_resident", True), ("calib_hbm", False)):
            self.mark(sec)
            for size in CALIB_SWEEP_SIZES:
                slots = 4 if resident else big // size
                for i in range(24):
                    o = (i % slots) * size
                    llmk.bw_probe(1, dst[o:o + size], size, a=src[o:o + size], blocks=0,
                                  unroll=CALIB_UNROLL)
                torch.cuda.synchronize()
        del src, dst
        self.free()
        self.mark("calib")
        for label, mode, unit, R in CALIB_PROBES:
            unit -= unit % 16
            n_in = 2 if mode == 2 else (0 if mode in (3, 4) else 1)
            bufs = [[torch.empty(unit, dtype=torch.uint8, device=self.dev)
                     for _ in range(n_in + (1 if mode != 0 else 0))] for _ in range(R)]
            for st in bufs:
                for t in st:
                    t.random_(0, 256)
            for i in range(3 + 20):
                st = bufs[i % R]
                if mode == 0:
                    llmk.bw_probe(0, st[0], unit, a=st[0], unroll=CALIB_UNROLL)
                elif mode == 1:
                    llmk.bw_probe(1, st[1], unit, a=st[0], unroll=CALIB_UNROLL)
                elif mode == 2:
                    llmk.bw_probe(2, st[2], unit, a=st[0], b=st[1], unroll=CALIB_UNROLL)
                else:
                    llmk.bw_probe(mode, st[0], unit, unroll=CALIB_UNROLL)
            torch.cuda.synchronize()
            del bufs
            self.free()

    def copy_probe(self):
        llmk, torch = self.llmk, self.torch
        nb = 1 << 30
        bufs = [torch.empty(nb, dtype=torch.uint8, device=self.dev) for _ in range(4)]
        self.mark("copy_1GiB")
        t = self.run(lambda i: llmk.copy_bytes(bufs[2 * (i % 2)], bufs[2 * (i % 2) + 1], nb), 2,
                     max(20, self.K // 4), 5)
        self.kernels["copy_1GiB"] = kernel_entry("copy probe 1 GiB", 2 * nb, t,
                                                 self.traffic.get("copy_1GiB"))
        del bufs
        self.free()

    # ------------------------------------------------------------------ CPU baselines
    def cpu_baselines(self, seconds):
        """The scalar C oracle (oracle/, test infrastructure) of each configuration's work on
        host copies of the configuration's first input set: all cores of the process's CPU
        affinity (rows split over threads, identical results), then one core. Outputs are
        preallocated and in-place operands keep being updated, so no copy or first-touch page
        fault is inside the timed loops."""
        import numpy as np
        sys.path.insert(0, ROOT)
        import oracle
        lib = oracle.lib()
        wl = self.wl
        u16 = ctypes.POINTER(ctypes.c_uint16)
        i32 = ctypes.POINTER(ctypes.c_int32)
        f32 = ctypes.POINTER(ctypes.c_float)

        def P(a, t=u16):
            return a.ctypes.data_as(t)

        threads = len(os.sched_getaffinity(0))
        info = {"cpu_model": cpu_model(), "os_cpu_count": os.cpu_count(),
                "affinity_cores": threads, "threads_used": threads}

        def timed(fn, budget, first=True):
            if first:
                fn()  # first call outside the timed loop (touches the output pages)
            reps, t0 = 0, time.perf_counter()
            while True:
                fn()
                reps += 1
                el = time.perf_counter() - t0
                if el >= budget:
                    return reps, el

        def figure(label, nbytes, make, sample):
            if label not in self.cpu_inputs:
                return
            fn_all, fn_one = make(threads), make(1)
            reps, el = timed(fn_all, seconds * 0.7)
            reps1, el1 = timed(fn_one, seconds * 0.3, first=False)
            v, v1 = nbytes * reps / el / 1e9, nbytes * reps1 / el1 / 1e9
            c = {"value": round(v, 3), "unit": "GB/s", "us": round(el / reps * 1e6, 1),
                 "cores": threads, "kind": "port",
                 "sample": f"{reps} {sample} in {el:.1f} s, the scalar C oracle over {threads} "
                           f"threads", "one_core": {"value": round(v1, 3), "unit": "GB/s",
                                                    "us": round(el1 / reps1 * 1e6, 1),
                                                    "cores": 1,
                                                    "sample": f"{reps1} in {el1:.1f} s"}}
            if label in self.kernels:
                self.kernels[label]["cpu"] = c
                c["gpu_over_cpu"] = round(self.kernels[label]["GBps"] / max(v, 1e-9), 1)
            log(f"  CPU oracle {label:26s} {v:7.3f} GB/s on {threads} threads, {v1:7.3f} on 1 "
                f"({el / reps * 1e6:.0f} us per call)")
            return c

        out = {}
        eps, H = wl.EPS, wl.HIDDEN
        d = self.cpu_inputs.get("add_rmsnorm_8192x2048")
        if d:
            o = np.empty_like(d["x"])

            def mk2(th):
                return lambda: lib.or_add_rmsnorm_mt(P(d["residual"]), P(d["x"]), P(d["w"]), P(o),
                                                     8192, H, eps, th)
            out["add_rmsnorm_8192x2048"] = figure("add_rmsnorm_8192x2048",
                                                  wl.bytes_add_rmsnorm(8192, H), mk2,
                                                  "full [8192,2048] add_rmsnorm passes")
        d = self.cpu_inputs.get("rmsnorm_16x2048")
        if d:
            o = np.empty_like(d["x"])

            def mk1(th):  # 16 rows: one thread per row at most; the scalar function on one core
                return lambda: lib.or_rmsnorm(P(d["x"]), P(d["w"]), P(o), 16, H, eps)
            c = figure("rmsnorm_16x2048", wl.bytes_rmsnorm(16, H), mk1, "[16,2048] rmsnorm calls")
            if c:
                c["cores"] = 1
                c["sample"] += " (single-threaded: 16 rows)"
            out["rmsnorm_16x2048"] = c
        d = self.cpu_inputs.get("rope_8192")
        if d:
            def mk3(th):
                return lambda: lib.or_rope_apply_mt(P(d["q"]), P(d["k"]), P(d["positions"], i32),
                                                    P(d["inv"], f32), 8192, wl.N_HEADS, wl.N_KV,
                                                    wl.HEAD_DIM, th)
            out["rope_8192"] = figure("rope_8192", wl.bytes_rope(8192, wl.N_HEADS, wl.N_KV,
                                                                 wl.HEAD_DIM), mk3,
                                      "in-place RoPE passes over Q [8192,32,64] + K [8192,8,64]")
        d = self.cpu_inputs.get("swiglu_8192x8192")
        if d:
            o = np.empty_like(d["gate"])

            def mk4(th):
                return lambda: lib.or_swiglu_mt(P(d["gate"]), P(d["up"]), P(o), d["gate"].size, th)
            out["swiglu_8192x8192"] = figure("swiglu_8192x8192", wl.bytes_swiglu(d["gate"].size),
                                             mk4, "[8192,8192] SwiGLU passes")
        d = self.cpu_inputs.get("embedding_8192")
        if d:
            o = np.empty((8192, H), np.uint16)

            def mk5(th):
                it = [0]

                def f():
                    ids = d["ids"][it[0] % len(d["ids"])]
                    it[0] += 1
                    lib.or_embedding_lookup_mt(P(d["table"]), P(ids, i32), P(o), 8192, H, th)
                return f
            out["embedding_8192"] = figure("embedding_8192", wl.bytes_embedding(8192, H), mk5,
                                           f"gathers of 8192 rows from [128256,2048] (cycling "
                                           f"through {len(d['ids'])} id sets)")
        d = self.cpu_inputs.get("residual_add_8192x2048")
        if d:
            r = d["residual"].copy()

            def mk6(th):  # in place, as the GPU runs it
                return lambda: lib.or_residual_add_mt(P(r), P(d["x"]), P(r), r.size, th)
            out["residual_add_8192x2048"] = figure(
                "residual_add_8192x2048", wl.bytes_residual_add(r.size), mk6,
                "in-place [8192,2048] residual adds")
            o = np.empty_like(d["x"])

            def mk7(th):
                return lambda: lib.or_rmsnorm_mt(P(d["x"]), P(d["w"]), P(o), 8192, H, eps, th)
            out["rmsnorm_8192x2048"] = figure("rmsnorm_8192x2048", wl.bytes_rmsnorm(8192, H), mk7,
                                              "[8192,2048] RMSNorm passes")
        d = self.cpu_inputs.get("kv_scatter_8192")
        if d:
            kvdim = wl.N_KV * wl.HEAD_DIM
            pool = np.full(d["pages"] * wl.PAGE * kvdim, 0x7F7F, np.uint16)

            def mk8(th):
                return lambda: lib.or_kv_scatter_mt(P(d["src"]), P(pool), P(d["table"], i32), 0,
                                                    8192, wl.PAGE, kvdim, th)
            out["kv_scatter_8192"] = figure("kv_scatter_8192",
                                            wl.bytes_kv_scatter(8192, kvdim, wl.PAGE), mk8,
                                            "prefill scatters of 8192 rows")
        d = self.cpu_inputs.get("kv_scatter_batch_256")
        if d:
            kvdim = wl.N_KV * wl.HEAD_DIM
            pool = np.full(d["total"] * wl.PAGE * kvdim, 0x7F7F, np.uint16)

            def mk9(th):  # 256 rows: the scalar function, one core
                return lambda: lib.or_kv_scatter_batch(P(d["src"]), P(pool), P(d["tables"], i32),
                                                       P(d["pos"], i32), 256, 128, wl.PAGE, kvdim)
            c = figure("kv_scatter_batch_256", wl.bytes_kv_scatter_batch(256, kvdim), mk9,
                       "decode scatters of 256 rows")
            if c:
                c["cores"] = 1
                c["sample"] += " (single-threaded: 256 rows)"
            out["kv_scatter_batch_256"] = c
        h = self.cpu_inputs.get("decode_pass_16x256")
        if h is not None:
            out["decode_pass_16x256"] = figure(
                "decode_pass_16x256", wl.bytes_decode_pass(h["n"], len(h["layers"])),
                cpu_decode_pass(h, lib, wl, P, i32, f32),
                "16-layer passes over 256 sequences (embedding; add+RMSNorm, RoPE + K/V "
                "scatter, SwiGLU per layer; each sequence's pool page remapped into a 256-page "
                "host pool, the same rows moved)")
        out["info"] = info
        self.cpu_info = info
        return out

    # ------------------------------------------------------------------ the engine
    def decode_step(self, n_seqs=256):
        wl, llmk, torch, np = self.wl, self.llmk, self.torch, self.np
        # The engine's set-up passes (GEMM plan timing, the eager pass, the capture) below are
        # not the step: a section of their own keeps them out of the previous section's trace.
        self.mark("setup")
        import importlib
        weights = importlib.import_module("llmk.weights")
        cfg = llmk.ModelConfig()
        lens = wl.attention_lens(n_seqs)
        tokens, pos, tables, used = wl.decode_step_rows(lens)
        n = lens.size
        eng = llmk.Engine(cfg, max_rows=n, max_pages=128, num_pages=used)
        w = weights.random_weights(cfg, wl.SEED_BASE + 9, device=self.dev)
        eng.set_weights(*weights.engine_layers(w, cfg))
        del w
        g = torch.Generator(device=self.dev)
        g.manual_seed(wl.SEED_BASE + 10)
        fill = torch.randn(used * wl.PAGE * wl.N_KV * wl.HEAD_DIM, generator=g,
                           device=self.dev).half()
        for l in range(cfg.n_layers):
            for which in (llmk.BUF_K_POOL, llmk.BUF_V_POOL):
                eng.write_pool(which, l, fill)
        del fill
        self.free()
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
        self.mark("step_256" if n_seqs == 256 else "step_8")
        t = self.run(lambda i: graph.replay(), 1, max(20, self.K // 4), max(5, self.W // 4))
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
        self.free()
        self.kernels[f"decode_step_1b_{n}"] = e
        if n > llmk.LINEAR_ROWS_MAX:  # the projections are hipBLASLt calls: time a C++ caller too
            c = self.decode_step_cpp(cfg, tokens, pos, tables, used, 128, nbytes,
                                     max(20, self.K // 4), max(5, self.W // 4))
            if c:
                self.kernels[f"decode_step_1b_{n}_cpp"] = c

    def decode_step_cpp(self, cfg, tokens, pos, tables, used, max_pages, nbytes, steps, warm):
        """The same step timed by llmk_step_bench, a C++ process linking the library: there
        libllmk's hipBLASLt and HIP runtime are the system's, as for any C/C++ caller, while in
        this process they are the copies torch loaded. Same config and rows (written to a file
        for it), weights and pools of the same distributions; graph launches timed back to back
        with HIP events."""
        import subprocess
        import tempfile
        np = self.np
        exe = os.path.join(ROOT, "cuda-llm-engine_amd", "llmk_step_bench")
        if not os.path.exists(exe):
            log("  decode step from C++: llmk_step_bench is not built; skipped")
            return None
        if os.environ.get("ROCPROF_OUTPUT_PATH"):  # set by rocprofv3 for the program it traces
            # Traced by rocprofv3, llmk_step_bench ended in a host segmentation fault inside the
            # HIP runtime, below llmk_engine_forward_graph; untraced it runs to the end.
            log("  decode step from C++: skipped under rocprofv3")
            return None
        n = np.asarray(tokens).size
        fd, path = tempfile.mkstemp(suffix=".rows")
        os.close(fd)
        try:
            write_step_rows(path, cfg, tokens, pos, tables, used, max_pages)
            r = subprocess.run([exe, path, str(steps), str(warm)], capture_output=True,
                               text=True, timeout=300)
        except subprocess.TimeoutExpired:
            log("  decode step from C++: llmk_step_bench did not finish in 300 s; skipped")
            return None
        finally:
            os.unlink(path)
        if r.returncode != 0:
            log(f"  decode step from C++: llmk_step_bench exited with {r.returncode}: "
                f"{r.stderr.strip()[-300:]}")
            return None
        d = json.loads(r.stdout.strip().splitlines()[-1])
        mean_s = d["us_mean"] * 1e-6
        t = {"mean_s": mean_s, "wall_s": mean_s * d["steps"], "steps": d["steps"],
             "queue_prefilled": False}
        e = kernel_entry(f"decode step 1B, {n} seqs, C++ caller (graph)", nbytes, t, None, {
            "tokens_per_s": round(n / mean_s, 1), "seqs": int(n), "steps": d["steps"],
            "hipblaslt": d["hipblaslt"], "amdhip64": d["amdhip64"],
            "note": "the same step from llmk_step_bench, a C++ process: the system's hipBLASLt "
                    "and HIP runtime, as any C/C++ caller of the library gets them (this Python "
                    "process uses the copies torch loaded)"})
        log(f"    -> {e['tokens_per_s']:.0f} tokens/s with {d['hipblaslt']}")
        return e

    def scheduler(self):
        """The reference's scheduler benchmark on the engine (Llama-3.2-1B shape, seeded random
        weights): 24 requests (prompts of 5 to 402 tokens, 32 new tokens each, one eligible every
        2 iterations), 256 pages of 16, one request at a time and up to 8 at once, two rounds
        each as the reference runs them (ref: tests/test_scheduler.cu:14-76). words/s = new
        tokens over the scheduler's own wall clock (first iteration to last retirement), as the
        reference reports it. Decode steps of each batch size run from the engine's HIP graph
        cache."""
        wl, llmk, torch, np = self.wl, self.llmk, self.torch, self.np
        import importlib
        weights = importlib.import_module("llmk.weights")
        cfg = llmk.ModelConfig()
        max_len = max(wl.SCHED_PROMPT_LENS) + wl.SCHED_NEW
        max_pages = (max_len + wl.PAGE - 1) // wl.PAGE
        max_rows = 512  # the longest prompt (402 tokens) prefills in one pass
        eng = llmk.Engine(cfg, max_rows=max_rows, max_pages=max_pages, num_pages=wl.SCHED_PAGES)
        # A wide embedding (std 0.5) makes the logits peaked, so that the greedy tokens do not
        # hinge on last-bit differences: a sequence's bits depend on its batch (the attention's
        # split count follows the batch size), as cuBLAS results do in the reference.
        w = weights.random_weights(cfg, wl.SEED_BASE + 9, device=self.dev, embed_std=0.5)
        eng.set_weights(*weights.engine_layers(w, cfg))
        del w
        self.free()
        stream = torch.cuda.Stream()
        model = eng.sched_model(stream)
        reqs = wl.scheduler_requests()
        order = np.random.default_rng(wl.SEED_BASE + 12).permutation(
            wl.SCHED_PAGES).astype(np.int32)

        def run(rs, max_running):
            pages = llmk.PageAllocator(wl.SCHED_PAGES)
            pages.set_free_list(order)
            outs, stats, _ = llmk.run_scheduler(rs, max_running, max_pages, wl.PAGE, pages, model)
            if pages.num_free() != wl.SCHED_PAGES:
                raise RuntimeError("scheduler run leaked pages")
            return outs, stats

        self.mark("sched")
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
                rounds.append({"round": rnd, "max_running": mr,
                               "decode_steps": st["decode_steps"],
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

        # The reference's A/B of where the greedy choice is made (tests/test_scheduler_ab.cu):
        # all 24 requests eligible at once, up to 8 at once and one at a time, the argmax on the
        # host (the reference's default: logits copied back, converted, searched) and on the
        # GPU; three rounds, the order of the four reversed every other round; per decode step
        # the time split of llmk_step_times (ref: engine/batched.h:6-11).
        self.mark("sched_ab")  # kept apart: host-argmax passes end without an argmax kernel
        ab_reqs = [dict(r, arrival_step=0) for r in reqs]
        cfgs = [("batched, CPU argmax", wl.SCHED_MAX_RUNNING, 1),
                ("batched, GPU argmax", wl.SCHED_MAX_RUNNING, 0),
                ("one at a time, CPU argmax", 1, 1), ("one at a time, GPU argmax", 1, 0)]
        for host in (1, 0):  # warm-up of both paths (and their graphs), as the reference's
            eng.set_option(llmk.ENGINE_HOST_ARGMAX, host)
            run(ab_reqs[:2], wl.SCHED_MAX_RUNNING)
            run(ab_reqs[:wl.SCHED_MAX_RUNNING], wl.SCHED_MAX_RUNNING)
        ab_rounds, ab_outs = [], None
        for rnd in (1, 2, 3):
            for k in range(4):
                name, mr, host = cfgs[k if rnd % 2 else 3 - k]
                eng.set_option(llmk.ENGINE_HOST_ARGMAX, host)
                outs, st = run(ab_reqs, mr)
                if ab_outs is None:
                    ab_outs = outs
                elif outs != ab_outs:
                    raise RuntimeError(f"scheduler A/B: outputs of '{name}' differ")
                steps = max(1, st["decode_steps"])
                wps = st["total_words"] / (st["total_ms"] * 1e-3)
                per = {key: round(st[key + "_ms"] / steps, 4)
                       for key in ("prep", "gpu", "copy", "convert", "argmax")}
                ab_rounds.append({"round": rnd, "config": name, "words_per_s": round(wps, 1),
                                  "decode_steps": st["decode_steps"],
                                  "prefill_ms": round(st["prefill_ms"], 2),
                                  "per_step_ms": per})
                log(f"  scheduler A/B round {rnd} | {name:26s} | {wps:6.0f} words/s | "
                    f"{st['decode_steps']:3d} steps | prefill {st['prefill_ms']:6.1f} ms | per "
                    f"step (ms): " + ", ".join(f"{k_} {v:.3f}" for k_, v in per.items()))
        eng.set_option(llmk.ENGINE_HOST_ARGMAX, 0)
        med = {}
        for name, _, _ in cfgs:
            v = sorted(r["words_per_s"] for r in ab_rounds if r["config"] == name)
            med[name] = v[len(v) // 2]
        eng.close()
        self.free()
        self.kernels["scheduler_24x32_1b"] = {
            "label": "continuous batching, 24 requests x 32 new tokens (Llama-3.2-1B shape)",
            "words_per_s": best[wl.SCHED_MAX_RUNNING], "words_per_s_one_at_a_time": best[1],
            "gain": round(best[wl.SCHED_MAX_RUNNING] / best[1], 2), "rounds": rounds,
            "note": "reference on an RTX 4050 Laptop: 249 words/s up to 8 at once, 60 one at a "
                    "time (docs/scheduler_results.md); outputs identical in both modes",
            "argmax_ab": {
                "median_words_per_s": med,
                "gpu_over_cpu_argmax": {
                    "batched": round(med["batched, GPU argmax"] / med["batched, CPU argmax"], 3),
                    "one_at_a_time": round(med["one at a time, GPU argmax"]
                                           / med["one at a time, CPU argmax"], 3)},
                "rounds": ab_rounds,
                "note": "all 24 requests eligible at once (ref: tests/test_scheduler_ab.cu); "
                        "outputs identical in all four configurations; reference on an RTX 4050 "
                        "Laptop: 291 / 291 / 64 / 68 words/s (docs/step_time_split_results.txt)"}}


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_pass_inputs(p, wl) -> dict:
    """Host copies of a decode-pass input set for the CPU baseline. Each sequence's pool page is
    remapped to page b of a 256-page host pool: the rows the pass moves are the same, and the
    8.6 GB of device pools, almost all untouched by one pass, are not copied."""
    import numpy as np
    n, kvdim = p.n, wl.N_KV * wl.HEAD_DIM
    pos = (p.lens - 1).astype(np.int32)
    tables = np.zeros((n, p.max_pages), np.int32)
    tables[np.arange(n), pos // wl.PAGE] = np.arange(n, dtype=np.int32)
    return {"n": n, "max_pages": p.max_pages, "pos": pos, "tables": tables,
            "table": p.table.cpu().numpy().view(np.uint16),
            "ids": p.token_ids.cpu().numpy().astype(np.int32),
            "inv": p.inv_freq.cpu().numpy().astype(np.float32),
            "kpool": np.full(n * wl.PAGE * kvdim, wl.POISON, np.uint16),
            "vpool": np.full(n * wl.PAGE * kvdim, wl.POISON, np.uint16),
            "residual": np.empty((n, wl.HIDDEN), np.uint16),
            "layers": [{k: v.cpu().numpy().view(np.uint16).copy() for k, v in lay.items()
                        if k not in ("k_pool", "v_pool")} for lay in p.per_layer]}


def cpu_decode_pass(h, lib, wl, P, i32, f32):
    """A maker of the CPU decode pass: the same ops as llmk_decode_nongemm_pass (embedding; per
    layer add+RMSNorm, RoPE of Q and K, K and V scattered into the pools, SwiGLU) by the scalar
    oracle, on the host copies of cpu_pass_inputs."""
    n, H, kvdim = h["n"], wl.HIDDEN, wl.N_KV * wl.HEAD_DIM

    def make(th):
        def f():
            lib.or_embedding_lookup_mt(P(h["table"]), P(h["ids"], i32), P(h["residual"]), n, H,
                                       th)
            for lay in h["layers"]:
                lib.or_add_rmsnorm_mt(P(h["residual"]), P(lay["x"]), P(lay["norm_w"]),
                                      P(lay["normed"]), n, H, wl.EPS, th)
                lib.or_rope_apply_mt(P(lay["q"]), P(lay["k"]), P(h["pos"], i32),
                                     P(h["inv"], f32), n, wl.N_HEADS, wl.N_KV, wl.HEAD_DIM, th)
                lib.or_kv_scatter_batch(P(lay["k"]), P(h["kpool"]), P(h["tables"], i32),
                                        P(h["pos"], i32), n, h["max_pages"], wl.PAGE, kvdim)
                lib.or_kv_scatter_batch(P(lay["v"]), P(h["vpool"]), P(h["tables"], i32),
                                        P(h["pos"], i32), n, h["max_pages"], wl.PAGE, kvdim)
                lib.or_swiglu_mt(P(lay["gate"]), P(lay["up"]), P(lay["act"]), n * wl.INTER, th)
        return f
    return make


def summary(kernels: dict, torch, dev, K: int, W: int) -> None:
    """The run's headline figures, a few lines at the very end of stderr (a reader that keeps
    only the tail of the log still gets every configuration's time and roofline fraction)."""
    p = torch.cuda.get_device_properties(dev)
    # The HBM vendor and the top shader clock level, from the amdgpu driver's sysfs (boxes of
    # the same model differ in both; unreadable entries are left out).
    box = []
    for name, pick in (("mem_info_vram_vendor", lambda t: f"HBM {t.strip()}"),
                       ("pp_dpm_sclk", lambda t: "sclk up to %d MHz" % max(
                           int(m) for m in re.findall(r"(\d+)\s*[Mm][Hh]z", t)))):
        vals = set()
        for f in sorted(glob.glob(f"/sys/class/drm/card*/device/{name}")):
            try:
                with open(f) as fh:
                    vals.add(pick(fh.read()))
            except (OSError, ValueError):
                pass
        box += sorted(vals)
    log(f"summary: {p.name} ({getattr(p, 'gcnArchName', '?')}, {p.multi_processor_count} CUs"
        f"{', ' + ', '.join(box) if box else ''}), steps={K} warmup={W}; us = event-timed mean "
        f"per launch, % of 8 TB/s")
    rows = [("config 2 add+RMSNorm [8192,2048]", "add_rmsnorm_8192x2048"),
            ("config 3 RoPE 8192 tokens", "rope_8192"),
            ("config 4a SwiGLU [8192,8192]", "swiglu_8192x8192"),
            ("config 4b embedding 8192 ids", "embedding_8192"),
            ("config 1 RMSNorm [16,2048]", "rmsnorm_16x2048"),
            ("config 5 pass, one launch", "decode_pass_16x256_fused_eager"),
            ("config 5 pass, one launch, graph", "decode_pass_16x256_fused"),
            ("config 5 pass, per layer", "decode_pass_16x256_layers"),
            ("config 5 pass, per layer, direct", "decode_pass_16x256_layers_eager"),
            ("config 5 pass, op by op", "decode_pass_16x256_eager"),
            ("config 5 pass, op by op, graph", "decode_pass_16x256"),
            ("attention 256 of U[1,2048]", "attention_decode_256"),
            ("attention 16 x 2048", "attention_decode_16x2048"),
            ("argmax [256,128256]", "argmax_256x128256"),
            ("residual add [8192,2048]", "residual_add_8192x2048"),
            ("RMSNorm [8192,2048]", "rmsnorm_8192x2048"),
            ("decode step 1B, 256 rows", "decode_step_1b_256"),
            ("decode step 1B, 256 rows, from C++", "decode_step_1b_256_cpp"),
            ("decode step 1B, 8 rows", "decode_step_1b_8"),
            ("copy probe 1 GiB", "copy_1GiB")]
    for label, key in rows:
        e = kernels.get(key)
        if not e or e.get("us_mean") is None:
            continue
        ceil = e.get("ceiling") or {}
        extra = (f", {100 * ceil['kernel_frac_of_ceiling']:.1f}% of its {ceil['mix']} ceiling"
                 if ceil.get("kernel_frac_of_ceiling") else "")
        log(f"  {label:34s} {e['us_mean']:9.2f} us {100 * e['frac_of_peak']:5.1f}%{extra}")
    s = kernels.get("scheduler_24x32_1b")
    if s and s.get("words_per_s"):
        log(f"  {'scheduler, 24 requests':34s} {s['words_per_s']:9.1f} words/s up to 8 at once, "
            f"{s['words_per_s_one_at_a_time']:.1f} one at a time")


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
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    b = Bench(args)
    K, W = args.steps, args.warmup
    log(f"device: {torch.cuda.get_device_name(b.dev)}  steps={K} warmup={W}")
    what = args.kernels
    allk = what in ("all", "kernels")
    t_head, nbytes, R = b.config2()
    if allk or what == "configs":
        b.config1()
        b.config3()
        b.config4a()
    table = b.config4b() if allk or what == "configs" else None
    if allk or what in ("configs", "pass"):
        b.config5(table)
        b.config5_two_norms(table)
    del table
    if allk or what == "attn":
        b.attention()
    if allk:
        b.argmax()
    if allk or what == "rows":
        b.other_rows()
    if what in ("all", "step"):
        b.decode_step(256)
    if what in ("all", "step8"):
        b.decode_step(8)
    if what in ("all", "sched"):
        b.scheduler()
    if allk or what in ("probe", "configs"):
        sweep = b.probes()
        b.kernel_ceilings(sweep)
    if allk or what == "calib":
        b.calibration()
    b.copy_probe()
    b.mark("end")
    torch.cuda.synchronize()

    cpu = None
    if not args.no_cpu:
        cpus = b.cpu_baselines(args.cpu_seconds)
        head_cpu = cpus.get("add_rmsnorm_8192x2048")
        if head_cpu:
            cpu = {k: v for k, v in head_cpu.items() if k != "gpu_over_cpu"}
            cpu.update(b.cpu_info)

    summary(b.kernels, torch, b.dev, K, W)
    head = b.kernels["add_rmsnorm_8192x2048"]
    value = nbytes * K / t_head["wall_s"] / 1e9
    rec = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": K,
        "warmup": W, "ms_per_step": round(t_head["wall_s"] / K * 1e3, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16", "data": "synthetic",
        "config": {"workload": "fused residual add + RMSNorm fp16 [8192,2048] (configs[1])",
                   "rows": 8192, "hidden": 2048, "eps": b.wl.EPS, "accumulate": "f32",
                   "input_sets": R, "algorithmic_bytes_per_step": nbytes},
        "roofline": {"bound": "hbm", "achieved": head["GBps"], "peak": PEAK_GBS,
                     "unit": "GB/s", "frac": round(head["GBps"] / PEAK_GBS, 4),
                     "traffic": b.traffic.get("add_rmsnorm_8192x2048")},
        "cpu_baseline": cpu,
        "kernels": b.kernels,
    }
    print(json.dumps(rec), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
