#!/usr/bin/env python3
"""Benchmark: FlashAttention forward on one MI355X.

One "step" is one forward call (O plus the fp32 row LSE) over the headline
workload, B4 H32 S2048 D128 bf16 causal, with q/k/v already resident in HBM.
Prints ONE JSON line on stdout:

  value        whole-job TFLOP/s = 4*B*H*S*S*D/2 / (wall time per step)
  roofline     the kernel's TFLOP/s from HIP events on the launch stream,
               against MI355X's dense bf16 MFMA peak (2516.6 TFLOP/s)
  cpu_baseline the CPU oracle (numpy fp32 formula) timed on this host's
               cores over a bounded sample of the same workload (whole heads)

Everything else (per-call evaluator-style wall clock, the run's sizes) goes to
stderr.  Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

METRIC = "attn fwd TFLOP/s + % bf16 MFMA peak, B4·H32·S2048·D128 causal, 1 GPU"
PEAK_BF16_TFLOPS = 2516.6   # MI355X dense bf16/fp16 MFMA: 256 CU x 4096 FLOP/clk x 2.4 GHz
PEAK_HBM_GBS = 8000.0


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def profile_summary_path(workload_tag: str) -> Path:
    return REPO / "profiles" / f"fa_fwd_{workload_tag}_rocprof.txt"


def read_traffic(workload_tag: str, build_id: str):
    """HBM bytes per launch from the committed rocprofv3 summary, if it was made
    with the library being benched.

    The summary (written by flash_attn_npu_amd.rocprof from FETCH_SIZE and
    WRITE_SIZE passes, each scaled by what the same counter reads for a plain
    256 MiB device copy in the same process) carries hbm_read_bytes= and
    hbm_write_bytes= in its kernel_metrics lines, and the profiled library's
    fa_build_id in its build: line.  A summary of another build (or one with no
    stamp) gives None: its bytes need not be this kernel's.
    """
    from flash_attn_npu_amd.rocprof import read_build_id

    path = profile_summary_path(workload_tag)
    if not path.exists():
        log(f"traffic: no summary {path.name}")
        return None
    stamped = read_build_id(path)
    if stamped != build_id:
        log(f"traffic: {path.name} was profiled with build {stamped}, this library is {build_id}: not used")
        return None
    vals = {}
    for line in path.read_text().splitlines():
        for item in line.split(","):
            if "=" in item:
                key, val = item.strip().split("=", 1)
                key = key.split(":")[-1].strip()
                if key in ("hbm_read_bytes", "hbm_write_bytes"):
                    try:
                        vals[key] = float(val)
                    except ValueError:
                        pass
    if len(vals) != 2:
        return None
    return int(vals["hbm_read_bytes"] + vals["hbm_write_bytes"])


def cpu_baseline(w, budget_s: float):
    """The CPU oracle (numpy fp32 formula) over the whole workload on this host.

    One untimed pass, then timed passes until `budget_s` is spent (at least
    3, as many as fit); the median pass time is charged the same FLOP formula
    as the GPU (causal halved, although the CPU computes every score).
    """
    from oracle.attention_oracle import attention_ref
    from flash_attn_npu_amd.workloads import make_inputs

    threads = len(os.sched_getaffinity(0))
    try:
        from threadpoolctl import threadpool_limits
        limiter = threadpool_limits(limits=threads)
    except Exception:  # noqa: BLE001
        limiter = None
    q, k, v = make_inputs(w)
    qn, kn, vn = (t.float().numpy() for t in (q, k, v))
    dt = "bfloat16" if "bf" in str(w.dtype) else "float16"

    def one_pass():
        t0 = time.perf_counter()
        for b in range(w.B):
            attention_ref(qn[b], kn[b], vn[b], w.causal, w.sm_scale, out_dtype=dt)
        return time.perf_counter() - t0

    first = one_pass()
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - t_start + first < budget_s and len(times) < 50):
        times.append(one_pass())
    if limiter is not None:
        limiter.restore_original_limits()
    med = statistics.median(times)
    try:
        model = next(l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo") if l.startswith("model name"))
    except Exception:  # noqa: BLE001
        model = "unknown"
    return {
        "value": w.flops / med / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": f"the whole workload ({w.B * w.H} heads, S={w.S}), numpy fp32 oracle, median of "
                  f"{len(times)} timed passes after 1 warmup ({med:.2f} s/pass; every score computed, "
                  f"charged the causal-halved FLOP formula); CPU: {model}",
    }


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--warmup-seconds", type=float, default=1.0)
    ap.add_argument("--config", type=int, default=2, help="1-based index of the measured configuration")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="CPU baseline budget (0 = skip)")
    ap.add_argument("--block-m", type=int, default=None, help="BLOCK_M override (default: the library's tiling)")
    ap.add_argument("--block-n", type=int, default=None, help="BLOCK_N override (default: the library's tiling)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="after timing, run a plain 256 MiB device copy (rocprofv3 FETCH/WRITE calibration)")
    args = ap.parse_args(argv)

    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported "
              "(this forward needs no collective; heads shard across GPUs with no exchange).",
              file=sys.stderr)
        return 2

    import torch
    from flash_attn_npu_amd import flash_attention_forward as fa
    from flash_attn_npu_amd.workloads import CONFIGS, make_inputs

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    fa._load_library()
    w = CONFIGS[args.config - 1]
    log(f"workload: {w.describe()} sm_scale={w.sm_scale:.6f}")
    q, k, v = make_inputs(w, device="cuda")
    torch.cuda.synchronize()
    rt = fa._describe_runtime(w.B, w.H, w.S, w.D, w.causal, bm=args.block_m, bn=args.block_n, dtype=w.dtype)
    log(f"runtime: {rt}")

    def step():
        return fa.attention(q, k, v, w.causal, w.sm_scale, BM=args.block_m, BN=args.block_n, return_lse=w.with_lse)

    # Warm up for at least W steps and at least one second, so the timed steps
    # run at the clocks a sustained load settles at.
    t_w = time.perf_counter()
    n_w = 0
    while n_w < args.warmup or time.perf_counter() - t_w < args.warmup_seconds:
        step()
        n_w += 1
        if n_w % 10 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    log(f"warmup: {n_w} steps in {time.perf_counter() - t_w:.2f} s")

    stream = torch.cuda.current_stream()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(args.steps):
        step()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ev_ms = ev0.elapsed_time(ev1)

    # Per-launch spread from events around single launches.
    per = []
    for _ in range(10):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        step()
        e1.record(stream)
        torch.cuda.synchronize()
        per.append(e0.elapsed_time(e1) * 1e3)
    log(f"single-launch events: min {min(per):.1f} median {statistics.median(per):.1f} max {max(per):.1f} us")

    # Evaluator-style per-call wall clock (perf_counter around call + synchronize,
    # evaluate_attention.py:233-264), for comparison only.
    samples = []
    for _ in range(20):
        s0 = time.perf_counter()
        step()
        torch.cuda.synchronize()
        samples.append((time.perf_counter() - s0) * 1e6)

    ms_per_step = wall * 1e3 / args.steps
    kernel_ms = ev_ms / args.steps
    value = w.flops / (ms_per_step * 1e-3) / 1e12
    achieved = w.flops / (kernel_ms * 1e-3) / 1e12
    log(f"wall {ms_per_step * 1e3:.1f} us/step, events {kernel_ms * 1e3:.1f} us/launch, "
        f"evaluator-style median {statistics.median(samples):.1f} us")
    log(f"HBM-level algorithmic bytes {w.io_bytes} -> {w.io_bytes / (kernel_ms * 1e-3) / 1e9:.0f} GB/s")

    if args.calibrate_copy:
        a = torch.empty(128 * 1024 * 1024, dtype=torch.float16, device="cuda").fill_(1.0)
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        del a, b

    tag = w.name
    build_id = fa._load_library().fa_build_id().decode()
    traffic = read_traffic(tag, build_id)
    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "pct_of_peak": round(100.0 * value / PEAK_BF16_TFLOPS, 2),
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if w.dtype == torch.bfloat16 else "fp16",
        "data": "synthetic (seeded N(0,1) q/k/v, CPU generator)",
        "config": {"workload": f"attn fwd {tag}", "B": w.B, "H": w.H, "S": w.S, "D": w.D,
                   "causal": w.causal, "sm_scale": w.sm_scale, "lse": w.with_lse,
                   "BLOCK_M": rt["selected_config"]["BLOCK_M"], "BLOCK_N": rt["selected_config"]["BLOCK_N"],
                   "waves": rt["waves"], "grid": rt["launched_programs"]},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": traffic, "kernel_us": round(kernel_ms * 1e3, 2),
                     "algorithmic_flops": w.flops, "algorithmic_bytes": w.io_bytes},
        "evaluator_median_us": round(statistics.median(samples), 2),
    }
    if args.cpu_seconds > 0:
        cb = cpu_baseline(w, args.cpu_seconds)
        cb.pop("seconds_per_step_extrapolated", None)
        result["cpu_baseline"] = cb
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
