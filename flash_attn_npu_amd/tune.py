"""gfx950 tiling tuner: the counterpart of tune_flash_attention_forward.py.

For each case (default: the evaluator's six performance shapes in float16 and
bfloat16, plus the five benchmark workloads in their own dtype) it times every
(BLOCK_M, BLOCK_N) that the library has a kernel for at that head dim, dtype
and causal flag (`fa.kernel_table()`; each instance has a fixed number of
resident workgroups per CU, recorded as WG_PER_CU), the way bench.py measures
the headline number:

  * at least `--warmup-seconds` (1 s) of launches before the first timing, so
    the clocks are those of a sustained load;
  * `--rounds` rounds; in each, every candidate gets 2 untimed launches and
    then `--launches` (>= 20) back-to-back launches between two HIP events on
    the launch stream; candidates rotate their order from round to round;
  * a candidate's time is the median over rounds of its per-launch average;
  * when the fastest candidate's launch is shorter than `--graph-below-us`
    (40 µs: the host's per-call cost, ~13 µs, then sets the pace of eager
    launches), the rounds are timed again as replays of HIP graphs that hold
    `--launches` launches each, so the ranking is by device time.

The winner is re-timed next to the vendor baseline (PyTorch-ROCm fused SDPA,
as in flash_attn_npu_amd/evaluate.py) both back to back and per call with a
synchronize (the reference's `_measure_candidate`, kept as `percall_*`).  When
the library's own default is within `--tie-pct` of the fastest, the default
is kept (a preset then only restates it).

With --profile, the winner and the runner-up of every case run under the
rocprofv3 passes of flash_attn_npu_amd/rocprof.py (kernel trace, compute, LDS,
L2, HBM read and HBM write counters; one child process per pass runs every
profiled configuration in turn, plus a 256 MiB device copy that calibrates the
byte counters), and each result records the counters that justify its choice:
kernel time, MfmaUtil(%), VALU instructions per MFMA, LDS bank conflicts,
L2 hit rate, L2-miss read/write bytes and the achieved GB/s.

Output: the reference's JSON schema (tune_flash_attention_forward.py:217-274,
:428-449), flash_attention_forward_tuned.json:

    {"meta": {...},
     "tuned_configs": {"Z:H:N_CTX:HEAD_DIM:causal[:bf16]": {"BLOCK_M", "BLOCK_N", "WAVES", "WG_PER_CU"}},
     "results": [{shape, dtype, best_config, candidate_*_us, percall_*_us, baseline_*_us,
                  speedup_vs_baseline, max_abs_diff, correctness_error, candidates: [...],
                  counters: {...}, choice: "..."}]}

Keys without a dtype suffix are float16 (the reference tunes float16); keys
ending in ":bf16" are bfloat16.  The DEFAULT_TILING_PRESETS block of the
module is rewritten between the reference's BEGIN/END markers
(tune_flash_attention_forward.py:20-21, :327-366): float16 entries into
DEFAULT_TILING_PRESETS, bfloat16 ones into DEFAULT_TILING_PRESETS_BF16.

    python -m flash_attn_npu_amd.tune [--suite all|evaluator|configs] [--profile --profile-dir DIR]
    python -m flash_attn_npu_amd.tune --shape 4,32,2048,128,1 --dtype bf16
    python -m flash_attn_npu_amd.tune --merge a.json b.json --output-json out.json
"""

from __future__ import annotations

import argparse
import json
import statistics
import sys
import tempfile
import time
from dataclasses import dataclass
from pathlib import Path

import torch

from flash_attn_npu_amd import evaluate as E
from flash_attn_npu_amd import workloads as W

PRESET_BEGIN = "# BEGIN AUTO-TUNED DEFAULT TILING PRESETS"
PRESET_END = "# END AUTO-TUNED DEFAULT TILING PRESETS"
PACKAGE_DIR = Path(__file__).resolve().parent
DEFAULT_OUTPUT_JSON = PACKAGE_DIR / "flash_attention_forward_tuned.json"
DEFAULTS = dict(sm_scale=W.REFERENCE_SM_SCALE, seed=0, warmup_seconds=1.0, rounds=5, launches=20,
                final_iters=20, tie_pct=1.0, graph_below_us=40.0)
DTYPE_SUFFIX = {torch.float16: "", torch.bfloat16: ":bf16"}
PROFILE_LAUNCHES = 5  # per profiled configuration and pass; the first is not counted


@dataclass
class Case:
    """One tuned case: a shape, its input dtype and how its inputs are drawn."""
    shape: tuple            # (Z, H, N_CTX, HEAD_DIM, causal)
    dtype: torch.dtype
    sm_scale: float
    seed: int
    workload: str | None = None   # name of a benchmark workload (inputs from workloads.make_inputs)

    @property
    def key(self) -> str:
        return shape_key(self.shape, self.dtype)

    def inputs(self, device):
        if self.workload is not None:
            w = next(w for w in W.CONFIGS if w.name == self.workload)
            return W.make_inputs(w, device=device)
        return E.make_case_inputs(device, self.dtype, self.shape, self.seed)

    def to_json(self):
        return {"shape": list(self.shape), "dtype": E.dtype_name(self.dtype), "sm_scale": self.sm_scale,
                "seed": self.seed, "workload": self.workload}

    @classmethod
    def from_json(cls, d):
        return cls(tuple(d["shape"][:4]) + (bool(d["shape"][4]),), E.dtype_from_name(d["dtype"]),
                   float(d["sm_scale"]), int(d["seed"]), d.get("workload"))


def shape_key(shape, dtype=torch.float16) -> str:
    z, h, n, d, causal = shape
    return f"{z}:{h}:{n}:{d}:{int(bool(causal))}" + DTYPE_SUFFIX.get(dtype, ":" + E.dtype_name(dtype))


def parse_key(key: str):
    """'Z:H:N:D:c[:bf16]' -> ((Z, H, N, D, causal), dtype)."""
    parts = key.split(":")
    shape = tuple(int(p) for p in parts[:4]) + (bool(int(parts[4])),)
    dtype = torch.bfloat16 if len(parts) > 5 and parts[5] in ("bf16", "bfloat16") else torch.float16
    return shape, dtype


def parse_shape(text: str):
    parts = [p.strip() for p in text.split(",")]
    if len(parts) != 5:
        raise ValueError(f"shape must be Z,H,N_CTX,HEAD_DIM,causal: {text!r}")
    causal = parts[4].lower() in ("1", "true", "yes")
    return (int(parts[0]), int(parts[1]), int(parts[2]), int(parts[3]), causal)


def default_cases(suite: str, sm_scale: float, seed: int):
    cases = []
    if suite in ("all", "evaluator"):
        for dtype in (torch.float16, torch.bfloat16):
            cases += [Case(tuple(s), dtype, sm_scale, seed) for s in W.REFERENCE_PERFORMANCE_CASES]
    if suite in ("all", "configs"):
        cases += [Case((w.B, w.H, w.S, w.D, w.causal), w.dtype, w.sm_scale, w.seed, workload=w.name)
                  for w in W.CONFIGS]
    return cases


def tiling_candidates(module, shape, dtype):
    """(BLOCK_M, BLOCK_N, waves, workgroups per CU) of every kernel for this head dim,
    dtype and causal flag."""
    d, causal = shape[3], bool(shape[4])
    dt = E.dtype_name(dtype)
    seen, out = set(), []
    for row in module.kernel_table():
        if row["HEAD_DIM"] != d or row["dtype"] != dt or bool(row["causal"]) != causal:
            continue
        key = (row["BLOCK_M"], row["BLOCK_N"])
        if key not in seen:
            seen.add(key)
            out.append((row["BLOCK_M"], row["BLOCK_N"], row["waves"], row.get("wg_per_cu")))
    return out


def library_default(module, shape, dtype):
    """(BLOCK_M, BLOCK_N) the library picks for this shape without a preset."""
    z, h, n, d, causal = shape
    cfg = module._query_config(z, h, n, d, causal, dtype=dtype)
    return cfg[0], cfg[1]


# --------------------------------------------------------------------------
# timing

def events_per_launch(fn, launches: int) -> float:
    """Mean µs per launch of `launches` back-to-back calls, from two HIP events on
    the launch stream (what bench.py's roofline figure uses)."""
    stream = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(launches):
        fn()
    e1.record(stream)
    e1.synchronize()
    return e0.elapsed_time(e1) * 1e3 / launches


def warm_up(fn, seconds: float, min_calls: int = 3):
    t0 = time.perf_counter()
    n = 0
    while n < min_calls or time.perf_counter() - t0 < seconds:
        fn()
        n += 1
        if n % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    return n


def percall_us(fn, iters: int):
    """The reference's per-call clock: perf_counter around a call and a synchronize."""
    fn()
    torch.cuda.synchronize()
    samples = []
    out = None
    for _ in range(iters):
        t0 = time.perf_counter()
        out = fn()
        torch.cuda.synchronize()
        samples.append((time.perf_counter() - t0) * 1e6)
    return out, {"avg_us": statistics.mean(samples), "min_us": min(samples), "max_us": max(samples)}


def graph_per_launch(fn, launches: int):
    """A callable that replays `launches` calls captured in one HIP graph and
    returns the µs per launch between two events: the device time of a launch
    without the host's per-call cost (which back-to-back eager launches of a
    short kernel cannot hide)."""
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # first use of the allocator pool outside the capture
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            for _ in range(launches):
                fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()

    def replay():
        stream = torch.cuda.current_stream()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        g.replay()
        e1.record(stream)
        e1.synchronize()
        return e0.elapsed_time(e1) * 1e3 / launches

    replay.graph = g
    return replay


def time_candidates(fns: dict, rounds: int, launches: int, graphs: dict | None = None):
    """Interleaved timing: per candidate, the per-round per-launch averages
    (rotating the order each round so drift hits every candidate).  Back-to-back
    eager launches, or replays of `graphs[name]` when given."""
    names = list(fns)
    per = {n: [] for n in names}
    for r in range(rounds):
        order = names[r % len(names):] + names[:r % len(names)]
        for n in order:
            if graphs is not None:
                graphs[n]()
                per[n].append(graphs[n]())
                continue
            fn = fns[n]
            fn()
            fn()
            per[n].append(events_per_launch(fn, launches))
    return per


# --------------------------------------------------------------------------
# one case

def tune_case(module, vendor, case: Case, opts) -> dict:
    z, h, n, d, causal = case.shape
    dtype = case.dtype
    q, k, v = case.inputs(module.DEVICE)
    cands = tiling_candidates(module, case.shape, dtype)
    if not cands:
        raise RuntimeError(f"no kernel for {case.key}")
    fns, rows = {}, {}
    for bm, bn, waves, wg in cands:
        tag = f"{bm}x{bn}"
        cfg = {"BLOCK_M": bm, "BLOCK_N": bn, "WAVES": waves, "WG_PER_CU": wg}
        fn = (lambda bm=bm, bn=bn: module._launch_kernel(q, k, v, causal, case.sm_scale, bm=bm, bn=bn)[0])
        try:
            fn()
            torch.cuda.synchronize()
        except Exception as exc:  # noqa: BLE001 - recorded per candidate, as the reference does
            rows[tag] = {"config": cfg, "avg_us": None,
                         "error": str(exc).splitlines()[0][:240] if str(exc) else type(exc).__name__}
            continue
        fns[tag] = fn
        rows[tag] = {"config": cfg}
    if not fns:
        raise RuntimeError(f"no viable config for {case.key}")
    default_tag = "{}x{}".format(*library_default(module, case.shape, dtype))
    warm_up(fns.get(default_tag, next(iter(fns.values()))), opts.warmup_seconds)
    per = time_candidates(fns, opts.rounds, opts.launches)
    timing = "eager"
    if min(statistics.median(xs) for xs in per.values()) < opts.graph_below_us:
        # A launch this short is shorter than the host's per-call cost: back-to-back
        # eager launches then time the host.  Rank the device time of graph replays.
        # A captured launch walks the static tile schedule (no queue counters), which
        # for these short grids (at most a few tiles per workgroup) is the eager
        # order up to the pulls of workgroups that finish early; the label says so.
        graphs = {tag: graph_per_launch(fn, opts.launches) for tag, fn in fns.items()}
        per = time_candidates(fns, opts.rounds, opts.launches, graphs)
        timing = "graph (static schedule)"
        del graphs
    for tag, xs in per.items():
        rows[tag].update(avg_us=statistics.median(xs), min_us=min(xs), max_us=max(xs), rounds_us=xs,
                         launches_per_round=opts.launches, timing=timing)
    viable = sorted((r for r in rows.values() if r.get("avg_us") is not None), key=lambda r: r["avg_us"])
    fastest = viable[0]
    best_row = fastest
    choice = "fastest"
    if default_tag in fns and default_tag != f"{fastest['config']['BLOCK_M']}x{fastest['config']['BLOCK_N']}":
        d_row = rows[default_tag]
        if d_row["avg_us"] <= fastest["avg_us"] * (1.0 + opts.tie_pct / 100.0):
            best_row = d_row
            choice = (f"library default kept: within {opts.tie_pct:.1f}% of the fastest "
                      f"({d_row['avg_us']:.2f} vs {fastest['avg_us']:.2f} us)")
    best = dict(best_row["config"])
    best_tag = f"{best['BLOCK_M']}x{best['BLOCK_N']}"
    if choice == "fastest":
        if len(viable) > 1:
            ru = viable[1]
            margin = 100.0 * (ru["avg_us"] / fastest["avg_us"] - 1.0)
            choice = ("fastest" + (" (the library default)" if best_tag == default_tag else "")
                      + f", {margin:.1f}% ahead of {ru['config']['BLOCK_M']}x{ru['config']['BLOCK_N']}")
        else:
            choice = "only candidate"
    best_fn = fns[best_tag]
    cand_out, pc = percall_us(best_fn, opts.final_iters)
    result = {"Z": z, "H": h, "N_CTX": n, "HEAD_DIM": d, "causal": bool(causal), "dtype": E.dtype_name(dtype),
              "sm_scale": case.sm_scale, "workload": case.workload, "best_config": best, "timing": timing,
              "library_default": default_tag, "choice": choice,
              "candidate_avg_us": best_row["avg_us"], "candidate_min_us": best_row["min_us"],
              "candidate_max_us": best_row["max_us"], "percall_avg_us": pc["avg_us"],
              "percall_min_us": pc["min_us"], "percall_max_us": pc["max_us"],
              "baseline_avg_us": None, "baseline_min_us": None, "baseline_max_us": None,
              "speedup_vs_baseline": None, "max_abs_diff": None, "correctness_error": None,
              "candidates": list(rows.values())}
    try:
        vfn = lambda: vendor(q, k, v, causal, case.sm_scale)  # noqa: E731
        ref_out = vfn()
        warm_up(vfn, 0.2)
        base = time_candidates({"v": vfn}, opts.rounds, opts.launches)["v"]
        result.update(baseline_avg_us=statistics.median(base), baseline_min_us=min(base), baseline_max_us=max(base),
                      baseline_op=vendor.used.get(tuple(q.shape) + (bool(causal),)))
        result["speedup_vs_baseline"] = result["baseline_avg_us"] / result["candidate_avg_us"]
        result["max_abs_diff"] = torch.max(torch.abs(cand_out.float() - ref_out.to(dtype).float())).item()
        del ref_out
    except Exception as exc:  # noqa: BLE001
        result["correctness_error"] = str(exc)[:240]
    del q, k, v, cand_out
    torch.cuda.empty_cache()
    return result


# --------------------------------------------------------------------------
# rocprofv3 counters for the top configurations

def profile_entries(results, top: int = 2):
    """(case, BLOCK_M, BLOCK_N) of the chosen config and the next fastest of each result."""
    entries = []
    for r in results:
        case = Case((r["Z"], r["H"], r["N_CTX"], r["HEAD_DIM"], r["causal"]), E.dtype_from_name(r["dtype"]),
                    r["sm_scale"], r.get("seed", 0), r.get("workload"))
        tags = [f"{r['best_config']['BLOCK_M']}x{r['best_config']['BLOCK_N']}"]
        for c in sorted((c for c in r["candidates"] if c.get("avg_us") is not None), key=lambda c: c["avg_us"]):
            t = f"{c['config']['BLOCK_M']}x{c['config']['BLOCK_N']}"
            if t not in tags:
                tags.append(t)
        for t in tags[:top]:
            bm, bn = (int(x) for x in t.split("x"))
            entries.append({"case": case.to_json(), "bm": bm, "bn": bn, "key": case.key, "tag": t})
    return entries


def run_plan(plan_path: Path, manifest_path: Path | None):
    """Child of --profile: PROFILE_LAUNCHES launches of each planned configuration
    in order, then a 256 MiB device copy for the byte-counter calibration."""
    from flash_attn_npu_amd import flash_attention_forward as fa
    from flash_attn_npu_amd import rocprof
    entries = json.loads(Path(plan_path).read_text())
    manifest = []
    for e in entries:
        case = Case.from_json(e["case"])
        z, h, n, d, causal = case.shape
        q, k, v = case.inputs(fa.DEVICE)
        rt = fa._describe_runtime(z, h, n, d, causal, bm=e["bm"], bn=e["bn"], dtype=case.dtype)
        for _ in range(PROFILE_LAUNCHES):
            fa._launch_kernel(q, k, v, causal, case.sm_scale, bm=e["bm"], bn=e["bn"])
        torch.cuda.synchronize()
        manifest.append({"key": e["key"], "tag": e["tag"], "launches": PROFILE_LAUNCHES,
                         "dispatches_per_launch": 2 if rt["kv_splits"] > 1 else 1})
        del q, k, v
        if manifest_path is not None:  # written as it grows: a long pass shows progress
            Path(manifest_path).write_text(json.dumps(manifest))
    a = torch.empty(rocprof.COPY_BYTES // 2, dtype=torch.float16, device="cuda")
    a.fill_(1.0)
    b = torch.empty_like(a)
    b.copy_(a)
    torch.cuda.synchronize()


def _is_attention_kernel(name: str) -> bool:
    return "fa_fwd" in name or "fa_merge" in name


def collect_counters(out_dir: Path, manifest: list, passes: dict) -> dict:
    """Per (key, tag): the counters of the configuration's launches after the first."""
    from flash_attn_npu_amd import rocprof
    res = {(m["key"], m["tag"]): {} for m in manifest}
    for pname in passes:
        pdir = out_dir / pname
        recs = rocprof.read_dispatches(pdir, _is_attention_kernel)
        factors = rocprof.copy_factors(pdir)
        i = 0
        for m in manifest:
            per = m["dispatches_per_launch"]
            launches = [recs[i + j * per:i + (j + 1) * per] for j in range(m["launches"])]
            i += per * m["launches"]
            dst = res[(m["key"], m["tag"])]
            kept = launches[1:] or launches
            if pname == "KernelTrace":
                dst["kernel_us"] = statistics.mean(sum(r.get("duration_us", 0.0) for r in ls) for ls in kept)
                continue
            sums: dict[str, list] = {}
            for ls in kept:
                tot: dict[str, float] = {}
                for j, r in enumerate(ls):
                    for c, val in r["counters"].items():
                        # Rates and utilisations come from the attention kernel itself (the
                        # first dispatch of a launch); bytes add the merge kernel's.
                        if j == 0 or c in ("FETCH_SIZE", "WRITE_SIZE", "TCC_EA0_RDREQ_DRAM_sum"):
                            tot[c] = tot.get(c, 0.0) + val
                for c, val in tot.items():
                    sums.setdefault(c, []).append(val)
            for c, vals in sums.items():
                dst[c] = statistics.mean(vals)
            for c in ("FETCH_SIZE", "WRITE_SIZE"):
                if c in dst and c in factors:
                    dst[f"{c}_copy_factor"] = factors[c]
            if "TCC_EA0_RDREQ_DRAM_sum" in dst and "TCC_EA0_RDREQ_DRAM_sum" in factors:
                dst["TCC_EA0_RDREQ_DRAM_sum_bytes_per_req"] = factors["TCC_EA0_RDREQ_DRAM_sum"]
        if i != len(recs):
            raise RuntimeError(f"pass {pname}: {len(recs)} attention dispatches, the plan expects {i}")
    for dst in res.values():
        derive(dst)
    return res


def derive(k: dict):
    """MfmaUtil(%), VALU per MFMA, LDS bank conflicts, L2 hit rate, bytes and GB/s."""
    from flash_attn_npu_amd import rocprof
    if k.get("GRBM_GUI_ACTIVE") and "SQ_VALU_MFMA_BUSY_CYCLES" in k:
        k["MfmaUtil(%)"] = 100.0 * k["SQ_VALU_MFMA_BUSY_CYCLES"] / rocprof.NUM_SIMDS / (k["GRBM_GUI_ACTIVE"] / 8)
    if k.get("SQ_INSTS_MFMA"):
        k["valu_per_mfma"] = k.get("SQ_INSTS_VALU", 0.0) / k["SQ_INSTS_MFMA"]
    if k.get("SQ_LDS_IDX_ACTIVE"):
        k["LDSBankConflict(%)"] = 100.0 * k.get("SQ_LDS_BANK_CONFLICT", 0.0) / k["SQ_LDS_IDX_ACTIVE"]
    if "TCC_HIT_sum" in k and "TCC_MISS_sum" in k:
        tot = k["TCC_HIT_sum"] + k["TCC_MISS_sum"]
        k["l2_hit_rate"] = k["TCC_HIT_sum"] / tot if tot else None
    for c, label in (("FETCH_SIZE", "l2_miss_read_bytes"), ("WRITE_SIZE", "l2_miss_write_bytes")):
        if c in k:
            k[label] = k[c] * 1024.0 * k.get(f"{c}_copy_factor", 1.0)
    if "TCC_EA0_RDREQ_DRAM_sum" in k and k.get("TCC_EA0_RDREQ_DRAM_sum_bytes_per_req"):
        # Second read figure: memory-side read requests times the bytes per
        # request that the calibration copy shows.
        k["l2_miss_read_bytes_by_requests"] = k["TCC_EA0_RDREQ_DRAM_sum"] * k["TCC_EA0_RDREQ_DRAM_sum_bytes_per_req"]
    if k.get("kernel_us") and "l2_miss_read_bytes" in k and "l2_miss_write_bytes" in k:
        k["achieved_GBps"] = (k["l2_miss_read_bytes"] + k["l2_miss_write_bytes"]) / (k["kernel_us"] * 1e-6) / 1e9
    return k


COUNTER_KEYS = ("kernel_us", "MfmaUtil(%)", "valu_per_mfma", "LDSBankConflict(%)", "l2_hit_rate",
                "l2_miss_read_bytes", "l2_miss_write_bytes", "l2_miss_read_bytes_by_requests", "achieved_GBps", "SQ_VALU_MFMA_COEXEC_CYCLES",
                "SQ_WAIT_INST_ANY", "SQ_WAIT_ANY", "FETCH_SIZE_copy_factor", "WRITE_SIZE_copy_factor")


def profile_results(results, out_dir: Path, top: int = 2):
    """Run the rocprofv3 passes over every result's top configurations and attach
    `counters` {tag: {...}} to each result."""
    from flash_attn_npu_amd import rocprof
    out_dir = Path(out_dir).resolve()
    out_dir.mkdir(parents=True, exist_ok=True)
    entries = profile_entries(results, top)
    plan = out_dir / "plan.json"
    plan.write_text(json.dumps(entries, indent=1))
    manifest_path = out_dir / "manifest.json"
    passes = dict(rocprof.METRIC_PLAN)
    cmd = [sys.executable, "-m", "flash_attn_npu_amd.tune", "--run-plan", str(plan), "--manifest", str(manifest_path)]
    rocprof.run_passes(out_dir, cmd, passes, timeout=900)
    manifest = json.loads(manifest_path.read_text())
    counters = collect_counters(out_dir, manifest, passes)
    for r in results:
        key = shape_key((r["Z"], r["H"], r["N_CTX"], r["HEAD_DIM"], r["causal"]), E.dtype_from_name(r["dtype"]))
        r["counters"] = {tag: {c: v for c, v in vals.items() if c in COUNTER_KEYS}
                         for (k, tag), vals in counters.items() if k == key}
    return results


# --------------------------------------------------------------------------
# JSON, presets, summary

def result_key(item: dict) -> str:
    return shape_key((item["Z"], item["H"], item["N_CTX"], item["HEAD_DIM"], item["causal"]),
                     E.dtype_from_name(item.get("dtype", "float16")))


def merge_payloads(old: dict, new: dict) -> dict:
    """`new` wins per key; keys only in `old` are kept, in their order."""
    configs = dict(old.get("tuned_configs", {}))
    configs.update(new.get("tuned_configs", {}))
    results, order = {}, []
    for item in list(old.get("results", [])) + list(new.get("results", [])):
        if not isinstance(item, dict):
            continue
        key = result_key(item)
        if key not in order:
            order.append(key)
        results[key] = item
    merged = dict(old)
    merged.update(new)
    merged.update(tuned_configs=configs, results=[results[k] for k in order])
    return merged


def merge_with_existing(path: Path, payload: dict) -> dict:
    if not path.exists():
        return payload
    try:
        old = json.loads(path.read_text(encoding="utf-8"))
    except (OSError, ValueError):
        return payload
    return merge_payloads(old, payload)


def presets_block(tuned_configs: dict) -> str:
    tables = {torch.float16: [], torch.bfloat16: []}
    for key, cfg in tuned_configs.items():
        shape, dtype = parse_key(key)
        tables[dtype].append((shape, cfg))
    lines = [PRESET_BEGIN,
             "# (Z, H, N_CTX, HEAD_DIM, causal) -> (BLOCK_M, BLOCK_N), rewritten by",
             "# python -m flash_attn_npu_amd.tune from gfx950 sweeps: float16 inputs here,",
             "# bfloat16 inputs in DEFAULT_TILING_PRESETS_BF16."]
    for name, dtype in (("DEFAULT_TILING_PRESETS", torch.float16), ("DEFAULT_TILING_PRESETS_BF16", torch.bfloat16)):
        lines.append(f"{name} = {{")
        for (z, h, n, d, c), cfg in sorted(tables[dtype], key=lambda e: e[0]):
            lines.append(f"    ({z}, {h}, {n}, {d}, {bool(c)}): ({int(cfg['BLOCK_M'])}, {int(cfg['BLOCK_N'])}),")
        lines.append("}")
    lines.append(PRESET_END)
    return "\n".join(lines)


def apply_presets(module_path: Path, tuned_json: Path):
    payload = json.loads(tuned_json.read_text(encoding="utf-8"))
    configs = payload.get("tuned_configs", {})
    if not configs:
        raise ValueError(f"no tuned_configs in {tuned_json}")
    src = module_path.read_text(encoding="utf-8")
    begin, end = src.find(PRESET_BEGIN), src.find(PRESET_END)
    if begin < 0 or end < begin:
        raise RuntimeError(f"cannot locate {PRESET_BEGIN!r} / {PRESET_END!r} in {module_path}")
    module_path.write_text(src[:begin] + presets_block(configs) + src[end + len(PRESET_END):], encoding="utf-8")


def _f(v, fmt):
    return "n/a" if v is None else format(v, fmt)


def summary_text(payload: dict) -> str:
    """One block per case: every candidate's time, the choice, and the counters of
    the two profiled configurations."""
    meta = payload.get("meta", {})
    lines = [f"# gfx950 tile sweep: {meta.get('device', '?')}, timing: {meta.get('timing', '?')}"]
    for r in payload.get("results", []):
        key = result_key(r)
        name = f" ({r['workload']})" if r.get("workload") else ""
        lines.append(f"[{key}]{name} sm_scale={_f(r.get('sm_scale'), '.5f')} best={r['best_config']['BLOCK_M']}x"
                     f"{r['best_config']['BLOCK_N']} default={r.get('library_default')} -- {r.get('choice', '')}")
        cells = []
        for c in sorted(r["candidates"], key=lambda c: (c.get("avg_us") is None, c.get("avg_us") or 0)):
            cfg = c["config"]
            cells.append(f"{cfg['BLOCK_M']}x{cfg['BLOCK_N']}/wg{cfg.get('WG_PER_CU', '?')}="
                         + (_f(c.get("avg_us"), ".2f") + "us" if c.get("avg_us") is not None else "error"))
        lines.append("  candidates: " + ", ".join(cells))
        lines.append(f"  best per-call {_f(r.get('percall_avg_us'), '.1f')} us; vendor {r.get('baseline_op', 'n/a')} "
                     f"{_f(r.get('baseline_avg_us'), '.1f')} us back to back, speedup "
                     f"{_f(r.get('speedup_vs_baseline'), '.2f')}x, max_abs_diff {_f(r.get('max_abs_diff'), '.2e')}")
        for tag, k in (r.get("counters") or {}).items():
            lines.append(f"  counters {tag}: kernel {_f(k.get('kernel_us'), '.2f')} us, MfmaUtil "
                         f"{_f(k.get('MfmaUtil(%)'), '.1f')}%, VALU/MFMA {_f(k.get('valu_per_mfma'), '.2f')}, "
                         f"LDS conflicts {_f(k.get('LDSBankConflict(%)'), '.2f')}%, L2 hit "
                         f"{_f(k.get('l2_hit_rate'), '.3f')}, L2-miss read/write "
                         f"{_f((k.get('l2_miss_read_bytes') or 0) / 1e6 if 'l2_miss_read_bytes' in k else None, '.1f')}/"
                         f"{_f((k.get('l2_miss_write_bytes') or 0) / 1e6 if 'l2_miss_write_bytes' in k else None, '.1f')}"
                         f" MB, {_f(k.get('achieved_GBps'), '.0f')} GB/s")
    return "\n".join(lines) + "\n"


# --------------------------------------------------------------------------
# CLI

def main(argv=None):
    ap = argparse.ArgumentParser(description="Tune BLOCK_M/BLOCK_N per shape on gfx950 and apply the presets.")
    ap.add_argument("--candidate-module", default=str(E.MODULE_PATH))
    ap.add_argument("--output-json", default=str(DEFAULT_OUTPUT_JSON))
    ap.add_argument("--summary-txt", help="also write the per-case summary text here")
    ap.add_argument("--sm-scale", type=float, default=DEFAULTS["sm_scale"])
    ap.add_argument("--seed", type=int, default=DEFAULTS["seed"])
    ap.add_argument("--dtype", default="float16", choices=["float16", "fp16", "bfloat16", "bf16"],
                    help="dtype of the --shape cases")
    ap.add_argument("--suite", default="all", choices=["all", "evaluator", "configs"],
                    help="default cases when no --shape is given")
    ap.add_argument("--warmup-seconds", type=float, default=DEFAULTS["warmup_seconds"])
    ap.add_argument("--rounds", type=int, default=DEFAULTS["rounds"])
    ap.add_argument("--launches", type=int, default=DEFAULTS["launches"], help="timed launches per round")
    ap.add_argument("--final-iters", type=int, default=DEFAULTS["final_iters"], help="per-call timing iterations")
    ap.add_argument("--tie-pct", type=float, default=DEFAULTS["tie_pct"])
    ap.add_argument("--graph-below-us", type=float, default=DEFAULTS["graph_below_us"],
                    help="rank by HIP-graph replays when the fastest eager launch is shorter than this")
    ap.add_argument("--replace-output", action="store_true")
    ap.add_argument("--shape", action="append", help="Z,H,N_CTX,HEAD_DIM,causal (repeatable)")
    ap.add_argument("--skip-apply", action="store_true")
    ap.add_argument("--apply-only", action="store_true")
    ap.add_argument("--merge", nargs="+", help="merge these tuned JSON files (later ones win) into --output-json")
    ap.add_argument("--profile", action="store_true", help="attach rocprofv3 counters for the top two configs")
    ap.add_argument("--profile-dir", help="where the rocprofv3 passes write (default: a temporary directory)")
    ap.add_argument("--run-plan", help=argparse.SUPPRESS)
    ap.add_argument("--manifest", help=argparse.SUPPRESS)
    args = ap.parse_args(argv)
    if args.launches < 1 or args.rounds < 1:
        ap.error("--launches and --rounds must be >= 1")
    module_path = Path(args.candidate_module).resolve()
    out_path = Path(args.output_json).resolve()
    if args.run_plan:
        run_plan(Path(args.run_plan), Path(args.manifest) if args.manifest else None)
        return None
    if args.merge:
        payload = {}
        for path in args.merge:
            payload = merge_payloads(payload, json.loads(Path(path).read_text(encoding="utf-8")))
        out_path.write_text(json.dumps(payload, indent=2, ensure_ascii=True) + "\n", encoding="utf-8")
        if args.summary_txt:
            Path(args.summary_txt).write_text(summary_text(payload))
        if not args.skip_apply:
            apply_presets(module_path, out_path)
        return payload
    if args.apply_only:
        apply_presets(module_path, out_path)
        print(f"Applied tuned presets from {out_path} to {module_path}")
        return None
    module = E.load_candidate(module_path)
    vendor = E.VendorAttention()
    if args.shape:
        dtype = E.dtype_from_name(args.dtype)
        cases = [Case(parse_shape(s), dtype, args.sm_scale, args.seed) for s in args.shape]
    else:
        cases = default_cases(args.suite, args.sm_scale, args.seed)
    results = []
    for i, case in enumerate(cases, start=1):
        print(f"[{i}/{len(cases)}] tuning {case.key}" + (f" ({case.workload})" if case.workload else ""), flush=True)
        r = tune_case(module, vendor, case, args)
        r["seed"] = case.seed
        sp = r["speedup_vs_baseline"]
        print(f"  best: config={r['best_config']}, candidate_avg_us={r['candidate_avg_us']:.3f} ({r['choice']}), "
              f"baseline_avg_us={r['baseline_avg_us'] if r['baseline_avg_us'] is None else round(r['baseline_avg_us'], 3)}, "
              f"speedup={sp if sp is None else round(sp, 3)}", flush=True)
        results.append(r)
    if args.profile:
        prof_dir = Path(args.profile_dir) if args.profile_dir else Path(tempfile.mkdtemp(prefix="fa_tune_prof_"))
        print(f"profiling the top configurations under rocprofv3 into {prof_dir}", flush=True)
        profile_results(results, prof_dir)
    payload = {"meta": {"candidate_module": str(module_path.relative_to(PACKAGE_DIR.parent))
                        if module_path.is_relative_to(PACKAGE_DIR.parent) else str(module_path),
                        "dtypes": sorted({r["dtype"] for r in results}), "seed": args.seed,
                        "timing": (f">= {args.warmup_seconds:g} s warmup, then {args.rounds} rounds x "
                                   f"{args.launches} back-to-back launches between HIP events per candidate "
                                   "(interleaved, median of rounds); per-call perf_counter+synchronize "
                                   f"over {args.final_iters} calls as percall_*"),
                        "tie_pct": args.tie_pct,
                        "device": torch.cuda.get_device_name(0),
                        "baseline_op": "PyTorch-ROCm scaled_dot_product_attention (flash, else memory-efficient)"},
               "tuned_configs": {shape_key((r["Z"], r["H"], r["N_CTX"], r["HEAD_DIM"], r["causal"]),
                                           E.dtype_from_name(r["dtype"])): r["best_config"] for r in results},
               "results": results}
    if not args.replace_output:
        payload = merge_with_existing(out_path, payload)
    out_path.write_text(json.dumps(payload, indent=2, ensure_ascii=True) + "\n", encoding="utf-8")
    print(f"Tuned config JSON written to: {out_path}")
    if args.summary_txt:
        Path(args.summary_txt).write_text(summary_text(payload))
    if not args.skip_apply:
        apply_presets(module_path, out_path)
        print(f"Applied tuned presets to: {module_path}")
    return payload


if __name__ == "__main__":
    main()
