"""rocprofv3 counter passes and the profile_summary.{json,txt} emitter.

MI355X counterpart of the reference's in-module profiling
(flash_attention_forward.py:255-613, 1204-1296): there, torch_npu's profiler
runs one pass per AiC metric and the CSVs are folded into
`profile_summary.json` / `profile_summary.txt` (write_profile_summary_files,
:436-522), which `compare_results_plus.py` (:274-367) reads.  Here each pass
is a `rocprofv3` subprocess (counters collected in their own runs, at most the
per-block hardware limits per pass), and the result folds into the same
schema, one entry per pass:

    {pass_name: {"profiler_output", "op_name", "op": {...}, "kernel": {...},
                 "kernel_columns": [...], "step": {}, "api": {...},
                 "l2": {...}, "l2_columns": [...]}}

so `python compare_results_plus.py A/profile_summary.json B/profile_summary.json`
compares two MI355X runs unmodified.  The kernel-trace pass also traces the
HIP API, which fills the entry's `step` and `api` sections:

* step: one step per launch of the target kernel, from its start to the next
  launch's start (the last ends with the last kernel).  Computing is the time
  some kernel ran, Free the rest; there are no collectives, so the
  communication, overlap and bubble columns are 0, Stage is the step's span
  and Preparing is 0 (a step begins with its kernel).  Each column is the
  median over steps, so the few long gaps between a benchmark's phases do not
  stand for every step (the reference averages the 30 steps of one loop).
* api: `launch` is the HIP launch call of each target dispatch (matched by
  correlation id), `launch_all` every kernel launch call, and each HIP
  *Synchronize function its own row; the reference's comparison tool prints
  the device-wide synchronisation row under the Ascend runtime's name
  (aclrtSynchronizeDeviceWithTimeout), which here holds hipDeviceSynchronize
  (what torch.cuda.synchronize calls).

    python -m flash_attn_npu_amd.rocprof run --out result_dir -- python3 bench.py --steps 5 --cpu-seconds 0
    python -m flash_attn_npu_amd.rocprof summarize result_dir
"""

from __future__ import annotations

import argparse
import csv
import json
import os
import statistics
import subprocess
import sys
from pathlib import Path

PROFILE_OP_NAME = "fa_fwd"

# One entry per rocprofv3 run.  None = kernel + HIP API trace.  Each counter list
# fits one pass (<= 8 SQ, <= 4 TCC (FETCH_SIZE takes 3, WRITE_SIZE 2), <= 2 GRBM).
METRIC_PLAN = {
    "KernelTrace": None,
    "Compute": ["SQ_WAVES", "SQ_BUSY_CYCLES", "SQ_WAVE_CYCLES", "SQ_INSTS_VALU", "SQ_INSTS_MFMA",
                "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_ACTIVE_INST_VALU", "SQ_INSTS_SALU", "GRBM_GUI_ACTIVE"],
    "LDS": ["SQ_INSTS_LDS", "SQ_LDS_BANK_CONFLICT", "SQ_LDS_IDX_ACTIVE", "SQ_WAIT_INST_LDS",
            "SQ_ACTIVE_INST_LDS", "SQ_VALU_MFMA_COEXEC_CYCLES", "SQ_WAIT_ANY", "SQ_WAIT_INST_ANY"],
    "L2": ["TCC_HIT_sum", "TCC_MISS_sum"],
    # FETCH_SIZE (3 TCC counters) and the memory-side read request count (1 more).
    "HBMRead": ["FETCH_SIZE", "TCC_EA0_RDREQ_DRAM_sum"],
    "HBMWrite": ["WRITE_SIZE"],
}

# gfx950: 256 CUs x 4 SIMDs; one v_mfma_f32_32x32x16 keeps a SIMD's matrix
# core busy for 32 cycles (SQ_VALU_MFMA_BUSY_CYCLES counts those cycles).
NUM_SIMDS = 1024
COPY_BYTES = 256 * 1024 * 1024  # the calibration copy in bench.py --calibrate-copy


def _read_csv(path: Path):
    with path.open(newline="", encoding="utf-8") as f:
        return list(csv.DictReader(f))


def _is_target(name: str, op: str) -> bool:
    return op in name


def _is_copy(name: str) -> bool:
    """The calibration copy (torch's device copy, a copy kernel or the runtime's
    copyBuffer blit); fills and other elementwise kernels of the same process
    read nothing and must not dilute the factor."""
    low = name.lower()
    return "copy" in low and "fill" not in low


def _find(root: Path, suffix: str):
    return sorted(root.rglob(f"*{suffix}"))


def summarize_pass(pass_dir: Path, op: str = PROFILE_OP_NAME) -> dict:
    """Fold one rocprofv3 output directory into one summary entry."""
    entry = {"profiler_output": str(pass_dir), "op_name": op, "op": {}, "kernel": {},
             "kernel_columns": [], "step": {}, "api": {}, "l2": {}, "l2_columns": []}
    traces = _find(pass_dir, "kernel_trace.csv")
    durations, all_total = [], 0.0
    for tr in traces:
        for r in _read_csv(tr):
            d = (float(r["End_Timestamp"]) - float(r["Start_Timestamp"])) / 1e3
            all_total += d
            if _is_target(r["Kernel_Name"], op):
                durations.append(d)
                entry["op"]["OP Type"] = r["Kernel_Name"]
                entry["kernel"]["Block Num"] = float(r["Grid_Size_X"]) / float(r["Workgroup_Size_X"])
                entry["kernel"]["LDS_Block_Size"] = float(r["LDS_Block_Size"])
                entry["kernel"]["VGPR_Count"] = float(r.get("VGPR_Count", 0) or 0)
                entry["kernel"]["Scratch_Size"] = float(r.get("Scratch_Size", 0) or 0)
    if durations:
        entry["op"].update({
            "Core Type": "MI355X gfx950",
            "Count": float(len(durations)),
            "Total Time(us)": sum(durations),
            "Min Time(us)": min(durations),
            "Avg Time(us)": statistics.mean(durations),
            "Max Time(us)": max(durations),
            "Ratio(%)": 100.0 * sum(durations) / all_total if all_total else None,
        })
        entry["kernel"]["Duration(us)"] = statistics.mean(durations)
        entry["kernel"]["kernel_count"] = float(len(durations))

    counters: dict[str, list[float]] = {}
    copy_counters: dict[str, list[float]] = {}
    for cc in _find(pass_dir, "counter_collection.csv"):
        for r in _read_csv(cc):
            dst = counters if _is_target(r["Kernel_Name"], op) else (
                copy_counters if _is_copy(r["Kernel_Name"]) else None)
            if dst is not None:
                dst.setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
    k = entry["kernel"]
    for name, vals in counters.items():
        k[name] = statistics.mean(vals)
        # A counter pass has no durations: count the dispatches sampled.
        k.setdefault("kernel_count", float(len(vals)))
    # Derived figures.
    if "SQ_VALU_MFMA_BUSY_CYCLES" in k and "GRBM_GUI_ACTIVE" in k and k["GRBM_GUI_ACTIVE"]:
        # GRBM_GUI_ACTIVE sums the 8 XCDs' busy cycles.
        k["MfmaUtil(%)"] = 100.0 * k["SQ_VALU_MFMA_BUSY_CYCLES"] / NUM_SIMDS / (k["GRBM_GUI_ACTIVE"] / 8)
    if "SQ_LDS_BANK_CONFLICT" in k and k.get("SQ_LDS_IDX_ACTIVE"):
        k["LDSBankConflict(%)"] = 100.0 * k["SQ_LDS_BANK_CONFLICT"] / k["SQ_LDS_IDX_ACTIVE"]
    for cname, label in (("FETCH_SIZE", "hbm_read_bytes"), ("WRITE_SIZE", "hbm_write_bytes")):
        if cname in k:
            factor = 1.0
            if copy_counters.get(cname):
                factor = COPY_BYTES / (statistics.mean(copy_counters[cname]) * 1024.0)
                k[f"{cname}_copy_factor"] = factor
            k[label] = k[cname] * 1024.0 * factor
    if "TCC_EA0_RDREQ_DRAM_sum" in k and copy_counters.get("TCC_EA0_RDREQ_DRAM_sum"):
        # Second read figure: memory-side read requests times the bytes per
        # request of the calibration copy.
        per_req = COPY_BYTES / statistics.mean(copy_counters["TCC_EA0_RDREQ_DRAM_sum"])
        k["TCC_EA0_RDREQ_DRAM_bytes_per_req"] = per_req
        k["hbm_read_bytes_by_requests"] = k["TCC_EA0_RDREQ_DRAM_sum"] * per_req
    if "TCC_HIT_sum" in k and "TCC_MISS_sum" in k:
        tot = k["TCC_HIT_sum"] + k["TCC_MISS_sum"]
        entry["l2"] = {"l2_count": 1.0, "Hit Rate": k["TCC_HIT_sum"] / tot if tot else None}
        entry["l2_columns"] = ["Hit Rate"]
    entry["kernel_columns"] = [c for c in k if c != "kernel_count"]
    entry["step"] = summarize_steps(pass_dir, op)
    entry["api"] = summarize_api(pass_dir, op)
    return entry


STEP_COLUMNS = ["Computing", "Communication(Not Overlapped)", "Overlapped", "Communication", "Free",
                "Stage", "Bubble", "Communication(Not Overlapped and Exclude Receive)", "Preparing"]
API_COLUMNS = ["Time(us)", "Count", "Avg(us)", "Min(us)", "Max(us)"]
DEVICE_SYNC_KEY = "aclrtSynchronizeDeviceWithTimeout"  # the row name the comparison tool prints


def _kernel_intervals(pass_dir: Path):
    """(name, start_ns, end_ns, correlation id or None) of every dispatch in the pass."""
    out = []
    for tr in _find(pass_dir, "kernel_trace.csv"):
        for r in _read_csv(tr):
            corr = r.get("Correlation_Id")
            out.append((r["Kernel_Name"], float(r["Start_Timestamp"]), float(r["End_Timestamp"]),
                        int(float(corr)) if corr not in (None, "") else None))
    out.sort(key=lambda x: x[1])
    return out


def summarize_steps(pass_dir: Path, op: str = PROFILE_OP_NAME) -> dict:
    """Step Trace columns (us) from the kernel trace; see the module docstring."""
    kernels = _kernel_intervals(Path(pass_dir))
    starts = [s for name, s, _, _ in kernels if _is_target(name, op)]
    if not starts:
        return {}
    last_end = max(e for _, _, e, _ in kernels)
    bounds = starts + [last_end]
    steps = []
    j = 0  # first kernel that may overlap the current step
    for lo, hi in zip(bounds[:-1], bounds[1:]):
        while j < len(kernels) and kernels[j][2] <= lo:
            j += 1
        busy, cur_s, cur_e = 0.0, None, None
        for _, s, e, _ in kernels[j:]:
            if s >= hi:
                break
            s, e = max(s, lo), min(e, hi)
            if e <= s:
                continue
            if cur_e is None or s > cur_e:
                busy += (cur_e - cur_s) if cur_e is not None else 0.0
                cur_s, cur_e = s, e
            else:
                cur_e = max(cur_e, e)
        busy += (cur_e - cur_s) if cur_e is not None else 0.0
        span = hi - lo
        steps.append({"Computing": busy / 1e3, "Free": (span - busy) / 1e3, "Stage": span / 1e3})
    out = {c: 0.0 for c in STEP_COLUMNS}
    for c in ("Computing", "Free", "Stage"):
        out[c] = statistics.median(st[c] for st in steps)
    out["step_count"] = float(len(steps))
    return out


def _api_row(durations_us: list[float]) -> dict:
    return {"Time(us)": sum(durations_us), "Count": float(len(durations_us)),
            "Avg(us)": statistics.mean(durations_us), "Min(us)": min(durations_us),
            "Max(us)": max(durations_us)}


def summarize_api(pass_dir: Path, op: str = PROFILE_OP_NAME) -> dict:
    """API Statistic rows from the HIP API trace; see the module docstring."""
    pass_dir = Path(pass_dir)
    calls: dict[str, list[tuple[int | None, float]]] = {}
    for tr in _find(pass_dir, "hip_api_trace.csv"):
        for r in _read_csv(tr):
            name = r.get("Function") or r.get("Operation") or r.get("Name") or ""
            corr = r.get("Correlation_Id")
            dur = (float(r["End_Timestamp"]) - float(r["Start_Timestamp"])) / 1e3
            calls.setdefault(name, []).append((int(float(corr)) if corr not in (None, "") else None, dur))
    if not calls:
        return {}
    target_corr = {c for name, _, _, c in _kernel_intervals(pass_dir) if _is_target(name, op) and c is not None}
    launch_all, launch_target = [], []
    api = {}
    for name, rows in sorted(calls.items()):
        if "LaunchKernel" in name:
            launch_all += [d for _, d in rows]
            launch_target += [d for c, d in rows if c in target_corr]
            api[name] = _api_row([d for _, d in rows])
        elif "Synchronize" in name:
            api[name] = _api_row([d for _, d in rows])
    if launch_all:
        api["launch_all"] = _api_row(launch_all)
        api["launch"] = _api_row(launch_target) if launch_target else api["launch_all"]
    if "hipDeviceSynchronize" in api:
        api[DEVICE_SYNC_KEY] = dict(api["hipDeviceSynchronize"])
    return api


def _dispatch_key(row: dict, index: int):
    for col in ("Dispatch_Id", "Correlation_Id"):
        val = row.get(col)
        if val not in (None, ""):
            return int(float(val))
    return index


def read_dispatches(pass_dir: Path, match) -> list[dict]:
    """Per-dispatch records of one pass, in dispatch order, for kernels whose name
    satisfies `match(name)`: {"name", "duration_us" (kernel-trace passes),
    "counters": {counter: value}}.

    Counter rows are grouped by Dispatch_Id (rocprofv3 writes one row per
    dispatch and counter); a file without that column is grouped by
    occurrence (the i-th value of a counter belongs to the i-th dispatch).
    """
    by_id: dict[int, dict] = {}
    for tr in _find(Path(pass_dir), "kernel_trace.csv"):
        for i, r in enumerate(_read_csv(tr)):
            if not match(r["Kernel_Name"]):
                continue
            rec = by_id.setdefault(_dispatch_key(r, i), {"name": r["Kernel_Name"], "counters": {}})
            rec["duration_us"] = (float(r["End_Timestamp"]) - float(r["Start_Timestamp"])) / 1e3
    for cc in _find(Path(pass_dir), "counter_collection.csv"):
        seen: dict[str, int] = {}
        for r in _read_csv(cc):
            if not match(r["Kernel_Name"]):
                continue
            name = r["Counter_Name"]
            if "Dispatch_Id" in r or "Correlation_Id" in r:
                key = _dispatch_key(r, 0)
            else:
                key = seen.get(name, 0)
                seen[name] = key + 1
            rec = by_id.setdefault(key, {"name": r["Kernel_Name"], "counters": {}})
            rec["counters"][name] = rec["counters"].get(name, 0.0) + float(r["Counter_Value"])
    return [by_id[k] for k in sorted(by_id)]


def copy_factors(pass_dir: Path) -> dict:
    """Copy calibration of a pass, from the plain device copy in the same process:
    for FETCH_SIZE / WRITE_SIZE (KiB) the factor COPY_BYTES / reading, for the
    memory-side read request count the bytes per request."""
    out = {}
    for rec in read_dispatches(pass_dir, _is_copy):
        for name, val in rec["counters"].items():
            if name in ("FETCH_SIZE", "WRITE_SIZE") and val > 0:
                out.setdefault(name, []).append(COPY_BYTES / (val * 1024.0))
            elif name == "TCC_EA0_RDREQ_DRAM_sum" and val > 0:
                out.setdefault(name, []).append(COPY_BYTES / val)
    return {k: statistics.mean(v) for k, v in out.items()}


BUILD_KEY = "__build__"


def build_stamp(summary_by_metric: dict | None = None) -> dict:
    """Which library the profiled process loaded: its fa_build_id (a hash of the
    kernel sources, host-only call, no GPU needed), its path, and the profiled
    kernel's name from the kernel-trace pass when there is one."""
    from flash_attn_npu_amd import flash_attention_forward as fa

    lib = fa._load_library()
    stamp = {"fa_build_id": lib.fa_build_id().decode(), "library": os.path.basename(str(fa.library_path()))}
    for s in (summary_by_metric or {}).values():
        name = s.get("op", {}).get("OP Type")
        if s.get("op_name") == PROFILE_OP_NAME and name and name != "n/a":
            stamp["kernel_name"] = name
            break
    return stamp


def write_profile_summary_files(root: Path, summary_by_metric: dict, build: dict | None = None):
    """profile_summary.json + profile_summary.txt, as flash_attention_forward.py:436-522.

    `build` (build_stamp()) goes into the JSON under the key "__build__", which
    compare_results_plus.py skips (it compares only keys without a leading
    "__", :492-495, after reading every entry's "kernel" / "l2" dicts, :318-338,
    so the stamp has no key of those names), and into the first line of the
    text summary.
    """
    root = Path(root)
    root.mkdir(parents=True, exist_ok=True)
    json_path = root / "profile_summary.json"
    txt_path = root / "profile_summary.txt"
    data = dict(summary_by_metric)
    if build is not None:
        data[BUILD_KEY] = build
    json_path.write_text(json.dumps(data, indent=2))
    lines = []
    if build is not None:
        lines.append("build: " + ", ".join(f"{k}={v}" for k, v in build.items()))
        lines.append("")
    for metric, s in summary_by_metric.items():
        op = s.get("op", {})
        lines.append(f"[{metric}]")
        lines.append(f"profiler_output={s.get('profiler_output')}")
        lines.append("op: type={}, count={}, avg_us={}, min_us={}, max_us={}, ratio_pct={}".format(
            op.get("OP Type", "n/a"), _fmt(op.get("Count")), _fmt(op.get("Avg Time(us)")),
            _fmt(op.get("Min Time(us)")), _fmt(op.get("Max Time(us)")), _fmt(op.get("Ratio(%)"))))
        if s.get("kernel_columns"):
            lines.append("kernel_metrics: " + ", ".join(
                f"{c}={_fmt(s['kernel'].get(c))}" for c in s["kernel_columns"]))
        step, api = s.get("step", {}), s.get("api", {})
        if step:
            lines.append("step: computing_us={}, free_us={}, bubble_us={}, preparing_us={}".format(
                _fmt(step.get("Computing")), _fmt(step.get("Free")), _fmt(step.get("Bubble")),
                _fmt(step.get("Preparing"))))
        if api:
            lines.append("api: launch_avg_us={}, sync_avg_us={}".format(
                _fmt(api.get("launch", {}).get("Avg(us)")), _fmt(api.get(DEVICE_SYNC_KEY, {}).get("Avg(us)"))))
        if s.get("l2_columns"):
            lines.append("l2_cache: " + ", ".join(f"{c}={_fmt(s['l2'].get(c), 6)}" for c in s["l2_columns"]))
        lines.append("")
    txt_path.write_text("\n".join(lines).rstrip() + "\n")
    return json_path, txt_path


def _fmt(v, precision=3):
    if v is None:
        return "n/a"
    if isinstance(v, str):
        return v
    return f"{v:.{precision}f}"


def run_passes(out: Path, target: list[str], plan=None, timeout=120) -> dict:
    """Run one rocprofv3 process per pass of `plan` over the command `target`."""
    plan = METRIC_PLAN if plan is None else plan
    cwd = Path.cwd()
    out = Path(out).resolve()
    out.mkdir(parents=True, exist_ok=True)
    # The passes run from /tmp: make the command's relative file arguments
    # (e.g. `python3 bench.py`) absolute first.
    target = [str(Path(a).resolve()) if not a.startswith("-") and Path(a).is_file() else a for a in target]
    # The passes run from /tmp (rocprofv3 writes scratch files there); keep
    # this repository importable for a `python -m flash_attn_npu_amd...` target.
    repo = str(Path(__file__).resolve().parent.parent)
    env = dict(os.environ, TMPDIR=os.environ.get("TMPDIR", "/tmp"),
               PYTHONPATH=os.pathsep.join(p for p in (repo, os.environ.get("PYTHONPATH", "")) if p))
    summary = {}
    for name, counters in plan.items():
        pdir = out / name
        cmd = ["rocprofv3"]
        # Traces (kernel + HIP API) and counters never share a run.
        cmd += ["--kernel-trace", "--hip-trace", "--stats"] if counters is None else ["--pmc", *counters]
        cmd += ["-d", str(pdir), "-o", "run", "--output-format", "csv", "--", *target]
        print(f"[rocprof] pass {name}: {' '.join(cmd)}", flush=True)
        proc = subprocess.run(cmd, env=env, cwd="/tmp", timeout=timeout, capture_output=True, text=True)
        (out / f"{name}.log").write_text(proc.stdout + proc.stderr)
        if proc.returncode != 0:
            raise RuntimeError(f"rocprofv3 pass {name} failed ({proc.returncode}); see {out / (name + '.log')}")
        summary[name] = summarize_pass(pdir)
        # Recorded relative to the caller's directory (the passes ran from /tmp).
        summary[name]["profiler_output"] = os.path.relpath(pdir, cwd)
    return summary


def summarize_dir(out: Path, plan=None) -> dict:
    plan = METRIC_PLAN if plan is None else plan
    return {name: summarize_pass(Path(out) / name) for name in plan if (Path(out) / name).exists()}


def read_build_id(summary_txt: Path) -> str | None:
    """The fa_build_id a text summary was stamped with (None if it carries none)."""
    for line in Path(summary_txt).read_text().splitlines():
        if line.startswith("build:"):
            for item in line[len("build:"):].split(","):
                key, _, val = item.strip().partition("=")
                if key == "fa_build_id":
                    return val
    return None


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    r = sub.add_parser("run", help="run every counter pass over a command, then summarize")
    r.add_argument("--out", required=True)
    r.add_argument("--passes", default=",".join(METRIC_PLAN), help="comma-separated subset of the plan")
    r.add_argument("target", nargs=argparse.REMAINDER)
    s = sub.add_parser("summarize", help="fold existing pass directories into profile_summary.*")
    s.add_argument("out")
    args = ap.parse_args(argv)
    if args.cmd == "run":
        target = args.target[1:] if args.target and args.target[0] == "--" else args.target
        if not target:
            ap.error("missing target command after --")
        plan = {k: METRIC_PLAN[k] for k in args.passes.split(",")}
        summary = run_passes(Path(args.out), target, plan)
    else:
        summary = summarize_dir(Path(args.out))
    # The library the target loaded: the one this process resolves the same way
    # (FA_MI355X_LIB or the in-tree build).
    j, t = write_profile_summary_files(Path(args.out), summary, build_stamp(summary))
    print(t.read_text())
    print(f"wrote {j} and {t}")


if __name__ == "__main__":
    sys.exit(main())
