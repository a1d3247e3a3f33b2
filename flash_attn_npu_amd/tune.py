"""gfx950 tiling tuner: the counterpart of tune_flash_attention_forward.py.

For each shape (default: the evaluator's performance shapes) it times every
(BLOCK_M, BLOCK_N) that the library has a kernel for at that head dim, dtype
and causal flag (`fa.kernel_table()`), re-times the winner next to the
vendor baseline (PyTorch-ROCm fused SDPA, as in flash_attn_npu_amd/evaluate.py),
and writes the reference's JSON schema (flash_attention_forward_tuned.json):

    {"meta": {...},
     "tuned_configs": {"Z:H:N_CTX:HEAD_DIM:causal": {"BLOCK_M": .., "BLOCK_N": .., "WAVES": ..}},
     "results": [{shape, best_config, candidate_*_us, baseline_*_us, speedup_vs_baseline,
                  max_abs_diff, correctness_error, candidates: [...], counters: {...}}]}

then rewrites the DEFAULT_TILING_PRESETS block of the module between the
same BEGIN/END markers (tune_flash_attention_forward.py:20-21, :327-366).

With --profile, each shape's winner and runner-up are also run under the
rocprofv3 counter passes of flash_attn_npu_amd/rocprof.py (one process per
pass), and the JSON records the counters that justify the choice (MFMA
utilisation, LDS bank conflicts, L2 hit rate, kernel time).

    python -m flash_attn_npu_amd.tune --dtype bf16 [--shape 4,32,2048,128,1] [--profile]
"""

from __future__ import annotations

import argparse
import json
import statistics
import subprocess
import sys
import tempfile
import time
from pathlib import Path

import torch

from flash_attn_npu_amd import evaluate as E
from flash_attn_npu_amd import workloads as W

PRESET_BEGIN = "# BEGIN AUTO-TUNED DEFAULT TILING PRESETS"
PRESET_END = "# END AUTO-TUNED DEFAULT TILING PRESETS"
PACKAGE_DIR = Path(__file__).resolve().parent
DEFAULT_OUTPUT_JSON = PACKAGE_DIR / "flash_attention_forward_tuned.json"
DEFAULTS = dict(sm_scale=W.REFERENCE_SM_SCALE, seed=0, tune_iters=3, final_iters=5)


def shape_key(shape) -> str:
    z, h, n, d, causal = shape
    return f"{z}:{h}:{n}:{d}:{int(bool(causal))}"


def parse_shape(text: str):
    parts = [p.strip() for p in text.split(",")]
    if len(parts) != 5:
        raise ValueError(f"shape must be Z,H,N_CTX,HEAD_DIM,causal: {text!r}")
    causal = parts[4].lower() in ("1", "true", "yes")
    return (int(parts[0]), int(parts[1]), int(parts[2]), int(parts[3]), causal)


def tiling_candidates(module, shape, dtype):
    """(BLOCK_M, BLOCK_N, waves) of every kernel for this head dim / dtype / causal."""
    d, causal = shape[3], bool(shape[4])
    dt = E.dtype_name(dtype)
    seen, out = set(), []
    for row in module.kernel_table():
        if row["HEAD_DIM"] != d or row["dtype"] != dt or bool(row["causal"]) != causal:
            continue
        key = (row["BLOCK_M"], row["BLOCK_N"])
        if key not in seen:
            seen.add(key)
            out.append((row["BLOCK_M"], row["BLOCK_N"], row["waves"]))
    return out


def time_calls(fn, iters):
    fn()
    torch.cuda.synchronize()
    samples = []
    out = None
    for _ in range(iters):
        t0 = time.perf_counter()
        out = fn()
        torch.cuda.synchronize()
        samples.append((time.perf_counter() - t0) * 1e6)
    return out, {"avg_us": statistics.mean(samples), "min_us": min(samples), "max_us": max(samples),
                 "samples_us": samples, "iters": iters}


def profile_config(shape, dtype, bm, bn, sm_scale, seed):
    """rocprofv3 counter passes over a child process that runs one config."""
    from flash_attn_npu_amd import rocprof
    with tempfile.TemporaryDirectory(prefix="fa_tune_prof_") as tmp:
        cmd = [sys.executable, "-m", "flash_attn_npu_amd.tune", "--run-one", ",".join(str(int(x)) for x in shape),
               "--dtype", E.dtype_name(dtype), "--bm", str(bm), "--bn", str(bn), "--sm-scale", str(sm_scale),
               "--seed", str(seed)]
        plan = {k: rocprof.METRIC_PLAN[k] for k in ("KernelTrace", "Compute", "LDS", "L2")}
        summary = rocprof.run_passes(Path(tmp), cmd, plan)
    k = {name: entry.get("kernel", {}) for name, entry in summary.items()}
    return {"kernel_us": k.get("KernelTrace", {}).get("Duration(us)"),
            "MfmaUtil(%)": k.get("Compute", {}).get("MfmaUtil(%)"),
            "LDSBankConflict(%)": k.get("LDS", {}).get("LDSBankConflict(%)"),
            "l2_hit_rate": summary.get("L2", {}).get("l2", {}).get("Hit Rate")}


def tune_case(module, vendor, shape, dtype, sm_scale, seed, tune_iters, final_iters, profile=False):
    z, h, n, d, causal = shape
    q, k, v = E.make_case_inputs(module.DEVICE, dtype, shape, seed)
    rows = []
    for bm, bn, waves in tiling_candidates(module, shape, dtype):
        try:
            _, st = time_calls(lambda: module._launch_kernel(q, k, v, causal, sm_scale, bm=bm, bn=bn)[0], tune_iters)
            rows.append({"config": {"BLOCK_M": bm, "BLOCK_N": bn, "WAVES": waves}, "avg_us": st["avg_us"],
                         "min_us": st["min_us"], "max_us": st["max_us"]})
        except Exception as exc:  # noqa: BLE001 - recorded per candidate, as the reference does
            rows.append({"config": {"BLOCK_M": bm, "BLOCK_N": bn, "WAVES": waves}, "avg_us": None,
                         "error": str(exc).splitlines()[0][:240] if str(exc) else type(exc).__name__})
    viable = sorted((r for r in rows if r.get("avg_us") is not None), key=lambda r: r["avg_us"])
    if not viable:
        raise RuntimeError(f"no viable config for shape {shape}")
    best = viable[0]["config"]
    bm, bn = best["BLOCK_M"], best["BLOCK_N"]
    cand_out, cand = time_calls(lambda: module._launch_kernel(q, k, v, causal, sm_scale, bm=bm, bn=bn)[0],
                                final_iters)
    result = {"Z": z, "H": h, "N_CTX": n, "HEAD_DIM": d, "causal": bool(causal), "best_config": best,
              "candidate_avg_us": cand["avg_us"], "candidate_min_us": cand["min_us"],
              "candidate_max_us": cand["max_us"], "baseline_avg_us": None, "baseline_min_us": None,
              "baseline_max_us": None, "speedup_vs_baseline": None, "max_abs_diff": None,
              "correctness_error": None, "candidates": rows}
    try:
        ref_out, base = time_calls(lambda: vendor(q, k, v, causal, sm_scale), final_iters)
        result.update(baseline_avg_us=base["avg_us"], baseline_min_us=base["min_us"],
                      baseline_max_us=base["max_us"], speedup_vs_baseline=base["avg_us"] / cand["avg_us"],
                      baseline_op=vendor.used.get(tuple(q.shape) + (bool(causal),)))
        result["max_abs_diff"] = torch.max(torch.abs(cand_out.float() - ref_out.to(dtype).float())).item()
    except Exception as exc:  # noqa: BLE001
        result["correctness_error"] = str(exc)
    if profile:
        result["counters"] = {}
        for r in viable[:2]:
            c = r["config"]
            tag = f"{c['BLOCK_M']}x{c['BLOCK_N']}"
            try:
                result["counters"][tag] = profile_config(shape, dtype, c["BLOCK_M"], c["BLOCK_N"], sm_scale, seed)
            except Exception as exc:  # noqa: BLE001 - the profiler is optional evidence
                result["counters"][tag] = {"error": str(exc)[:240]}
    del q, k, v, cand_out
    torch.cuda.empty_cache()
    return result


def merge_with_existing(path: Path, payload: dict) -> dict:
    if not path.exists():
        return payload
    try:
        old = json.loads(path.read_text(encoding="utf-8"))
    except (OSError, ValueError):
        return payload
    configs = dict(old.get("tuned_configs", {}))
    configs.update(payload["tuned_configs"])
    results, order = {}, []
    for item in list(old.get("results", [])) + list(payload["results"]):
        if not isinstance(item, dict):
            continue
        key = shape_key((item["Z"], item["H"], item["N_CTX"], item["HEAD_DIM"], item["causal"]))
        if key not in order:
            order.append(key)
        results[key] = item
    return dict(payload, tuned_configs=configs, results=[results[k] for k in order])


def presets_block(tuned_configs: dict) -> str:
    lines = [PRESET_BEGIN,
             "# (Z, H, N_CTX, HEAD_DIM, causal) -> (BLOCK_M, BLOCK_N), rewritten by",
             "# python -m flash_attn_npu_amd.tune from gfx950 sweeps.",
             "DEFAULT_TILING_PRESETS = {"]
    for key, cfg in sorted(tuned_configs.items(), key=lambda kv: tuple(int(p) for p in kv[0].split(":"))):
        z, h, n, d, c = (int(p) for p in key.split(":"))
        lines.append(f"    ({z}, {h}, {n}, {d}, {bool(c)}): ({int(cfg['BLOCK_M'])}, {int(cfg['BLOCK_N'])}),")
    lines += ["}", PRESET_END]
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


def run_one(args):
    """Child of --profile: a few launches of one config (what rocprofv3 records)."""
    module = E.load_candidate(Path(args.candidate_module))
    shape = parse_shape(args.run_one)
    dtype = E.dtype_from_name(args.dtype)
    q, k, v = E.make_case_inputs(module.DEVICE, dtype, shape, args.seed)
    for _ in range(5):
        module._launch_kernel(q, k, v, shape[4], args.sm_scale, bm=args.bm, bn=args.bn)
    torch.cuda.synchronize()


def main(argv=None):
    ap = argparse.ArgumentParser(description="Tune BLOCK_M/BLOCK_N per shape on gfx950 and apply the presets.")
    ap.add_argument("--candidate-module", default=str(E.MODULE_PATH))
    ap.add_argument("--output-json", default=str(DEFAULT_OUTPUT_JSON))
    ap.add_argument("--sm-scale", type=float, default=DEFAULTS["sm_scale"])
    ap.add_argument("--seed", type=int, default=DEFAULTS["seed"])
    ap.add_argument("--dtype", default="float16", choices=["float16", "fp16", "bfloat16", "bf16"])
    ap.add_argument("--tune-iters", type=int, default=DEFAULTS["tune_iters"])
    ap.add_argument("--final-iters", type=int, default=DEFAULTS["final_iters"])
    ap.add_argument("--replace-output", action="store_true")
    ap.add_argument("--shape", action="append", help="Z,H,N_CTX,HEAD_DIM,causal (repeatable)")
    ap.add_argument("--skip-apply", action="store_true")
    ap.add_argument("--apply-only", action="store_true")
    ap.add_argument("--profile", action="store_true", help="attach rocprofv3 counters for the top two configs")
    ap.add_argument("--run-one", help=argparse.SUPPRESS)
    ap.add_argument("--bm", type=int, help=argparse.SUPPRESS)
    ap.add_argument("--bn", type=int, help=argparse.SUPPRESS)
    args = ap.parse_args(argv)
    module_path = Path(args.candidate_module).resolve()
    out_path = Path(args.output_json).resolve()
    if args.run_one:
        run_one(args)
        return None
    if args.apply_only:
        apply_presets(module_path, out_path)
        print(f"Applied tuned presets from {out_path} to {module_path}")
        return None
    module = E.load_candidate(module_path)
    dtype = E.dtype_from_name(args.dtype)
    vendor = E.VendorAttention()
    shapes = [parse_shape(s) for s in args.shape] if args.shape else list(W.REFERENCE_PERFORMANCE_CASES)
    results = []
    for i, shape in enumerate(shapes, start=1):
        print(f"[{i}/{len(shapes)}] tuning shape={shape}", flush=True)
        r = tune_case(module, vendor, shape, dtype, args.sm_scale, args.seed, args.tune_iters, args.final_iters,
                      args.profile)
        sp = r["speedup_vs_baseline"]
        print(f"  best: config={r['best_config']}, candidate_avg_us={r['candidate_avg_us']:.3f}, "
              f"baseline_avg_us={r['baseline_avg_us'] if r['baseline_avg_us'] is None else round(r['baseline_avg_us'], 3)}, "
              f"speedup={sp if sp is None else round(sp, 3)}", flush=True)
        results.append(r)
    payload = {"meta": {"candidate_module": str(module_path), "dtype": E.dtype_name(dtype), "sm_scale": args.sm_scale,
                        "seed": args.seed, "tune_iters": args.tune_iters, "final_iters": args.final_iters,
                        "device": torch.cuda.get_device_name(0),
                        "baseline_op": "PyTorch-ROCm scaled_dot_product_attention (flash, else memory-efficient)"},
               "tuned_configs": {shape_key((r["Z"], r["H"], r["N_CTX"], r["HEAD_DIM"], r["causal"])): r["best_config"]
                                 for r in results},
               "results": results}
    if not args.replace_output:
        payload = merge_with_existing(out_path, payload)
    out_path.write_text(json.dumps(payload, indent=2, ensure_ascii=True) + "\n", encoding="utf-8")
    print(f"Tuned config JSON written to: {out_path}")
    if not args.skip_apply:
        apply_presets(module_path, out_path)
        print(f"Applied tuned presets to: {module_path}")
    return payload


if __name__ == "__main__":
    main()
