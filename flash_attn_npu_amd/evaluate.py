"""ROCm counterpart of the reference evaluator (evaluate_attention.py).

Loads a candidate module by path, exactly as the reference does
(evaluate_attention.py:55-59), and runs the same two suites with the same
seeds (`seed + idx`), tolerances, paired alternating timing and scoring:

* correctness: the 18 shapes of evaluate_attention.py:15-34, each compared
  with `allclose(atol, rtol)` against the fp32 formula of
  evaluate_attention.py:134-143 computed on the device (the reference's own
  fallback when its vendor op is unavailable, :150-155), in chunks of heads so
  that no scores tensor exceeds ~2 GiB;
* performance: the 6 shapes of :36-43.  The reference times its candidate
  against the vendor op `torch_npu.npu_fusion_attention`; here the vendor op
  is PyTorch-ROCm's own fused attention (scaled_dot_product_attention pinned
  to the flash backend, else the memory-efficient one; never the math
  backend, whose bf16 batched products are not safe on this platform).  The
  score formula is the reference's: 10 * min(baseline / candidate, 1) points
  per case when the outputs match.

A third suite, `configs`, runs the five benchmark workloads
(flash_attn_npu_amd/workloads.py) against a float64 device restatement with
the workloads' accuracy gates (O <= 5e-3 fp16 / 2e-2 bf16, LSE <= 1e-3).

Reports: `evaluation_report.json` / `.txt` in --report-dir with the reference
schema (evaluate_attention.py:425-507); the `configs` suite adds one key.

    python -m flash_attn_npu_amd.evaluate --dtype bf16 --report-dir evaluation_reports
"""

from __future__ import annotations

import argparse
import importlib.util
import json
import math
import statistics
import time
from pathlib import Path

import torch

from flash_attn_npu_amd import workloads as W

CORRECTNESS_CASES = W.REFERENCE_CORRECTNESS_CASES
PERFORMANCE_CASES = W.REFERENCE_PERFORMANCE_CASES
CORRECTNESS_TOTAL_POINTS = 40.0
PERFORMANCE_TOTAL_POINTS = 60.0
DEFAULTS = dict(sm_scale=W.REFERENCE_SM_SCALE, atol=W.REFERENCE_ATOL, rtol=W.REFERENCE_RTOL,
                warmup=5, iters=30, speed_metric="median_us", trim_ratio=0.1)
MODULE_PATH = Path(__file__).resolve().with_name("flash_attention_forward.py")


# --------------------------------------------------------------------------
# inputs, candidate, references

def load_candidate(path: Path):
    spec = importlib.util.spec_from_file_location("flash_attention_candidate", path)
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module


def dtype_from_name(name: str):
    key = name.strip().lower()
    table = {"float16": torch.float16, "fp16": torch.float16, "bfloat16": torch.bfloat16, "bf16": torch.bfloat16}
    if key not in table:
        raise ValueError(f"Unsupported dtype: {name}")
    return table[key]


def dtype_name(dtype) -> str:
    return {torch.float16: "float16", torch.bfloat16: "bfloat16"}.get(dtype, str(dtype))


def make_case_inputs(device, dtype, shape, seed):
    """N(0, 0.5) q, k, v drawn on the device after torch.manual_seed(seed), as :90-95."""
    z, h, n_ctx, head_dim = shape[:4]
    torch.manual_seed(seed)
    return tuple(torch.empty((z, h, n_ctx, head_dim), dtype=dtype, device=device).normal_(mean=0.0, std=0.5)
                 for _ in range(3))


def formula_attention(q, k, v, causal: bool, sm_scale: float, max_scores_bytes: int = 2 << 30):
    """softmax(scale * Q K^T + causal mask) V in fp32, cast to q.dtype (:134-143).

    Heads are processed in chunks so that one fp32 scores tensor stays below
    `max_scores_bytes`; K^T is made contiguous before the batched product.
    """
    B, H, S, D = q.shape
    Sk = k.shape[2]
    flat = B * H
    qf, kf, vf = (t.reshape(flat, -1, D) for t in (q, k, v))
    out = torch.empty((flat, S, D), dtype=q.dtype, device=q.device)
    rows = max(1, min(S, max_scores_bytes // (4 * Sk)))
    mask = torch.triu(torch.ones((S, Sk), dtype=torch.bool, device=q.device), diagonal=1) if causal else None
    for i in range(flat):
        kt = kf[i].float().t().contiguous()
        vs = vf[i].float()
        for r0 in range(0, S, rows):
            r1 = min(S, r0 + rows)
            s = torch.matmul(qf[i, r0:r1].float(), kt) * sm_scale
            if mask is not None:
                s = s.masked_fill(mask[r0:r1], float("-inf"))
            out[i, r0:r1] = torch.matmul(torch.softmax(s, dim=-1, dtype=torch.float32), vs).to(q.dtype)
    return out.reshape(B, H, S, D)


class VendorAttention:
    """PyTorch-ROCm fused attention as the timing baseline (the vendor op's role)."""

    def __init__(self):
        from torch.nn.attention import SDPBackend
        self.order = [("torch_sdpa_flash", SDPBackend.FLASH_ATTENTION),
                      ("torch_sdpa_efficient", SDPBackend.EFFICIENT_ATTENTION)]
        self.used = {}

    def __call__(self, q, k, v, causal: bool, sm_scale: float):
        import torch.nn.functional as F
        from torch.nn.attention import sdpa_kernel
        errors = []
        for name, backend in self.order:
            try:
                with sdpa_kernel([backend]):
                    out = F.scaled_dot_product_attention(q, k, v, is_causal=causal, scale=sm_scale)
                self.used[tuple(q.shape) + (causal,)] = name
                return out
            except RuntimeError as exc:  # backend not built for this GPU/shape
                errors.append(f"{name}: {exc}")
        raise RuntimeError("no fused PyTorch attention backend: " + " | ".join(errors))


def candidate_attention(module, q, k, v, causal, sm_scale):
    return module.attention(q, k, v, causal, sm_scale).to(q.dtype)


# --------------------------------------------------------------------------
# timing and statistics (same statistics and keys as :186-264)

def _quantile(sorted_values, frac):
    if len(sorted_values) == 1:
        return float(sorted_values[0])
    pos = (len(sorted_values) - 1) * frac
    lo, hi = math.floor(pos), math.ceil(pos)
    return float(sorted_values[lo] + (sorted_values[hi] - sorted_values[lo]) * (pos - lo))


def summarize_samples(samples_us, trim_ratio):
    if not samples_us:
        return None
    xs = sorted(float(x) for x in samples_us)
    trim = min(int(len(xs) * trim_ratio), max((len(xs) - 1) // 2, 0))
    kept = xs[trim:len(xs) - trim] if trim else xs
    avg = statistics.mean(xs)
    std = statistics.pstdev(xs) if len(xs) > 1 else 0.0
    return {"avg_us": avg, "median_us": float(statistics.median(xs)), "trimmed_avg_us": float(statistics.mean(kept)),
            "min_us": xs[0], "max_us": xs[-1], "stddev_us": std, "cv": std / avg if avg else None,
            "p10_us": _quantile(xs, 0.10), "p90_us": _quantile(xs, 0.90), "samples_us": xs}


def measure_pair_us(baseline_fn, candidate_fn, warmup, iters, trim_ratio):
    """Alternating paired wall-clock timing with a synchronize per call (:233-264)."""
    for _ in range(warmup):
        baseline_fn()
        candidate_fn()
    torch.cuda.synchronize()
    samples = {"baseline": [], "candidate": []}
    fns = {"baseline": baseline_fn, "candidate": candidate_fn}
    for idx in range(iters):
        for name in (("baseline", "candidate") if idx % 2 == 0 else ("candidate", "baseline")):
            t0 = time.perf_counter()
            fns[name]()
            torch.cuda.synchronize()
            samples[name].append((time.perf_counter() - t0) * 1e6)
    stats = {}
    for name in samples:
        st = summarize_samples(samples[name], trim_ratio)
        st.update(iters=iters, warmup=warmup)
        stats[name] = st
    return stats["baseline"], stats["candidate"]


def metric_value(stats, metric):
    if not stats:
        return None
    value = stats.get(metric)
    return stats.get("avg_us") if value is None and metric == "median_us" else value


def shape_key(shape):
    z, h, n_ctx, head_dim, causal = shape
    return {"Z": z, "H": h, "N_CTX": n_ctx, "HEAD_DIM": head_dim, "causal": causal}


# --------------------------------------------------------------------------
# suites

@torch.no_grad()
def run_correctness_case(module, device, dtype, shape, sm_scale, seed, atol, rtol):
    q, k, v = make_case_inputs(device, dtype, shape, seed)
    error, passed, diff = None, False, None
    try:
        ref = formula_attention(q, k, v, shape[4], sm_scale)
        out = candidate_attention(module, q, k, v, shape[4], sm_scale)
        diff = torch.max(torch.abs(out.float() - ref.float())).item()
        passed = bool(torch.allclose(ref, out, atol=atol, rtol=rtol))
    except Exception as exc:  # noqa: BLE001 - reported per case, as :310-311
        error = str(exc)
    pts = CORRECTNESS_TOTAL_POINTS / len(CORRECTNESS_CASES) if passed else 0.0
    return {**shape_key(shape), "dtype": dtype_name(dtype), "seed": seed, "atol": atol, "rtol": rtol,
            "passed": passed, "max_abs_diff": diff, "score": pts, "error": error}


@torch.no_grad()
def run_performance_case(module, vendor, device, dtype, shape, sm_scale, seed, atol, rtol, warmup, iters, metric,
                         trim_ratio):
    q, k, v = make_case_inputs(device, dtype, shape, seed)
    causal = shape[4]
    result = {**shape_key(shape), "dtype": dtype_name(dtype), "seed": seed, "atol": atol, "rtol": rtol,
              "output_match": False, "max_abs_diff": None, "baseline": None, "candidate": None,
              "speed_metric": metric, "speedup": None, "score": 0.0, "error": None, "baseline_op": None}
    try:
        ref = vendor(q, k, v, causal, sm_scale).to(dtype)
        result["baseline_op"] = vendor.used.get(tuple(q.shape) + (causal,))
        out = candidate_attention(module, q, k, v, causal, sm_scale)
        result["max_abs_diff"] = torch.max(torch.abs(out.float() - ref.float())).item()
        result["output_match"] = bool(torch.allclose(ref, out, atol=atol, rtol=rtol))
        if result["output_match"]:
            base, cand = measure_pair_us(lambda: vendor(q, k, v, causal, sm_scale),
                                         lambda: candidate_attention(module, q, k, v, causal, sm_scale),
                                         warmup, iters, trim_ratio)
            result["baseline"], result["candidate"] = base, cand
            b, c = metric_value(base, metric), metric_value(cand, metric)
            if b is not None and c:
                result["speedup"] = b / c
                result["score"] = PERFORMANCE_TOTAL_POINTS / len(PERFORMANCE_CASES) * min(max(b / c, 0.0), 1.0)
    except Exception as exc:  # noqa: BLE001
        result["error"] = str(exc)
    return result


def formula_attention_fp64(q, k, v, causal: bool, sm_scale: float, heads_per_chunk: int = 8):
    """The same formula in float64 with its logsumexp: (O, LSE) on q's device."""
    B, H, S, D = q.shape
    Sk = k.shape[2]
    qf, kf, vf = (t.reshape(B * H, -1, D) for t in (q, k, v))
    out = torch.empty((B * H, S, D), dtype=torch.float64, device=q.device)
    lse = torch.empty((B * H, S), dtype=torch.float64, device=q.device)
    mask = torch.triu(torch.ones((S, Sk), dtype=torch.bool, device=q.device), diagonal=1) if causal else None
    for i in range(0, B * H, heads_per_chunk):
        j = min(B * H, i + heads_per_chunk)
        s = torch.bmm(qf[i:j].double(), kf[i:j].double().transpose(1, 2).contiguous()) * sm_scale
        if mask is not None:
            s = s.masked_fill(mask, float("-inf"))
        lse[i:j] = torch.logsumexp(s, dim=-1)
        out[i:j] = torch.bmm(torch.softmax(s, dim=-1), vf[i:j].double().contiguous())
        del s
    return out.reshape(B, H, S, D), lse.reshape(B, H, S)


@torch.no_grad()
def run_config_case(module, w: W.Workload):
    """One benchmark workload against the float64 formula (all heads)."""
    q, k, v = W.make_inputs(w, device="cuda")
    out, lse = module.attention(q, k, v, w.causal, w.sm_scale, return_lse=True)
    o64, l64 = formula_attention_fp64(q, k, v, w.causal, w.sm_scale)
    d_o = (out.float() - o64.to(w.dtype).float()).abs().max().item()
    d_l = (lse.double() - l64).abs().max().item()
    return {"workload": w.name, "shape": [w.B, w.H, w.S, w.D], "causal": w.causal, "dtype": dtype_name(w.dtype),
            "seed": w.seed, "max_abs_diff_o": d_o, "max_abs_diff_lse": d_l, "o_tolerance": w.tolerance,
            "lse_tolerance": 1e-3, "passed": d_o <= w.tolerance and d_l <= 1e-3}


# --------------------------------------------------------------------------
# reports (same JSON keys and text lines as :425-507)

def _fmt(value, precision=3):
    if value is None:
        return "n/a"
    if isinstance(value, bool):
        return str(value)
    if isinstance(value, (int, float)):
        return str(value) if not math.isfinite(float(value)) else f"{value:.{precision}f}"
    return str(value)


def write_reports(report_root: Path, summary: dict):
    report_root.mkdir(parents=True, exist_ok=True)
    json_path, txt_path = report_root / "evaluation_report.json", report_root / "evaluation_report.txt"
    json_path.write_text(json.dumps(summary, indent=2, ensure_ascii=True))
    cfg = summary["config"]
    lines = ["Evaluation Summary", "==================",
             f"candidate_module={cfg['candidate_module']}",
             f"dtype={cfg['dtype']}, sm_scale={cfg['sm_scale']}",
             f"performance_metric={cfg['speed_metric']}, trim_ratio={cfg['trim_ratio']}, warmup={cfg['warmup']}, "
             f"iters={cfg['iters']}",
             "correctness_score={} / {}, performance_score={} / {}, total_score={} / 100".format(
                 _fmt(summary["correctness"]["score"]), _fmt(summary["correctness"]["max_score"]),
                 _fmt(summary["performance"]["score"]), _fmt(summary["performance"]["max_score"]),
                 _fmt(summary["total_score"])),
             "", "Correctness Cases", "-----------------"]
    for i, c in enumerate(summary["correctness"]["cases"], start=1):
        lines.append(f"[{i}] shape=({c['Z']},{c['H']},{c['N_CTX']},{c['HEAD_DIM']}, causal={c['causal']}) "
                     f"passed={c['passed']} score={_fmt(c['score'])} max_abs_diff={_fmt(c['max_abs_diff'], 6)} "
                     f"error={c['error'] or ''}")
    lines += ["", "Performance Cases", "-----------------"]
    for i, c in enumerate(summary["performance"]["cases"], start=1):
        m = c["speed_metric"]
        lines.append(
            f"[{i}] shape=({c['Z']},{c['H']},{c['N_CTX']},{c['HEAD_DIM']}, causal={c['causal']}) "
            f"match={c['output_match']} score={_fmt(c['score'])} baseline_{m}={_fmt(metric_value(c['baseline'], m))} "
            f"candidate_{m}={_fmt(metric_value(c['candidate'], m))} speedup={_fmt(c['speedup'], 4)} "
            f"baseline_cv={_fmt(c['baseline']['cv'] if c['baseline'] else None, 4)} "
            f"candidate_cv={_fmt(c['candidate']['cv'] if c['candidate'] else None, 4)} "
            f"max_abs_diff={_fmt(c['max_abs_diff'], 6)} error={c['error'] or ''}")
    if summary.get("configs"):
        lines += ["", "Benchmark Workloads", "-------------------"]
        for i, c in enumerate(summary["configs"]["cases"], start=1):
            lines.append(f"[{i}] {c['workload']} shape={tuple(c['shape'])} causal={c['causal']} dtype={c['dtype']} "
                         f"passed={c['passed']} max_abs_diff_o={_fmt(c['max_abs_diff_o'], 6)} "
                         f"(tol {c['o_tolerance']}) max_abs_diff_lse={_fmt(c['max_abs_diff_lse'], 6)} (tol 0.001)")
    txt_path.write_text("\n".join(lines).rstrip() + "\n")
    return json_path, txt_path


def build_arg_parser():
    ap = argparse.ArgumentParser(description="Evaluate a flash-attention module on MI355X (correctness, performance).")
    ap.add_argument("--candidate", default=str(MODULE_PATH), help="path to the candidate module")
    ap.add_argument("--mode", choices=["all", "correctness", "performance", "configs"], default="all")
    ap.add_argument("--dtype", default="float16", choices=["float16", "fp16", "bfloat16", "bf16"])
    ap.add_argument("--sm-scale", dest="sm_scale", type=float, default=DEFAULTS["sm_scale"])
    ap.add_argument("--atol", type=float, default=DEFAULTS["atol"])
    ap.add_argument("--rtol", type=float, default=DEFAULTS["rtol"])
    ap.add_argument("--warmup", type=int, default=DEFAULTS["warmup"])
    ap.add_argument("--iters", type=int, default=DEFAULTS["iters"])
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--speed-metric", choices=["avg_us", "median_us", "trimmed_avg_us", "min_us"],
                    default=DEFAULTS["speed_metric"])
    ap.add_argument("--trim-ratio", type=float, default=DEFAULTS["trim_ratio"])
    ap.add_argument("--report-dir", default="evaluation_reports")
    ap.add_argument("--with-configs", action="store_true", help="also run the five benchmark workloads")
    return ap


def main(argv=None):
    args = build_arg_parser().parse_args(argv)
    candidate_path = Path(args.candidate).resolve()
    module = load_candidate(candidate_path)
    dtype = dtype_from_name(args.dtype)
    device = getattr(module, "DEVICE", "cuda")
    vendor = VendorAttention()
    corr, perf, cfgs = [], [], []
    if args.mode in ("all", "correctness"):
        for idx, shape in enumerate(CORRECTNESS_CASES):
            print(f"Running correctness case {idx + 1}/{len(CORRECTNESS_CASES)}: {shape}", flush=True)
            corr.append(run_correctness_case(module, device, dtype, shape, args.sm_scale, args.seed + idx,
                                             args.atol, args.rtol))
            torch.cuda.empty_cache()
    if args.mode in ("all", "performance"):
        offset = len(CORRECTNESS_CASES)
        for idx, shape in enumerate(PERFORMANCE_CASES):
            print(f"Running performance case {idx + 1}/{len(PERFORMANCE_CASES)}: {shape}", flush=True)
            perf.append(run_performance_case(module, vendor, device, dtype, shape, args.sm_scale,
                                             args.seed + offset + idx, args.atol, args.rtol, args.warmup, args.iters,
                                             args.speed_metric, args.trim_ratio))
            torch.cuda.empty_cache()
    if args.mode == "configs" or args.with_configs:
        for w in W.CONFIGS:
            print(f"Running benchmark workload {w.name}", flush=True)
            cfgs.append(run_config_case(module, w))
            torch.cuda.empty_cache()
    valid = [c["speedup"] for c in perf if c["speedup"] is not None]
    correctness = {"total_cases": len(corr), "passed_cases": sum(c["passed"] for c in corr),
                   "points_per_case": CORRECTNESS_TOTAL_POINTS / len(CORRECTNESS_CASES),
                   "score": sum(c["score"] for c in corr), "max_score": CORRECTNESS_TOTAL_POINTS, "cases": corr}
    performance = {"total_cases": len(perf), "matched_cases": sum(c["output_match"] for c in perf),
                   "points_per_case": PERFORMANCE_TOTAL_POINTS / len(PERFORMANCE_CASES),
                   "score": sum(c["score"] for c in perf), "max_score": PERFORMANCE_TOTAL_POINTS,
                   "mean_speedup": statistics.mean(valid) if valid else None,
                   "median_speedup": statistics.median(valid) if valid else None, "cases": perf}
    summary = {
        "config": {"candidate_module": str(candidate_path), "report_dir": str(Path(args.report_dir).resolve()),
                   "dtype": dtype_name(dtype), "sm_scale": args.sm_scale, "atol": args.atol, "rtol": args.rtol,
                   "warmup": args.warmup, "iters": args.iters, "seed": args.seed, "speed_metric": args.speed_metric,
                   "trim_ratio": args.trim_ratio, "device": torch.cuda.get_device_name(0),
                   "baseline_op": "PyTorch-ROCm scaled_dot_product_attention (flash, else memory-efficient backend)",
                   "correctness_reference": "fp32 formula of evaluate_attention.py:134-143 on the device",
                   "scoring": {"correctness_total": CORRECTNESS_TOTAL_POINTS,
                               "performance_total": PERFORMANCE_TOTAL_POINTS,
                               "correctness_points_per_case": CORRECTNESS_TOTAL_POINTS / len(CORRECTNESS_CASES),
                               "performance_points_per_case": PERFORMANCE_TOTAL_POINTS / len(PERFORMANCE_CASES),
                               "performance_formula": "per_case_score = 10 * min(baseline_<metric>_us / "
                                                      "candidate_<metric>_us, 1.0) when output matches"}},
        "correctness": correctness,
        "performance": performance,
        "total_score": correctness["score"] + performance["score"],
    }
    if cfgs:
        summary["configs"] = {"total_cases": len(cfgs), "passed_cases": sum(c["passed"] for c in cfgs), "cases": cfgs}
    json_path, txt_path = write_reports(Path(args.report_dir), summary)
    print(f"Evaluation complete\nJSON report: {json_path}\nText report: {txt_path}")
    print(f"Correctness: {correctness['score']:.3f} / {CORRECTNESS_TOTAL_POINTS:.3f} "
          f"({correctness['passed_cases']}/{correctness['total_cases']} passed)")
    print(f"Performance: {performance['score']:.3f} / {PERFORMANCE_TOTAL_POINTS:.3f} "
          f"({performance['matched_cases']}/{performance['total_cases']} matched, "
          f"mean_speedup={_fmt(performance['mean_speedup'], 4)})")
    if cfgs:
        print(f"Benchmark workloads: {summary['configs']['passed_cases']}/{len(cfgs)} passed")
    print(f"Total score: {_fmt(summary['total_score'])} / 100")
    return summary


if __name__ == "__main__":
    main()
