"""CPU: the reference's comparison tool reads this repository's profile summaries.

tests/golden/compare_results/comparison.txt is what compare_results_plus.py
(the reference's tool, run unmodified by tests/golden/make_compare_fixture.py
where the reference tree is mounted) printed for two summaries that
flash_attn_npu_amd.rocprof wrote on an MI355X: config 2 at BLOCK_M x BLOCK_N
128 x 64 and 128 x 32.  The tool prints one section per shared metric (pass)
with op statistics, kernel details, L2, step-trace and API rows
(compare_results_plus.py:438-489); a key the summary lacks prints as n/a.
"""

from __future__ import annotations

import json
import re
from pathlib import Path

from flash_attn_npu_amd import rocprof

HERE = Path(__file__).resolve().parent / "golden" / "compare_results"
ROW = re.compile(r"^(?P<label>.+?)\s+(?P<a>\S+)\s+(?P<b>\S+)\s+(?P<d>\S+)\s+(?P<p>\S+%)(\s+\S+)?$")


def _sections():
    """{metric: {section title: {row label: (a, b)}}} from the printed comparison."""
    out, metric, title = {}, None, None
    lines = (HERE / "comparison.txt").read_text().splitlines()
    for i, line in enumerate(lines):
        nxt = lines[i + 1] if i + 1 < len(lines) else ""
        if line.startswith("Metric: "):
            metric = line[len("Metric: "):]
            out[metric] = {}
            continue
        if nxt and set(nxt) == {"-"} and len(nxt) == len(line):
            title = line
            if metric is not None:
                out[metric][title] = {}
            continue
        m = ROW.match(line)
        if m and metric is not None and title in out[metric] and m["label"] != "metric":
            out[metric][title][m["label"].strip()] = (m["a"], m["b"])
    return out


def _numeric(v):
    return re.fullmatch(r"-?\d+(\.\d+)?", v) is not None


def test_fixture_inputs_are_this_writers_summaries():
    for name in ("config2_128x64", "config2_128x32"):
        data = json.loads((HERE / name / "profile_summary.json").read_text())
        assert set(k for k in data if not k.startswith("__")) == set(rocprof.METRIC_PLAN)
        build = data[rocprof.BUILD_KEY]
        assert re.fullmatch(r"[0-9a-f]{16}", build["fa_build_id"]) and "fa_fwd_dma_kernel<128, " in build["kernel_name"]


def test_tool_compares_every_pass():
    sec = _sections()
    assert set(sec) == set(rocprof.METRIC_PLAN)
    text = (HERE / "comparison.txt").read_text()
    assert "Shared metrics: " + ", ".join(sorted(rocprof.METRIC_PLAN)) in text


def test_kernel_trace_rows_are_all_filled():
    # The kernel-trace pass fills the op, kernel, step and api rows the tool prints.
    kt = _sections()["KernelTrace"]
    for title in ("Op Statistic", "Kernel Details", "Step Trace", "API Statistic"):
        rows = kt[title]
        assert rows, title
        for label, (a, b) in rows.items():
            assert _numeric(a) and _numeric(b), f"{title} / {label}: {a} {b}"
    assert float(kt["Op Statistic"]["Avg Time(us)"][0]) > 0 and float(kt["Step Trace"]["Computing"][0]) > 0
    assert int(float(kt["API Statistic"]["aclrtSynchronizeDeviceWithTimeout:Count"][0])) > 0
    assert "speedup vs" in (HERE / "comparison.txt").read_text()


def test_counter_and_l2_rows_are_filled():
    # Counter passes carry their counters (and derived figures) as kernel
    # details; the L2 pass also fills the L2 Cache rows.  (A counter pass has
    # no kernel durations, so its op-statistic rows are n/a.)
    sec = _sections()
    want = {"Compute": "MfmaUtil(%)", "LDS": "LDSBankConflict(%)", "L2": "TCC_HIT_sum",
            "HBMRead": "hbm_read_bytes", "HBMWrite": "hbm_write_bytes"}
    for metric, key in want.items():
        rows = {k: v for k, v in sec[metric]["Kernel Details"].items() if k != "kernel_count"}
        assert key in rows, metric
        for label, (a, b) in rows.items():
            assert _numeric(a) and _numeric(b), f"{metric} / {label}: {a} {b}"
    hit = sec["L2"]["L2 Cache"]["Hit Rate"]
    assert 0.0 < float(hit[0]) < 1.0 and 0.0 < float(hit[1]) < 1.0
