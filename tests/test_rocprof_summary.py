"""CPU: the rocprofv3 pass summarizer and the profile_summary.{json,txt} writer.

The summary must carry every key the reference's comparison tool reads
(compare_results_plus.py:283-338 for an entry, :447-479 for the printed
comparison), so two MI355X runs compare with that tool unmodified, and the
HBM byte figures must be scaled by the plain-copy calibration that runs in
the same process.
"""

from __future__ import annotations

import csv
import json

import pytest

from flash_attn_npu_amd import rocprof

KERNEL = "void (anonymous namespace)::fa_fwd_dma_kernel<128, 64, 4, 2, 2, true, true, false>(KernelArgs)"
COPY = "void at::native::elementwise_kernel<copy>(...)"


def _write_trace(path, rows):
    with path.open("w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Kernel_Name", "Start_Timestamp", "End_Timestamp", "Grid_Size_X",
                                          "Workgroup_Size_X", "LDS_Block_Size", "VGPR_Count", "Scratch_Size"])
        w.writeheader()
        for name, start_ns, dur_ns in rows:
            w.writerow({"Kernel_Name": name, "Start_Timestamp": start_ns, "End_Timestamp": start_ns + dur_ns,
                        "Grid_Size_X": 512 * 256, "Workgroup_Size_X": 256, "LDS_Block_Size": 66048,
                        "VGPR_Count": 128, "Scratch_Size": 12})


def _write_counters(path, rows):
    with path.open("w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Kernel_Name", "Counter_Name", "Counter_Value"])
        w.writeheader()
        for name, counter, value in rows:
            w.writerow({"Kernel_Name": name, "Counter_Name": counter, "Counter_Value": value})


@pytest.fixture()
def passes(tmp_path):
    trace = tmp_path / "KernelTrace" / "host"
    trace.mkdir(parents=True)
    # Three attention launches (150, 152, 154 us) and one 50 us copy.
    _write_trace(trace / "run_kernel_trace.csv",
                 [(KERNEL, 0, 150_000), (KERNEL, 200_000, 152_000), (KERNEL, 400_000, 154_000), (COPY, 600_000, 50_000)])
    read = tmp_path / "HBMRead" / "host"
    read.mkdir(parents=True)
    # The 256 MiB copy reads as 96 MiB (factor 8/3); the kernel reads 190,000 KiB per launch.
    _write_counters(read / "run_counter_collection.csv",
                    [(KERNEL, "FETCH_SIZE", 190_000.0), (KERNEL, "FETCH_SIZE", 190_000.0),
                     (COPY, "FETCH_SIZE", 96 * 1024.0)])
    l2 = tmp_path / "L2" / "host"
    l2.mkdir(parents=True)
    _write_counters(l2 / "run_counter_collection.csv",
                    [(KERNEL, "TCC_HIT_sum", 740.0), (KERNEL, "TCC_MISS_sum", 260.0)])
    return tmp_path


def test_kernel_trace_pass(passes):
    e = rocprof.summarize_pass(passes / "KernelTrace")
    op = e["op"]
    assert op["OP Type"] == KERNEL and op["Count"] == 3.0
    assert op["Avg Time(us)"] == pytest.approx(152.0) and op["Min Time(us)"] == pytest.approx(150.0)
    assert op["Max Time(us)"] == pytest.approx(154.0) and op["Total Time(us)"] == pytest.approx(456.0)
    assert op["Ratio(%)"] == pytest.approx(100.0 * 456.0 / 506.0)  # the copy is not the target op
    assert e["kernel"]["kernel_count"] == 3.0 and e["kernel"]["Block Num"] == 512.0
    assert e["kernel"]["Duration(us)"] == pytest.approx(152.0)


def test_fetch_scaled_by_copy_calibration(passes):
    k = rocprof.summarize_pass(passes / "HBMRead")["kernel"]
    factor = rocprof.COPY_BYTES / (96 * 1024.0 * 1024.0)
    assert k["FETCH_SIZE_copy_factor"] == pytest.approx(factor) == pytest.approx(8 / 3)
    assert k["hbm_read_bytes"] == pytest.approx(190_000.0 * 1024.0 * factor)


def test_l2_hit_rate(passes):
    e = rocprof.summarize_pass(passes / "L2")
    assert e["l2"]["Hit Rate"] == pytest.approx(0.74) and e["l2_columns"] == ["Hit Rate"]


def test_summary_files_carry_the_comparison_tool_keys(passes):
    summary = rocprof.summarize_dir(passes, plan={"KernelTrace": None, "HBMRead": ["FETCH_SIZE"], "L2": ["x"]})
    j, t = rocprof.write_profile_summary_files(passes / "out", summary)
    data = json.loads(j.read_text())
    assert set(data) == {"KernelTrace", "HBMRead", "L2"}
    for entry in data.values():
        # Keys read per entry by compare_results_plus.py:319-338 and printed at :447-479.
        assert {"profiler_output", "op_name", "op", "kernel", "kernel_columns", "step", "api", "l2",
                "l2_columns"} <= set(entry)
        assert isinstance(entry["kernel_columns"], list) and isinstance(entry["l2_columns"], list)
        for c in entry["kernel_columns"]:
            assert c in entry["kernel"]
    op = data["KernelTrace"]["op"]
    for key in ("OP Type", "Count", "Total Time(us)", "Min Time(us)", "Avg Time(us)", "Max Time(us)", "Ratio(%)"):
        assert key in op
    text = t.read_text()
    assert "[KernelTrace]" in text and "avg_us=152.000" in text and "Hit Rate=0.740000" in text


def test_step_trace_from_kernel_trace(passes):
    """Steps run from one attention launch to the next; the copy at 600 us falls in
    the last step, which ends with it (650 us)."""
    step = rocprof.summarize_pass(passes / "KernelTrace")["step"]
    # Steps: [0, 200) busy 150; [200, 400) busy 152; [400, 650) busy 154 + 50.
    assert step["Computing"] == pytest.approx(152.0)           # median of 150, 152, 204
    assert step["Free"] == pytest.approx(48.0)                 # median of 50, 48, 46
    assert step["Stage"] == pytest.approx(200.0)               # median of 200, 200, 250
    assert step["step_count"] == 3.0
    for col in ("Communication", "Overlapped", "Bubble", "Preparing"):
        assert step[col] == 0.0
    assert set(rocprof.STEP_COLUMNS) <= set(step)


def test_step_trace_merges_overlapping_kernels(tmp_path):
    d = tmp_path / "KernelTrace"
    d.mkdir()
    # Two target launches 100 us apart; an overlapping 30 us kernel inside the first
    # step (40..70 against 0..50) and an idle gap: busy = 70, not 80.
    _write_trace(d / "run_kernel_trace.csv", [(KERNEL, 0, 50_000), (COPY, 40_000, 30_000), (KERNEL, 100_000, 10_000)])
    step = rocprof.summarize_steps(d)
    assert step["step_count"] == 2.0
    assert step["Computing"] == pytest.approx((70.0 + 10.0) / 2)
    assert step["Stage"] == pytest.approx((100.0 + 10.0) / 2)


def _write_rows(path, fields, rows):
    with path.open("w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=fields)
        w.writeheader()
        for r in rows:
            w.writerow(dict(zip(fields, r)))


def test_api_statistic_from_hip_trace(tmp_path):
    d = tmp_path / "KernelTrace"
    d.mkdir()
    _write_rows(d / "run_kernel_trace.csv", ["Kernel_Name", "Correlation_Id", "Start_Timestamp", "End_Timestamp"],
                [(KERNEL, 7, 1_000, 2_000), (COPY, 8, 3_000, 4_000), (KERNEL, 9, 5_000, 6_000)])
    _write_rows(d / "run_hip_api_trace.csv", ["Domain", "Function", "Correlation_Id", "Start_Timestamp", "End_Timestamp"],
                [("HIP_RUNTIME_API", "hipLaunchKernel", 7, 0, 4_000),
                 ("HIP_RUNTIME_API", "hipLaunchKernel", 8, 0, 9_000),
                 ("HIP_RUNTIME_API", "hipLaunchKernel", 9, 0, 6_000),
                 ("HIP_RUNTIME_API", "hipDeviceSynchronize", 10, 0, 20_000),
                 ("HIP_RUNTIME_API", "hipDeviceSynchronize", 11, 0, 40_000),
                 ("HIP_RUNTIME_API", "hipEventSynchronize", 12, 0, 5_000),
                 ("HIP_RUNTIME_API", "hipMalloc", 13, 0, 100_000)])
    api = rocprof.summarize_api(d)
    # launch = the attention kernel's own launch calls (correlation 7 and 9): 4 and 6 us.
    assert api["launch"] == {"Time(us)": 10.0, "Count": 2.0, "Avg(us)": 5.0, "Min(us)": 4.0, "Max(us)": 6.0}
    assert api["launch_all"]["Count"] == 3.0 and api["launch_all"]["Max(us)"] == 9.0
    sync = api[rocprof.DEVICE_SYNC_KEY]
    assert sync == api["hipDeviceSynchronize"] and sync["Avg(us)"] == 30.0 and sync["Count"] == 2.0
    assert api["hipEventSynchronize"]["Count"] == 1.0
    assert "hipMalloc" not in api
    for row in api.values():
        assert set(row) == set(rocprof.API_COLUMNS)


def test_summary_text_carries_step_and_api_lines(tmp_path, passes):
    d = passes / "KernelTrace" / "host"
    _write_rows(d / "run_hip_api_trace.csv", ["Function", "Correlation_Id", "Start_Timestamp", "End_Timestamp"],
                [("hipLaunchKernel", 1, 0, 3_000), ("hipDeviceSynchronize", 2, 0, 8_000)])
    summary = rocprof.summarize_dir(passes, plan={"KernelTrace": None})
    _, t = rocprof.write_profile_summary_files(tmp_path / "out", summary)
    text = t.read_text()
    # The trace has no correlation ids: launch falls back to every launch call.
    assert "step: computing_us=152.000, free_us=48.000, bubble_us=0.000, preparing_us=0.000" in text
    assert "api: launch_avg_us=3.000, sync_avg_us=8.000" in text


def test_build_stamp_in_both_summary_files(tmp_path, passes):
    # The stamp names the profiled library's build; the comparison tool skips
    # keys with a leading "__" (compare_results_plus.py:492-495).
    summary = rocprof.summarize_dir(passes, plan={"KernelTrace": None})
    stamp = {"fa_build_id": "0123456789abcdef", "library": "libfa_mi355x.so", "kernel_name": KERNEL}
    j, t = rocprof.write_profile_summary_files(tmp_path / "out", summary, stamp)
    data = json.loads(j.read_text())
    assert data[rocprof.BUILD_KEY] == stamp and [k for k in data if not k.startswith("__")] == ["KernelTrace"]
    assert t.read_text().splitlines()[0].startswith("build: fa_build_id=0123456789abcdef, library=libfa_mi355x.so")
    assert rocprof.read_build_id(t) == "0123456789abcdef"
    _, t2 = rocprof.write_profile_summary_files(tmp_path / "plain", summary)
    assert rocprof.read_build_id(t2) is None


def test_build_stamp_of_the_tree_library():
    # build_stamp() loads the library (host-only call) and names the kernel of
    # the kernel-trace pass.
    from flash_attn_npu_amd import flash_attention_forward as fa
    stamp = rocprof.build_stamp({"KernelTrace": {"op_name": rocprof.PROFILE_OP_NAME, "op": {"OP Type": KERNEL}}})
    assert stamp["fa_build_id"] == fa._load_library().fa_build_id().decode()
    assert stamp["kernel_name"] == KERNEL
    assert not {"kernel", "l2", "op", "step", "api"} & set(stamp)  # read by the comparison tool


def test_bench_uses_traffic_of_its_own_build_only(tmp_path, monkeypatch):
    import bench
    body = ("[HBMRead]\nkernel_metrics: hbm_read_bytes=1000.000, x=1\n[HBMWrite]\n"
            "kernel_metrics: hbm_write_bytes=24.000\n")
    prof = tmp_path / "fa_fwd_w_rocprof.txt"
    monkeypatch.setattr(bench, "profile_summary_path", lambda tag: prof)
    assert bench.read_traffic("w", "aaaa") is None                      # no summary
    prof.write_text("# header\n\n" + body)
    assert bench.read_traffic("w", "aaaa") is None                      # no stamp
    prof.write_text("build: fa_build_id=bbbb, library=x.so\n\n" + body)
    assert bench.read_traffic("w", "aaaa") is None                      # another build
    prof.write_text("# header\n\nbuild: fa_build_id=aaaa, library=x.so\n\n" + body)
    assert bench.read_traffic("w", "aaaa") == 1024
