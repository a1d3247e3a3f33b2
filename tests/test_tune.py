"""The gfx950 tuner (flash_attn_npu_amd/tune.py): host logic on the CPU."""

from __future__ import annotations

import json
import shutil

import pytest
import torch

from flash_attn_npu_amd import flash_attention_forward as fa
from flash_attn_npu_amd import tune as T


def test_shape_parsing_and_keys():
    assert T.parse_shape("128,8,1024,128,1") == (128, 8, 1024, 128, True)
    assert T.parse_shape("1, 2, 64, 64, false") == (1, 2, 64, 64, False)
    assert T.shape_key((128, 8, 1024, 128, True)) == "128:8:1024:128:1"
    assert T.shape_key((128, 8, 1024, 128, True), torch.bfloat16) == "128:8:1024:128:1:bf16"
    assert T.parse_key("128:8:1024:128:1") == ((128, 8, 1024, 128, True), torch.float16)
    assert T.parse_key("4:32:2048:128:0:bf16") == ((4, 32, 2048, 128, False), torch.bfloat16)
    with pytest.raises(ValueError):
        T.parse_shape("1,2,3")


def test_default_cases_cover_the_evaluator_and_the_workloads():
    cases = T.default_cases("all", 0.5, 0)
    keys = [c.key for c in cases]
    assert len(keys) == len(set(keys)) == 2 * 6 + 5
    for s in T.W.REFERENCE_PERFORMANCE_CASES:
        assert T.shape_key(s) in keys and T.shape_key(s, torch.bfloat16) in keys
    for w in T.W.CONFIGS:
        c = next(c for c in cases if c.workload == w.name)
        assert c.shape == (w.B, w.H, w.S, w.D, w.causal) and c.dtype == w.dtype and c.sm_scale == w.sm_scale
        assert T.Case.from_json(c.to_json()) == c


@pytest.mark.parametrize("d", [16, 32, 64, 128, 256])
def test_candidates_come_from_the_kernel_table(d):
    cands = T.tiling_candidates(fa, (4, 8, 1024, d, True), torch.bfloat16)
    assert cands, d
    for bm, bn, waves, wg in cands:
        assert bm == 32 * waves and 1 <= wg <= 4
        assert fa._resolve_tiling(4, 8, 1024, d, True, bm=bm, bn=bn)[:2] == (bm, bn)
    assert len({(bm, bn) for bm, bn, _, _ in cands}) == len(cands)
    # The library's own choice is always among the candidates.
    assert T.library_default(fa, (4, 8, 1024, d, True), torch.bfloat16) in {(bm, bn) for bm, bn, _, _ in cands}


def test_presets_block_round_trip(tmp_path):
    module = tmp_path / "flash_attention_forward.py"
    shutil.copy(fa.__file__, module)
    tuned = tmp_path / "tuned.json"
    tuned.write_text(json.dumps({"tuned_configs": {"128:8:1024:128:1": {"BLOCK_M": 128, "BLOCK_N": 32, "WAVES": 4},
                                                    "4:32:2048:128:0": {"BLOCK_M": 256, "BLOCK_N": 64},
                                                    "4:32:2048:128:1:bf16": {"BLOCK_M": 128, "BLOCK_N": 64}}}))
    T.apply_presets(module, tuned)
    text = module.read_text()
    assert "    (4, 32, 2048, 128, False): (256, 64)," in text
    assert "    (128, 8, 1024, 128, True): (128, 32)," in text
    mod = T.E.load_candidate(module)
    assert mod.get_tiling(128, 8, 1024, 128, True) == (128, 32)
    assert mod.get_tiling_source(128, 8, 1024, 128, True) == "preset"
    # The bfloat16 entry lands in the bfloat16 table only.
    assert mod.DEFAULT_TILING_PRESETS_BF16 == {(4, 32, 2048, 128, True): (128, 64)}
    assert (4, 32, 2048, 128, True) not in mod.DEFAULT_TILING_PRESETS
    assert mod.get_tiling_source(4, 32, 2048, 128, True, dtype=torch.bfloat16) == "preset"
    assert mod.get_tiling_source(4, 32, 2048, 128, True) == "fallback"
    T.apply_presets(module, tuned)  # idempotent: one block, same content
    assert module.read_text() == text


def test_merge_keeps_old_shapes(tmp_path):
    out = tmp_path / "t.json"
    rec = lambda z, bm: {"Z": z, "H": 8, "N_CTX": 1024, "HEAD_DIM": 64, "causal": False, "best_config": {"BLOCK_M": bm}}
    out.write_text(json.dumps({"tuned_configs": {"1:8:1024:64:0": {"BLOCK_M": 128}}, "results": [rec(1, 128)]}))
    merged = T.merge_with_existing(out, {"tuned_configs": {"2:8:1024:64:0": {"BLOCK_M": 256}},
                                         "results": [rec(2, 256), rec(1, 256)]})
    assert set(merged["tuned_configs"]) == {"1:8:1024:64:0", "2:8:1024:64:0"}
    assert [r["Z"] for r in merged["results"]] == [1, 2] and merged["results"][0]["best_config"]["BLOCK_M"] == 256
    # A bfloat16 result of the same shape is a different entry.
    merged2 = T.merge_payloads(merged, {"tuned_configs": {"1:8:1024:64:0:bf16": {"BLOCK_M": 128}},
                                        "results": [dict(rec(1, 128), dtype="bfloat16")]})
    assert set(merged2["tuned_configs"]) == {"1:8:1024:64:0", "2:8:1024:64:0", "1:8:1024:64:0:bf16"}
    assert len(merged2["results"]) == 3


def _dispatch_csvs(root, pass_name, rows, counters=None):
    """A fake rocprofv3 pass: kernel-trace rows (name, start, dur) or counter rows."""
    import csv
    d = root / pass_name / "host"
    d.mkdir(parents=True)
    if counters is None:
        with (d / "run_kernel_trace.csv").open("w", newline="") as f:
            w = csv.DictWriter(f, fieldnames=["Dispatch_Id", "Kernel_Name", "Start_Timestamp", "End_Timestamp"])
            w.writeheader()
            for i, (name, start, dur) in enumerate(rows):
                w.writerow({"Dispatch_Id": i + 1, "Kernel_Name": name, "Start_Timestamp": start,
                            "End_Timestamp": start + dur})
    else:
        with (d / "run_counter_collection.csv").open("w", newline="") as f:
            w = csv.DictWriter(f, fieldnames=["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
            w.writeheader()
            for i, (name, vals) in enumerate(rows):
                for c, v in vals.items():
                    w.writerow({"Dispatch_Id": i + 1, "Kernel_Name": name, "Counter_Name": c, "Counter_Value": v})


def test_counters_follow_the_plan_order(tmp_path):
    """Dispatches are assigned to the planned configurations in order (a split-KV
    launch has two), the first launch of each is dropped, and the byte counters
    are scaled by the plain copy's reading in the same pass."""
    A, B, M, CP, FILL = "fa_fwd_dma_kernel<128, 64>", "fa_fwd_dma_kernel<128, 32>", "fa_merge_kernel<true>", \
        "__amd_rocclr_copyBuffer", "vectorized_elementwise_kernel<FillFunctor>"
    manifest = [{"key": "k1", "tag": "128x64", "launches": 3, "dispatches_per_launch": 1},
                {"key": "k1", "tag": "128x32", "launches": 2, "dispatches_per_launch": 2}]
    trace = [(A, 0, 9000), (A, 10000, 100_000), (A, 200_000, 102_000),
             (B, 400_000, 50_000), (M, 460_000, 5_000), (B, 500_000, 60_000), (M, 570_000, 4_000),
             (FILL, 600_000, 1_000), (CP, 700_000, 40_000)]
    _dispatch_csvs(tmp_path, "KernelTrace", trace)
    fetch = [(A, {"FETCH_SIZE": 1.0}), (A, {"FETCH_SIZE": 100_000.0}), (A, {"FETCH_SIZE": 110_000.0}),
             (B, {"FETCH_SIZE": 1.0}), (M, {"FETCH_SIZE": 1.0}), (B, {"FETCH_SIZE": 50_000.0}),
             (M, {"FETCH_SIZE": 2_000.0}), (FILL, {"FETCH_SIZE": 0.0}), (CP, {"FETCH_SIZE": 128 * 1024.0})]
    _dispatch_csvs(tmp_path, "HBMRead", fetch, counters=True)
    comp = [(A, {"SQ_INSTS_VALU": 10.0, "SQ_INSTS_MFMA": 1.0, "SQ_VALU_MFMA_BUSY_CYCLES": 1024.0 * 50,
                 "GRBM_GUI_ACTIVE": 800.0})] * 3 + \
           [(B, {"SQ_INSTS_VALU": 6.0, "SQ_INSTS_MFMA": 1.0, "SQ_VALU_MFMA_BUSY_CYCLES": 1024.0 * 25,
                 "GRBM_GUI_ACTIVE": 800.0}), (M, {"SQ_INSTS_VALU": 1000.0, "SQ_INSTS_MFMA": 0.0})] * 2 + \
           [(CP, {"SQ_INSTS_VALU": 1.0})]
    _dispatch_csvs(tmp_path, "Compute", comp, counters=True)
    res = T.collect_counters(tmp_path, manifest, {"KernelTrace": None, "HBMRead": ["FETCH_SIZE"], "Compute": []})
    a, b = res[("k1", "128x64")], res[("k1", "128x32")]
    assert a["kernel_us"] == pytest.approx(101.0) and b["kernel_us"] == pytest.approx(64.0)
    assert a["FETCH_SIZE_copy_factor"] == pytest.approx(2.0)  # the fill is not the copy
    assert a["l2_miss_read_bytes"] == pytest.approx(105_000.0 * 1024 * 2.0)
    assert b["l2_miss_read_bytes"] == pytest.approx(52_000.0 * 1024 * 2.0)  # attention + merge kernel
    assert "achieved_GBps" not in a  # no WRITE_SIZE pass here
    assert a["valu_per_mfma"] == pytest.approx(10.0) and b["valu_per_mfma"] == pytest.approx(6.0)  # merge excluded
    assert a["MfmaUtil(%)"] == pytest.approx(50.0) and b["MfmaUtil(%)"] == pytest.approx(25.0)
    with pytest.raises(RuntimeError, match="expects"):
        T.collect_counters(tmp_path, manifest[:1], {"KernelTrace": None})


def test_summary_text_lists_candidates_and_counters():
    payload = {"meta": {"device": "MI355X", "timing": "events"},
               "results": [{"Z": 4, "H": 32, "N_CTX": 2048, "HEAD_DIM": 128, "causal": True, "dtype": "bfloat16",
                            "sm_scale": 0.088, "workload": "w2", "best_config": {"BLOCK_M": 128, "BLOCK_N": 64},
                            "library_default": "128x64", "choice": "fastest",
                            "candidates": [{"config": {"BLOCK_M": 128, "BLOCK_N": 64, "WG_PER_CU": 2}, "avg_us": 145.0},
                                           {"config": {"BLOCK_M": 256, "BLOCK_N": 64, "WG_PER_CU": 1}, "avg_us": 150.0}],
                            "counters": {"128x64": {"kernel_us": 148.0, "MfmaUtil(%)": 45.0,
                                                    "l2_miss_read_bytes": 3.7e8, "l2_miss_write_bytes": 6.8e7,
                                                    "achieved_GBps": 2959.0}}}]}
    text = T.summary_text(payload)
    assert "[4:32:2048:128:1:bf16] (w2)" in text and "128x64/wg2=145.00us" in text
    assert "MfmaUtil 45.0%" in text and "370.0/68.0 MB" in text and "2959 GB/s" in text


@pytest.mark.gpu
def test_tune_one_shape_on_gpu(tmp_path, monkeypatch):
    module = tmp_path / "flash_attention_forward.py"
    shutil.copy(fa.__file__, module)
    monkeypatch.setenv("FA_MI355X_LIB", str(fa.library_path()))  # the copy loads the built library
    payload = T.main(["--candidate-module", str(module), "--output-json", str(tmp_path / "t.json"), "--dtype", "bf16",
                      "--shape", "4,8,1024,128,1", "--rounds", "2", "--launches", "3", "--final-iters", "2",
                      "--warmup-seconds", "0.1"])
    res = payload["results"][0]
    assert res["best_config"]["BLOCK_M"] in (128, 256) and res["candidate_avg_us"] > 0
    assert res["max_abs_diff"] is None or res["max_abs_diff"] < 2e-2
    assert all(len(c["rounds_us"]) == 2 for c in res["candidates"] if c.get("avg_us") is not None)
    assert "4:8:1024:128:1:bf16" in payload["tuned_configs"]
    assert "DEFAULT_TILING_PRESETS_BF16 = {\n    (4, 8, 1024, 128, True):" in module.read_text()
