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
    with pytest.raises(ValueError):
        T.parse_shape("1,2,3")


@pytest.mark.parametrize("d", [16, 32, 64, 128, 256])
def test_candidates_come_from_the_kernel_table(d):
    cands = T.tiling_candidates(fa, (4, 8, 1024, d, True), torch.bfloat16)
    assert cands, d
    for bm, bn, waves in cands:
        assert bm == 32 * waves
        assert fa._resolve_tiling(4, 8, 1024, d, True, bm=bm, bn=bn)[:2] == (bm, bn)
    assert len({(bm, bn) for bm, bn, _ in cands}) == len(cands)


def test_presets_block_round_trip(tmp_path):
    module = tmp_path / "flash_attention_forward.py"
    shutil.copy(fa.__file__, module)
    tuned = tmp_path / "tuned.json"
    tuned.write_text(json.dumps({"tuned_configs": {"128:8:1024:128:1": {"BLOCK_M": 128, "BLOCK_N": 32, "WAVES": 4},
                                                    "4:32:2048:128:0": {"BLOCK_M": 256, "BLOCK_N": 64}}}))
    T.apply_presets(module, tuned)
    text = module.read_text()
    assert "    (4, 32, 2048, 128, False): (256, 64)," in text
    assert "    (128, 8, 1024, 128, True): (128, 32)," in text
    mod = T.E.load_candidate(module)
    assert mod.get_tiling(128, 8, 1024, 128, True) == (128, 32)
    assert mod.get_tiling_source(128, 8, 1024, 128, True) == "preset"
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


@pytest.mark.gpu
def test_tune_one_shape_on_gpu(tmp_path, monkeypatch):
    module = tmp_path / "flash_attention_forward.py"
    shutil.copy(fa.__file__, module)
    monkeypatch.setenv("FA_MI355X_LIB", str(fa.library_path()))  # the copy loads the built library
    payload = T.main(["--candidate-module", str(module), "--output-json", str(tmp_path / "t.json"), "--dtype", "bf16",
                      "--shape", "4,8,1024,128,1", "--tune-iters", "2", "--final-iters", "2"])
    res = payload["results"][0]
    assert res["best_config"]["BLOCK_M"] in (128, 256) and res["candidate_avg_us"] > 0
    assert res["max_abs_diff"] is None or res["max_abs_diff"] < 2e-2
    assert "(4, 8, 1024, 128, True):" in module.read_text()
