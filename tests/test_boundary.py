"""CPU: the C-ABI library and the drop-in module's host logic (no GPU needed).

The library must load, export every function include/fa_fwd.h declares, and
answer the host-only calls (fa_validate, fa_query_config, fa_kernel_info,
fa_error_string, fa_abi_version, fa_params_size) without touching a GPU.  The
Python layer must reproduce the reference's argument checks and tiling API
(flash_attention_forward.py:156-252, 616-644, 1114-1122).
"""

from __future__ import annotations

import ctypes
import math
import re
import subprocess
import sys
from pathlib import Path

import pytest
import torch

from flash_attn_npu_amd import flash_attention_forward as fa
from flash_attn_npu_amd import workloads as W

REPO = Path(__file__).resolve().parent.parent
HEADER = REPO / "include" / "fa_fwd.h"


@pytest.fixture(scope="module")
def lib():
    return fa._load_library()


def header_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(fa_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_function(lib):
    names = header_functions()
    assert {"fa_fwd", "fa_validate", "fa_query_config", "fa_error_string", "fa_abi_version",
            "fa_num_kernels", "fa_kernel_info", "fa_params_size"} <= set(names)
    for name in names:
        assert hasattr(lib, name), name


def test_exported_symbols_in_dynamic_table():
    out = subprocess.run(["nm", "-D", "--defined-only", str(fa.library_path())], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (fa_\w+)", out))
    assert set(header_functions()) <= exported


def test_library_is_built_from_the_current_sources(lib):
    """The loaded library carries the hash of the kernel source and header it was
    compiled from; a library older than its sources fails here (rebuild it)."""
    from flash_attn_npu_amd.build import source_hash
    assert lib.fa_build_id().decode() == source_hash(), "stale libfa_mi355x.so: rebuild it"


def test_kernel_workgroups_per_cu(lib):
    table = fa.kernel_table()
    assert len(table) == lib.fa_num_kernels()
    assert lib.fa_kernel_wg_per_cu(-1) == lib.fa_kernel_wg_per_cu(len(table)) == -7
    for i, row in enumerate(table):
        assert 1 <= row["wg_per_cu"] <= 4
        # LDS bytes of one workgroup times the resident count fit one CU's 160 KB.
        p = _params(shape=(64, 64, 4096, row["HEAD_DIM"]), dtype={"float16": 0, "bfloat16": 1,
                    "float16+float8_e5m2_v": 2, "bfloat16+float8_e5m2_v": 3}[row["dtype"]],
                    causal=int(row["causal"]))
        p.block_m, p.block_n = row["BLOCK_M"], row["BLOCK_N"]
        out = (ctypes.c_int32 * fa.FA_CFG_COUNT)()
        assert lib.fa_query_config(ctypes.byref(p), out) == 0
        assert out[7] == i  # every entry is reachable by its own key
        assert out[5] * row["wg_per_cu"] <= 160 * 1024
        # The persistent grid is the resident capacity of the 256 CUs.
        assert out[3] == row["wg_per_cu"] * 256


def test_abi_version_and_struct_layout(lib):
    assert lib.fa_abi_version() == 1
    assert lib.fa_params_size() == ctypes.sizeof(fa.FaFwdParams) == 216


def _params(**kw):
    p = fa.FaFwdParams()
    B, H, S, D = kw.get("shape", (1, 2, 128, 64))
    # Fake but 16-byte-aligned device addresses: fa_validate never dereferences them.
    base = 1 << 40
    p.q, p.k, p.v, p.o = base, base + (1 << 30), base + (2 << 30), base + (3 << 30)
    p.lse = kw.get("lse", base + (4 << 30))
    for arr in (p.q_stride, p.k_stride, p.v_stride, p.o_stride):
        arr[0], arr[1], arr[2], arr[3] = H * S * D, S * D, D, 1
    p.B, p.H, p.Sq, p.Sk, p.D = B, H, S, S, D
    p.dtype = kw.get("dtype", 1)
    p.causal = kw.get("causal", 1)
    p.sm_scale = kw.get("scale", 0.125)
    p.block_m, p.block_n = kw.get("bm", 0), kw.get("bn", 0)
    p.num_programs = kw.get("programs", 0)
    return p


def test_validate_accepts_good_params(lib):
    assert lib.fa_validate(ctypes.byref(_params())) == 0
    assert lib.fa_validate(ctypes.byref(_params(lse=None))) == 0
    assert lib.fa_validate(ctypes.byref(_params(shape=(0, 4, 128, 128)))) == 0  # empty is fine
    for d in (16, 32, 64, 128, 256):  # every head dim of flash_attention_forward.py:1121
        assert lib.fa_validate(ctypes.byref(_params(shape=(1, 2, 128, d)))) == 0, d


@pytest.mark.parametrize("mutate,code", [
    (lambda p: setattr(p, "q", None), -1),
    (lambda p: setattr(p, "Sq", -1), -2),
    (lambda p: setattr(p, "Sk", 0), -2),
    (lambda p: setattr(p, "D", 96), -3),
    (lambda p: setattr(p, "D", 48), -3),
    (lambda p: setattr(p, "dtype", 7), -4),
    (lambda p: p.k_stride.__setitem__(3, 2), -5),
    (lambda p: p.v_stride.__setitem__(2, 12), -5),
    (lambda p: p.o_stride.__setitem__(2, 8), -5),       # seq stride below D
    (lambda p: setattr(p, "o", (1 << 40) + 8), -6),
    (lambda p: setattr(p, "block_m", 128), -7),          # BM without BN
    (lambda p: (setattr(p, "block_m", 96), setattr(p, "block_n", 64)), -7),
    (lambda p: setattr(p, "sm_scale", float("nan")), -8),
    (lambda p: setattr(p, "sm_scale", float("inf")), -8),
    (lambda p: setattr(p, "num_programs", -3), -9),
])
def test_validate_rejects(lib, mutate, code):
    p = _params()
    mutate(p)
    assert lib.fa_validate(ctypes.byref(p)) == code
    assert lib.fa_error_string(code) != b"unknown fa_fwd status"


def test_validate_fp8_v(lib):
    # dtype 2 / 3: fp16 / bf16 q, k, o with an fp8-e5m2 v, every head dim.
    for dt in (2, 3):
        for d in (16, 32, 64, 128, 256):
            assert lib.fa_validate(ctypes.byref(_params(shape=(1, 2, 128, d), dtype=dt))) == 0, (dt, d)
        assert lib.fa_validate(ctypes.byref(_params(shape=(1, 2, 128, 48), dtype=dt))) == -3
    # 16-byte rows: an fp8 v needs strides in multiples of 16 elements.
    p = _params(shape=(1, 2, 128, 64), dtype=3)
    p.v_stride[2] = 72
    assert lib.fa_validate(ctypes.byref(p)) == -5
    p.dtype = 1
    assert lib.fa_validate(ctypes.byref(p)) == 0
    out = (ctypes.c_int32 * 8)()
    assert lib.fa_query_config(ctypes.byref(_params(shape=(4, 32, 2048, 128), dtype=3)), out) == 0
    assert (out[0], out[1]) == (128, 64) and out[5] == 2 * (64 * 256 + 64 * 128)  # two K + fp8 V stages
    assert lib.fa_query_config(ctypes.byref(_params(shape=(1, 2, 128, 32), dtype=2)), out) == 0
    assert out[1] == 64 and out[5] == 2 * (64 * 64 + 4 * 1024)  # 2 KB fp8 V tile padded to a DMA per wave
    assert lib.fa_query_config(ctypes.byref(_params(shape=(1, 2, 128, 16), dtype=2)), out) == 0
    assert out[1] == 128 and out[5] == 2 * (128 * 32 + 4 * 1024)
    # D = 256: 64-key tiles with fp8 V (32 with a 16-bit V), one workgroup per CU.
    assert lib.fa_query_config(ctypes.byref(_params(shape=(1, 2, 4096, 256), dtype=3)), out) == 0
    assert out[1] == 64 and out[5] == 2 * (64 * 512 + 64 * 256)
    assert lib.fa_query_config(ctypes.byref(_params(shape=(1, 2, 4096, 256), dtype=1)), out) == 0
    # 16-bit V: two 32-key K + V stages and the 64 KB Q area of 128 whole rows.
    assert out[1] == 32 and out[5] == 2 * (32 * 512 + 32 * 512) + 128 * 512
    # 64-key D = 256 tiles hold the Q rows in the wave's own DMA chunks: no Q area.
    assert lib.fa_query_config(ctypes.byref(_params(shape=(1, 2, 4096, 256), dtype=1, bm=128, bn=64)), out) == 0
    assert out[1] == 64 and out[5] == 2 * (64 * 512 + 64 * 512)


def test_validate_rejects_slices_over_2gib(lib):
    p = _params(shape=(1, 1, 9_000_000, 128))  # 9e6 rows x 256 B > 2 GiB
    assert lib.fa_validate(ctypes.byref(p)) == -2


def test_error_strings(lib):
    assert lib.fa_error_string(0) == b"ok"
    assert lib.fa_error_string(-100).startswith(b"the HIP runtime")
    assert lib.fa_error_string(12345) == b"unknown fa_fwd status"


def test_query_config_headline(lib):
    out = (ctypes.c_int32 * 8)()
    assert lib.fa_query_config(ctypes.byref(_params(shape=(4, 32, 2048, 128))), out) == 0
    bm, bn, waves, grid, tiles, lds, stage, kid = list(out)
    assert (bm, bn) == tuple(fa.get_tiling(4, 32, 2048, 128, True))
    # Persistent grid: two waves per SIMD on 256 CUs, capped by the tile count.
    assert waves == bm // 32 and tiles == math.ceil(2048 / bm) * 128 and grid == min(tiles, 8 // waves * 256)
    assert stage == 3 and 0 < lds <= 160 * 1024 and 0 <= kid < lib.fa_num_kernels()


def test_query_config_persistent_cap(lib):
    out = (ctypes.c_int32 * 8)()
    assert lib.fa_query_config(ctypes.byref(_params(shape=(4, 32, 2048, 128), programs=20)), out) == 0
    assert out[3] == 20


def test_kernel_table_is_consistent(lib):
    rows = fa.kernel_table()
    assert rows, "library has no kernels"
    seen = set()
    for r in rows:
        assert r["HEAD_DIM"] in fa.SUPPORTED_HEAD_DIMS
        assert r["BLOCK_M"] == 32 * r["waves"] and r["BLOCK_N"] % 32 == 0
        seen.add((r["HEAD_DIM"], r["dtype"], r["causal"]))
    for d in fa.SUPPORTED_HEAD_DIMS:
        for dt in ("float16", "bfloat16"):
            for c in (False, True):
                assert (d, dt, c) in seen
    for d in fa.FP8_V_HEAD_DIMS:
        for dt in ("float16+float8_e5m2_v", "bfloat16+float8_e5m2_v"):
            for c in (False, True):
                assert (d, dt, c) in seen


# ---------------------------------------------------------------------------
# Python layer (the reference's module API)

def test_module_surface():
    for name in ("DEVICE", "attention", "flash_attention_forward", "_launch_kernel", "get_tiling",
                 "get_tiling_source", "_describe_runtime", "_get_persistent_programs", "_make_inputs",
                 "_validate_inputs", "_resolve_tiling", "PROFILE_OP_NAME", "DEFAULT_TILING_PRESETS"):
        assert hasattr(fa, name), name
    assert fa.DEVICE == "cuda"
    assert fa.flash_attention_forward is fa.attention


def test_module_loads_by_path():
    import importlib.util
    spec = importlib.util.spec_from_file_location("flash_attention_candidate",
                                                  REPO / "flash_attn_npu_amd" / "flash_attention_forward.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    assert mod.DEVICE == "cuda" and callable(mod.attention)
    assert mod._load_library().fa_abi_version() == 1


@pytest.mark.parametrize("shapes,msg", [
    (((2, 3, 4), (2, 3, 4), (2, 3, 4)), "4D"),
    (((1, 2, 8, 64), (1, 2, 9, 64), (1, 2, 8, 64)), "same shape"),
    (((1, 2, 8, 48), (1, 2, 8, 48), (1, 2, 8, 48)), "HEAD_DIM must be one of"),
    (((1, 2, 8, 96), (1, 2, 8, 96), (1, 2, 8, 96)), "HEAD_DIM must be one of"),
])
def test_validate_inputs_like_reference(shapes, msg):
    q, k, v = (torch.zeros(s, dtype=torch.float16) for s in shapes)
    with pytest.raises(ValueError, match=msg):
        fa._validate_inputs(q, k, v)


def test_fp8_v_validation():
    q = torch.zeros((1, 2, 8, 64), dtype=torch.bfloat16)
    v8 = torch.zeros((1, 2, 8, 64), dtype=torch.float8_e5m2)
    with pytest.raises(ValueError, match="GPU tensors"):  # accepted dtype mix, then the device check
        fa._validate_inputs(q, q, v8)
    q48 = torch.zeros((1, 2, 8, 48), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="HEAD_DIM"):
        fa._validate_inputs(q48, q48, torch.zeros((1, 2, 8, 48), dtype=torch.float8_e5m2))
    with pytest.raises(ValueError, match="float16"):  # fp8 q / k are not accepted
        fa._validate_inputs(v8, v8, v8)


def test_rejects_cpu_tensors_and_bad_dtype():
    q = torch.zeros((1, 2, 8, 64), dtype=torch.float16)
    with pytest.raises(ValueError, match="GPU tensors"):
        fa.attention(q, q, q, False, 0.1)
    q32 = torch.zeros((1, 2, 8, 64), dtype=torch.float32)
    with pytest.raises(ValueError, match="float16"):
        fa.attention(q32, q32, q32, False, 0.1)


def test_tiling_resolution(monkeypatch):
    with pytest.raises(ValueError, match="together"):
        fa._resolve_tiling(1, 1, 128, 64, False, bm=128)
    assert fa._resolve_tiling(1, 1, 128, 64, False, bm=256, bn=64) == (256, 64, "override")
    monkeypatch.setitem(fa.DEFAULT_TILING_PRESETS, (2, 3, 4096, 128, True), (256, 64))
    assert fa.get_tiling(2, 3, 4096, 128, True) == (256, 64)
    assert fa.get_tiling_source(2, 3, 4096, 128, True) == "preset"
    assert fa.get_tiling_source(2, 3, 4097, 128, True) == "fallback"


def test_presets_are_per_dtype(monkeypatch):
    """A bfloat16 sweep's presets serve bfloat16 calls only, and the float16 table
    (the reference's DEFAULT_TILING_PRESETS) float16 calls only."""
    key = (2, 3, 4096, 128, True)
    monkeypatch.setitem(fa.DEFAULT_TILING_PRESETS, key, (256, 64))
    monkeypatch.setitem(fa.DEFAULT_TILING_PRESETS_BF16, key, (128, 32))
    assert fa.get_tiling(*key) == (256, 64)
    assert fa.get_tiling(*key, dtype=torch.float16) == (256, 64)
    assert fa.get_tiling(*key, dtype=torch.bfloat16) == (128, 32)
    assert fa._resolve_tiling(*key, dtype=torch.bfloat16) == (128, 32, "preset")
    assert fa._describe_runtime(*key, dtype=torch.bfloat16)["selected_config"] == {"BLOCK_M": 128, "BLOCK_N": 32}
    assert fa._describe_runtime(*key)["selected_config"] == {"BLOCK_M": 256, "BLOCK_N": 64}
    monkeypatch.delitem(fa.DEFAULT_TILING_PRESETS_BF16, key)
    assert fa.get_tiling_source(*key, dtype=torch.bfloat16) == "fallback"
    assert fa.get_tiling(*key, dtype=torch.bfloat16) == tuple(fa._query_config(*key, dtype=torch.bfloat16)[:2])


def test_fallback_tiling_cached_per_shape(monkeypatch):
    """The library's default tiling is asked once per shape and the cached
    answer is the library's; a preset for the shape still wins."""
    key = (3, 5, 777, 64, True)
    fa._FALLBACK_TILING.pop(key + (torch.float16,), None)
    want = tuple(fa._query_config(*key)[:2])
    calls = []
    real = fa._query_config
    monkeypatch.setattr(fa, "_query_config", lambda *a, **k: calls.append(a) or real(*a, **k))
    assert fa.get_tiling(*key) == want
    assert fa.get_tiling(*key) == want
    assert len(calls) == 1
    monkeypatch.setitem(fa.DEFAULT_TILING_PRESETS, key, (128, 32))
    assert fa.get_tiling(*key) == (128, 32)


def test_call_key_follows_the_environment(monkeypatch):
    """The repeated-call cache key reads PERSISTENT_PROGRAMS and KV_SPLITS on every call
    (through os.environ's own dict on POSIX): a change made through os.environ gives a
    new key, and undoing it gives the old one back."""
    q = torch.zeros((1, 2, 40, 64), dtype=torch.float16)
    monkeypatch.delenv("KV_SPLITS", raising=False)
    monkeypatch.delenv("PERSISTENT_PROGRAMS", raising=False)
    base = fa._call_key(q, q, q, True, None, None)
    monkeypatch.setenv("KV_SPLITS", "3")
    split = fa._call_key(q, q, q, True, None, None)
    monkeypatch.setenv("PERSISTENT_PROGRAMS", "7")
    both = fa._call_key(q, q, q, True, None, None)
    assert len({base, split, both}) == 3
    monkeypatch.setenv("KV_SPLITS", "4")
    assert fa._call_key(q, q, q, True, None, None) != both
    monkeypatch.delenv("KV_SPLITS")
    monkeypatch.delenv("PERSISTENT_PROGRAMS")
    assert fa._call_key(q, q, q, True, None, None) == base
    assert fa._call_key(q, q, q, False, None, None) != base
    assert fa._call_key(q.permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3), q, q, True, None, None) != base


def test_kernel_ready_fast_path_and_copies():
    t = torch.zeros((2, 3, 40, 64), dtype=torch.float16)
    assert fa._kernel_ready(t) is t  # contiguous, 16-byte aligned: read in place
    view = t.permute(0, 2, 1, 3)  # [B, S, H, D] strides: still readable in place
    assert fa._kernel_ready(view) is view
    odd = torch.zeros((1, 2, 40, 72), dtype=torch.float16)[..., 1:65]  # misaligned base
    ready = fa._kernel_ready(odd)
    assert ready is not odd and ready.is_contiguous() and torch.equal(ready, odd)
    # A contiguous view at an odd storage offset: contiguous() would hand back the
    # same misaligned view, so the module must copy it.
    buf = torch.arange(2 * 3 * 40 * 64 + 1, dtype=torch.float32).to(torch.float16)
    shifted = buf[1:].view(2, 3, 40, 64)
    assert shifted.is_contiguous() and shifted.data_ptr() % 16 == 2
    ready = fa._kernel_ready(shifted)
    assert ready is not shifted and ready.data_ptr() % 16 == 0 and torch.equal(ready, shifted)


def test_persistent_programs_env(monkeypatch):
    monkeypatch.delenv("PERSISTENT_PROGRAMS", raising=False)
    assert fa._get_persistent_programs() == fa.DEFAULT_PERSISTENT_PROGRAMS
    monkeypatch.setenv("PERSISTENT_PROGRAMS", "64")
    assert fa._get_persistent_programs() == 64
    monkeypatch.setenv("PERSISTENT_PROGRAMS", "0")
    with pytest.raises(ValueError):
        fa._get_persistent_programs()


def test_describe_runtime_keys(monkeypatch):
    monkeypatch.delenv("PERSISTENT_PROGRAMS", raising=False)
    rt = fa._describe_runtime(4, 32, 2048, 128, True)
    assert set(rt) >= {"selected_config", "tiling_source", "total_tiles", "launched_programs", "stage"}
    assert rt["stage"] == 3 and rt["launched_programs"] == min(rt["total_tiles"], 8 // rt["waves"] * 256)
    assert fa._describe_runtime(4, 32, 2048, 128, False)["stage"] == 1


def test_describe_runtime_follows_dtype(monkeypatch):
    """The description queries the kernel the call would launch: an fp8-e5m2 V selects the
    fp8-V kernels' tiling (64-key tiles), a bf16 call the bf16 kernel."""
    monkeypatch.delenv("PERSISTENT_PROGRAMS", raising=False)
    monkeypatch.delenv("KV_SPLITS", raising=False)
    plain = fa._describe_runtime(1, 2, 300, 128, False, dtype=torch.bfloat16)
    fp8 = fa._describe_runtime(1, 2, 300, 128, False, dtype=torch.bfloat16, v_dtype=torch.float8_e5m2)
    assert fp8["selected_config"] == {"BLOCK_M": 128, "BLOCK_N": 64}
    assert fp8["kernel_id"] != plain["kernel_id"]
    rows = fa.kernel_table()
    assert rows[plain["kernel_id"]]["dtype"] == "bfloat16"
    assert rows[fp8["kernel_id"]]["dtype"] == "bfloat16+float8_e5m2_v"


def test_check_maps_errors():
    with pytest.raises(ValueError):
        fa._check(-5, "x")
    with pytest.raises(RuntimeError):
        fa._check(-100, "x")


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(fa, "_LIB", None)
    monkeypatch.setenv("FA_MI355X_LIB", str(tmp_path / "nope.so"))
    with pytest.raises(RuntimeError, match="no fallback"):
        fa._load_library()


# ---------------------------------------------------------------------------
# Workloads and bench contract

def test_workload_inputs_are_seeded():
    w = W.CONFIGS[0]
    a = W.make_inputs(w)
    b = W.make_inputs(w)
    for x, y in zip(a, b):
        assert torch.equal(x, y) and x.dtype == w.dtype and x.shape == (w.B, w.H, w.S, w.D)


def test_ragged_config_distributions():
    w = W.CONFIGS[4]
    q, k, v = W.make_inputs(w, batch_slice=slice(0, 1))
    assert float(v.float().abs().max()) <= 1.0
    frac_big = float((q.float().abs() > 4.5).float().mean())
    assert 0.003 < frac_big < 0.02  # ~1% of entries scaled x8
    assert w.S % 64 != 0 and w.causal and w.dtype == torch.bfloat16


def test_configs_match_task():
    shapes = [(c.B, c.H, c.S, c.D, c.causal) for c in W.CONFIGS]
    assert shapes == [(1, 8, 512, 64, False), (4, 32, 2048, 128, True), (2, 16, 8192, 128, True),
                      (16, 16, 1024, 64, False), (8, 32, 3000, 128, True)]
    assert W.HEADLINE.flops == pytest.approx(1.3744e11, rel=1e-4)


def test_bench_refuses_multi_gpu():
    r = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=60)
    assert r.returncode == 2 and "one GPU" in r.stderr


# ---------------------------------------------------------------------------
# Split-KV host logic (no launch)

def test_split_workspace_bytes(lib):
    p = _params(shape=(2, 3, 100, 64))
    part_o = 4 * 2 * 3 * 100 * 64 * 4
    assert lib.fa_split_workspace_bytes(ctypes.byref(p), 4) == (part_o + 255) // 256 * 256 + 4 * 2 * 3 * 100 * 4
    assert lib.fa_split_workspace_bytes(ctypes.byref(p), 1) == 0
    assert lib.fa_split_workspace_bytes(ctypes.byref(p), 0) == -9
    assert lib.fa_split_workspace_bytes(ctypes.byref(p), 65) == -9


@pytest.mark.parametrize("shape,causal,splits", [
    ((1, 1, 4096, 128), 0, 8),    # 32 tiles: one run per CU, 512-key runs
    ((1, 8, 512, 64), 0, 1),      # runs below 64K key-columns
    ((1, 4, 1024, 64), 0, 1),
    ((4, 32, 2048, 128), 0, 1),   # grid already fills the chip
    ((1, 8, 4096, 64), 0, 1),     # 256 tiles: one per CU, no split
    ((1, 1, 16384, 64), 0, 2),    # 128 tiles: two runs fill the CUs
    ((1, 1, 16384, 64), 1, 4),    # causal: two runs per CU
    ((1, 4, 2048, 128), 1, 4),
    ((1, 2, 2048, 256), 1, 8),
    ((1, 1, 300, 64), 0, 1)])
def test_default_kv_splits(lib, shape, causal, splits):
    p = _params(shape=shape, causal=causal)
    assert lib.fa_default_kv_splits(ctypes.byref(p)) == splits


def test_split_argument_errors_before_launch(lib):
    p = _params(shape=(1, 2, 700, 128))
    assert lib.fa_fwd_split(ctypes.byref(p), 0, None, 0, None) == -9
    assert lib.fa_fwd_split(ctypes.byref(p), 4, None, 1 << 20, None) == -1
    assert lib.fa_fwd_split(ctypes.byref(p), 4, (1 << 40), 16, None) == -2
    assert lib.fa_fwd_split(ctypes.byref(p), 4, (1 << 40) + 64, 1 << 30, None) == -6


def test_static_split_argument_errors_before_launch(lib):
    """fa_fwd_split_static checks its split count and the scratch limit before any HIP call."""
    p = _params(shape=(2, 16, 4096, 128))
    assert lib.fa_fwd_split_static(ctypes.byref(p), 0, None) == -9
    assert lib.fa_fwd_split_static(ctypes.byref(p), 65, None) == -9
    assert lib.fa_split_workspace_bytes(ctypes.byref(p), 3) > 32 * 1024 * 1024
    assert lib.fa_fwd_split_static(ctypes.byref(p), 3, None) == -10
    assert b"static scratch" in lib.fa_error_string(-10)


def test_call_key_follows_preset_tables(monkeypatch):
    # The fast-path key changes when a preset table is edited or replaced.
    from flash_attn_npu_amd import flash_attention_forward as fa
    q = torch.zeros((1, 2, 16, 64), dtype=torch.float16)
    k0 = fa._call_key(q, q, q, True, None, None)
    assert fa._call_key(q, q, q, True, None, None) == k0
    monkeypatch.setitem(fa.DEFAULT_TILING_PRESETS_BF16, (1, 2, 16, 64, True), (128, 32))
    k1 = fa._call_key(q, q, q, True, None, None)
    assert k1 != k0
    monkeypatch.setattr(fa, "DEFAULT_TILING_PRESETS", dict(fa.DEFAULT_TILING_PRESETS))
    assert fa._call_key(q, q, q, True, None, None) != k1
