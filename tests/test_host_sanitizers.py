"""CPU: the ABI's host code under sanitizers, and a fresh gfx950 build of the kernels.

* The host-only planning half of the library (flash_attn_npu_amd/csrc/fa_plan.cpp:
  fa_validate, fa_query_config, make_plan, fa_default_kv_splits,
  fa_split_workspace_bytes, the kernel table) is compiled with g++ under
  AddressSanitizer and UndefinedBehaviorSanitizer together with
  tests/abi_host_check.cpp, which sweeps every entry point over edge cases and
  a seeded random set of parameters.  Any sanitizer report fails the test.
* The kernel source is compiled for gfx950 from scratch with the library's own
  recipe (hipcc cross-compiles without a GPU), and the fresh library must
  describe the same kernel table and carry the same source hash as the one in
  the tree, so the boundary tests never pass on a stale build.  The same
  compile reports each kernel's registers (-Rpass-analysis=kernel-resource-usage):
  every kernel must reach the occupancy its table entry launches with, and no
  kernel that the default tiling or a preset selects may use scratch.
"""

from __future__ import annotations

import ctypes
import os
import re
import shutil
import subprocess
from pathlib import Path

import pytest
import torch

from flash_attn_npu_amd import build as B
from flash_attn_npu_amd import flash_attention_forward as fa

REPO = Path(__file__).resolve().parent.parent
CHECK_SRC = REPO / "tests" / "abi_host_check.cpp"


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_abi_host_code_under_asan_and_ubsan(tmp_path):
    exe = tmp_path / "abi_host_check"
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", "-Wall", "-Wextra", "-Werror",
           "-fsanitize=address,undefined", "-fno-sanitize-recover=all", f"-I{B.INCLUDE_DIR}",
           str(CHECK_SRC), str(B.PLAN_SRC), "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    env.pop("LD_PRELOAD", None)  # the sanitizer runtime must come first in the process
    proc = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=300)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "runtime error" not in proc.stderr and "AddressSanitizer" not in proc.stderr, proc.stderr
    assert f"abi host check ok: {fa._load_library().fa_num_kernels()} kernels" in proc.stdout


def _table(lib):
    rows = []
    out = (ctypes.c_int32 * 6)()
    lib.fa_kernel_info.argtypes = [ctypes.c_int, ctypes.POINTER(ctypes.c_int32)]
    lib.fa_kernel_wg_per_cu.argtypes = [ctypes.c_int]
    for i in range(lib.fa_num_kernels()):
        assert lib.fa_kernel_info(i, out) == 0
        rows.append(tuple(out) + (lib.fa_kernel_wg_per_cu(i),))
    return rows


@pytest.mark.skipif(not Path("/opt/rocm/bin/hipcc").exists() and shutil.which("hipcc") is None,
                    reason="needs hipcc")
def test_kernel_source_compiles_for_gfx950_and_matches_the_tree(tmp_path):
    out = tmp_path / "libfa_fresh.so"
    cmd = B.compile_command(out, extra=["-Rpass-analysis=kernel-resource-usage"])
    proc = subprocess.run(cmd, capture_output=True, text=True, timeout=900)
    assert proc.returncode == 0, proc.stderr[-4000:]
    fresh = ctypes.CDLL(str(out))
    fresh.fa_build_id.restype = ctypes.c_char_p
    tree = fa._load_library()
    assert fresh.fa_build_id().decode() == B.source_hash() == tree.fa_build_id().decode(), \
        "the library in the tree was not built from the current sources"
    assert _table(fresh) == _table(tree)
    assert fresh.fa_params_size() == tree.fa_params_size() == ctypes.sizeof(fa.FaFwdParams)
    _check_resources(_resource_remarks(proc.stderr), _table(tree))


def _resource_remarks(stderr):
    """{mangled kernel name: {remark key: int value}} from the compiler's report."""
    kernels, cur = {}, None
    for line in stderr.splitlines():
        m = re.search(r"remark: Function Name: (\S+)", line)
        if m:
            cur = kernels.setdefault(m.group(1), {})
            continue
        m = re.search(r"remark:\s+([A-Za-z][A-Za-z /\[\]]*?): (\d+) \[-Rpass-analysis", line)
        if m and cur is not None:
            cur[m.group(1).strip()] = int(m.group(2))
    return kernels


_DMA = re.compile(r"fa_fwd_dma_kernelILi(\d+)ELi(\d+)ELi(\d+)ELi\d+ELi(\d+)ELb([01])ELb([01])ELb([01])E")
_PP = re.compile(r"fa_fwd_pp_kernelILi(\d+)ELi(\d+)ELi\d+ELb([01])ELb([01])E")


def _entry_key(row):
    """The template arguments that name table entry `row` = (D, dtype, causal, BM, BN, waves, wg/CU)."""
    d, dtype, causal, _, bn, nw, wg = row
    bf16, v8 = int(dtype in (1, 3)), int(dtype in (2, 3))
    if nw == 8:
        return ("pp", d, bn, bf16, causal)
    return ("dma", d, bn, nw, wg, bf16, causal, v8)


def _remark_key(name):
    m = _DMA.search(name)
    if m:
        d, bn, nw, occ, bf16, causal, v8 = map(int, m.groups())
        return ("dma", d, bn, nw, occ, bf16, causal, v8)
    m = _PP.search(name)
    if m:
        d, bn, bf16, causal = map(int, m.groups())
        return ("pp", d, bn, bf16, causal)
    return None


def _default_kernel_ids():
    """Kernels the library's default tiling or a preset selects, over head dims, dtypes,
    fp8 V, masks and lengths."""
    ids = set()
    for d in (16, 32, 64, 128, 256):
        for dt in (torch.float16, torch.bfloat16):
            for v8 in (None, fa.FP8_V_DTYPE):
                for causal in (False, True):
                    for n in (64, 512, 2048, 8192):
                        ids.add(fa._describe_runtime(2, 4, n, d, causal, dtype=dt, v_dtype=v8)["kernel_id"])
    for dt in (torch.float16, torch.bfloat16):
        for (z, h, n, d, causal) in fa._presets_for(dt):
            ids.add(fa._describe_runtime(z, h, n, d, causal, dtype=dt)["kernel_id"])
    return ids


def _check_resources(remarks, table):
    by_key = {}
    for name, res in remarks.items():
        key = _remark_key(name)
        if key is not None:
            assert key not in by_key, f"two kernels named {key}"
            by_key[key] = (name, res)
    for i, row in enumerate(table):
        name, res = by_key[_entry_key(row)]
        waves_per_simd = row[6] * row[5] // 4
        assert res["Occupancy [waves/SIMD]"] >= waves_per_simd, \
            f"entry {i} ({name}) reaches {res['Occupancy [waves/SIMD]']} waves/SIMD, launched with {waves_per_simd}"
    defaults = _default_kernel_ids()
    assert len(defaults) >= 10
    for i in sorted(defaults):
        name, res = by_key[_entry_key(table[i])]
        assert res["ScratchSize [bytes/lane]"] == 0 and res["VGPRs Spill"] == 0, \
            f"default kernel {i} ({name}) spills: {res}"
    merge = [res for name, res in remarks.items() if "fa_merge_kernel" in name]
    assert len(merge) == 2 and all(r["ScratchSize [bytes/lane]"] == 0 for r in merge)
