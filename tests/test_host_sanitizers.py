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
  the tree, so the boundary tests never pass on a stale build.
"""

from __future__ import annotations

import ctypes
import os
import shutil
import subprocess
from pathlib import Path

import pytest

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
    proc = subprocess.run(B.compile_command(out), capture_output=True, text=True, timeout=900)
    assert proc.returncode == 0, proc.stderr[-4000:]
    fresh = ctypes.CDLL(str(out))
    fresh.fa_build_id.restype = ctypes.c_char_p
    tree = fa._load_library()
    assert fresh.fa_build_id().decode() == B.source_hash() == tree.fa_build_id().decode(), \
        "the library in the tree was not built from the current sources"
    assert _table(fresh) == _table(tree)
    assert fresh.fa_params_size() == tree.fa_params_size() == ctypes.sizeof(fa.FaFwdParams)
