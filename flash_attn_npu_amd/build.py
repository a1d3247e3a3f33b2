"""Build recipe for libfa_mi355x.so (the HIP kernels + C ABI) for gfx950.

Plain `hipcc -shared -fPIC` on the one source file: no torch cpp_extension,
no hipify, one code path.  The library lands next to this file so the
in-tree loader (flash_attention_forward._load_library) finds it and it
travels with the source tree.

    python -m flash_attn_npu_amd.build          # or __graft_entry__.build()
"""

from __future__ import annotations

import hashlib
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
SRC = PKG_DIR / "csrc" / "fa_fwd.hip"
PLAN_SRC = PKG_DIR / "csrc" / "fa_plan.cpp"  # included by fa_fwd.hip
INCLUDE_DIR = REPO_DIR / "include"
LIB_NAME = "libfa_mi355x.so"
LIB_PATH = PKG_DIR / LIB_NAME
# Standalone probe of the sustained dense bf16 MFMA rate (a roofline reference point).
PROBE_SRC = PKG_DIR / "csrc" / "mfma_ceiling.hip"
PROBE_PATH = PKG_DIR / "mfma_ceiling"
OFFLOAD_ARCH = os.environ.get("FA_OFFLOAD_ARCH", "gfx950")


def hipcc_path() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: install ROCm or set HIPCC")


def source_hash() -> str:
    """sha256 (first 16 hex digits) of the kernel source, the host planning
    source it includes and the ABI header.

    Compiled into the library as fa_build_id(), so a library older than its
    sources is detectable without a GPU.
    """
    h = hashlib.sha256()
    for path in (SRC, PLAN_SRC, INCLUDE_DIR / "fa_fwd.h"):
        h.update(path.name.encode())
        h.update(b"\0")
        h.update(path.read_bytes())
    return h.hexdigest()[:16]


def compile_command(out: Path = LIB_PATH, extra: list[str] | None = None) -> list[str]:
    return [
        hipcc_path(),
        f"--offload-arch={OFFLOAD_ARCH}",
        "-O3",
        "-std=c++17",
        "-shared",
        "-fPIC",
        # Keep packed-fp32 VALU forms (v_pk_{add,mul,fma}_f32) out of the device code.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wno-unused-command-line-argument",
        f"-I{INCLUDE_DIR}",
        f'-DFA_SOURCE_HASH="{source_hash()}"',
        *(extra or []),
        "-o", str(out),
        str(SRC),
    ]


def build_library(verbose: bool = False) -> Path:
    """Compile the library (always; a stale .so is replaced atomically)."""
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = compile_command(tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # The host pass warns that it does not know the packed-fp32 feature; drop that noise.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def build_probe() -> Path:
    """Compile the MFMA-rate probe executable (always; replaced atomically)."""
    tmp = PROBE_PATH.with_name(PROBE_PATH.name + ".tmp")
    cmd = [hipcc_path(), f"--offload-arch={OFFLOAD_ARCH}", "-O3", "-std=c++17",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-Wno-unused-command-line-argument", "-o", str(tmp), str(PROBE_SRC)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{proc.stderr}")
    os.replace(tmp, PROBE_PATH)
    return PROBE_PATH


if __name__ == "__main__":
    print(build_library(verbose=True))
    print(build_probe())
