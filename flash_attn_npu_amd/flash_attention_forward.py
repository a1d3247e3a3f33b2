"""FlashAttention forward for AMD Instinct MI355X -- drop-in for the reference
module `flash_attention_forward.py` (ZyEng-Art/flash_attn_npu).

Callers use this file exactly as they use the reference: import it, or load it
by path (evaluate_attention.py:55-59 uses importlib's spec_from_file_location),
read `DEVICE`, and call

    attention(q, k, v, causal, sm_scale, BM=None, BN=None, return_lse=False)

(flash_attention_forward.py:1197-1201).  `flash_attention_forward` is the same
function under the name the task statement uses.  q, k, v are BNSD
[Z, H, N_CTX, HEAD_DIM] fp16/bf16 tensors on the GPU; the result is O in the
input dtype and, with return_lse=True, the fp32 natural-log row LSE [Z, H, N].

Below this module is one C-ABI call (`fa_fwd` in libfa_mi355x.so, declared in
include/fa_fwd.h) that launches the hand-written gfx950 kernel on the current
stream.  There is no other implementation: without the library, or on a
non-GPU tensor, the call raises.

The file is self-contained (no package-relative imports) so it can be loaded
by path like the reference.
"""

from __future__ import annotations

import ctypes
import math
import os
from pathlib import Path

import torch

DEVICE = "cuda"
RESULT_DIR_NAME = "result_dir"
# 0 = the library's persistent grid (as many workgroups as are resident at
# once: 512 for 4-wave kernels on 256 CUs); >0 sets the program count.  Either
# way every workgroup walks its share of the balanced tile schedule (the
# reference's persistent grid, flash_attention_forward.py:24,616-623).
DEFAULT_PERSISTENT_PROGRAMS = 0
# 0 = the library's split-KV choice (fa_default_kv_splits: only grids of at
# most half a tile per CU, into runs that stay long); KV_SPLITS in [1, 64]
# overrides.
DEFAULT_KV_SPLITS = 0
# Name prefix of the attention kernels in a profiler trace (fa_fwd_dma_kernel,
# fa_fwd_pp_kernel); the reference names its Triton kernel here
# (flash_attention_forward.py:25).
PROFILE_OP_NAME = "fa_fwd"
LIB_NAME = "libfa_mi355x.so"
SUPPORTED_HEAD_DIMS = (16, 32, 64, 128, 256)
# The reference accepts these head dims (flash_attention_forward.py:1121-1122).
REFERENCE_HEAD_DIMS = (16, 32, 64, 128, 256)

# BEGIN AUTO-TUNED DEFAULT TILING PRESETS
# (Z, H, N_CTX, HEAD_DIM, causal) -> (BLOCK_M, BLOCK_N), rewritten by
# python -m flash_attn_npu_amd.tune from gfx950 sweeps: float16 inputs here,
# bfloat16 inputs in DEFAULT_TILING_PRESETS_BF16.
DEFAULT_TILING_PRESETS = {
    (1, 8, 512, 64, False): (128, 128),
    (16, 16, 1024, 64, False): (128, 64),
    (128, 8, 1024, 128, True): (128, 64),
    (128, 8, 1024, 256, True): (128, 32),
    (128, 8, 2048, 128, True): (128, 64),
    (128, 8, 2048, 256, False): (128, 32),
    (128, 8, 4096, 128, False): (128, 32),
    (128, 8, 8192, 64, False): (128, 64),
}
DEFAULT_TILING_PRESETS_BF16 = {
    (2, 16, 8192, 128, True): (128, 64),
    (4, 32, 2048, 128, True): (128, 64),
    (8, 32, 3000, 128, True): (128, 64),
    (128, 8, 1024, 128, True): (128, 64),
    (128, 8, 1024, 256, True): (128, 32),
    (128, 8, 2048, 128, True): (128, 64),
    (128, 8, 2048, 256, False): (128, 32),
    (128, 8, 4096, 128, False): (128, 32),
    (128, 8, 8192, 64, False): (128, 64),
}
# END AUTO-TUNED DEFAULT TILING PRESETS


class _PresetTable(dict):
    """A preset table that counts its changes, so the cached launch plans (which hold
    the resolved tiling) follow a table edited in a live process the way the
    reference, which reads its presets on every call, does.  Replacing a table
    by another object is seen through its identity; a plain dict put in its
    place is only followed when it is replaced again."""

    version = 0

    def _changed(self):
        _PresetTable.version += 1

    def __setitem__(self, key, value):
        super().__setitem__(key, value)
        self._changed()

    def __delitem__(self, key):
        super().__delitem__(key)
        self._changed()

    def update(self, *args, **kwargs):
        super().update(*args, **kwargs)
        self._changed()

    def pop(self, *args):
        out = super().pop(*args)
        self._changed()
        return out

    def popitem(self):
        out = super().popitem()
        self._changed()
        return out

    def setdefault(self, key, default=None):
        out = super().setdefault(key, default)
        self._changed()
        return out

    def clear(self):
        super().clear()
        self._changed()

    def __ior__(self, other):
        out = super().__ior__(other)
        self._changed()
        return out


DEFAULT_TILING_PRESETS = _PresetTable(DEFAULT_TILING_PRESETS)
DEFAULT_TILING_PRESETS_BF16 = _PresetTable(DEFAULT_TILING_PRESETS_BF16)

# --------------------------------------------------------------------------
# C ABI binding (include/fa_fwd.h)

FA_OK = 0
FA_ERR_LAUNCH = -100
_ARGUMENT_ERRORS = {-1, -2, -3, -4, -5, -6, -7, -8, -9, -10}
FA_CFG_COUNT = 8
FA_DTYPE = {torch.float16: 0, torch.bfloat16: 1}
# fp8-e5m2 V with fp16 / bf16 q, k, o: dtype code + FA_DTYPE_V_E5M2_OFFSET
# (FA_DTYPE_FP16_V_E5M2 = 2, FA_DTYPE_BF16_V_E5M2 = 3).
FP8_V_DTYPE = torch.float8_e5m2
FA_DTYPE_V_E5M2_OFFSET = 2
FP8_V_HEAD_DIMS = (16, 32, 64, 128, 256)


def fp8_v_tiling(head_dim):
    """(BLOCK_M, BLOCK_N) of the fp8-V kernels: 64-key tiles, 128 at D = 16."""
    return (128, 128) if head_dim == 16 else (128, 64)

_DTYPE_NAMES = {0: "float16", 1: "bfloat16", 2: "float16+float8_e5m2_v", 3: "bfloat16+float8_e5m2_v"}


class FaFwdParams(ctypes.Structure):
    """Mirror of `fa_fwd_params` (include/fa_fwd.h)."""

    _fields_ = [
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p),
        ("lse", ctypes.c_void_p),
        ("q_stride", ctypes.c_int64 * 4),
        ("k_stride", ctypes.c_int64 * 4),
        ("v_stride", ctypes.c_int64 * 4),
        ("o_stride", ctypes.c_int64 * 4),
        ("B", ctypes.c_int32),
        ("H", ctypes.c_int32),
        ("Sq", ctypes.c_int32),
        ("Sk", ctypes.c_int32),
        ("D", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("causal", ctypes.c_int32),
        ("sm_scale", ctypes.c_float),
        ("block_m", ctypes.c_int32),
        ("block_n", ctypes.c_int32),
        ("num_programs", ctypes.c_int32),
    ]


_LIB = None


def library_path() -> Path:
    override = os.environ.get("FA_MI355X_LIB")
    if override:
        return Path(override)
    return Path(__file__).resolve().parent / LIB_NAME


def _load_library():
    """Load libfa_mi355x.so once; raise if it has not been built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    path = library_path()
    if not path.exists():
        raise RuntimeError(
            f"{path} is missing: build it first (python -m flash_attn_npu_amd.build, "
            "or __graft_entry__.build()). There is no fallback implementation."
        )
    lib = ctypes.CDLL(str(path))
    P = ctypes.POINTER(FaFwdParams)
    I32P = ctypes.POINTER(ctypes.c_int32)
    lib.fa_fwd.argtypes = [P, ctypes.c_void_p]
    lib.fa_fwd.restype = ctypes.c_int
    lib.fa_validate.argtypes = [P]
    lib.fa_validate.restype = ctypes.c_int
    lib.fa_query_config.argtypes = [P, I32P]
    lib.fa_query_config.restype = ctypes.c_int
    lib.fa_error_string.argtypes = [ctypes.c_int]
    lib.fa_error_string.restype = ctypes.c_char_p
    lib.fa_abi_version.argtypes = []
    lib.fa_abi_version.restype = ctypes.c_int
    lib.fa_num_kernels.argtypes = []
    lib.fa_num_kernels.restype = ctypes.c_int
    lib.fa_kernel_info.argtypes = [ctypes.c_int, I32P]
    lib.fa_kernel_info.restype = ctypes.c_int
    lib.fa_params_size.argtypes = []
    lib.fa_params_size.restype = ctypes.c_int
    lib.fa_kernel_wg_per_cu.argtypes = [ctypes.c_int]
    lib.fa_kernel_wg_per_cu.restype = ctypes.c_int
    lib.fa_build_id.argtypes = []
    lib.fa_build_id.restype = ctypes.c_char_p
    lib.fa_split_workspace_bytes.argtypes = [P, ctypes.c_int32]
    lib.fa_split_workspace_bytes.restype = ctypes.c_int64
    lib.fa_fwd_split.argtypes = [P, ctypes.c_int32, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
    lib.fa_fwd_split.restype = ctypes.c_int
    lib.fa_fwd_split_static.argtypes = [P, ctypes.c_int32, ctypes.c_void_p]
    lib.fa_fwd_split_static.restype = ctypes.c_int
    lib.fa_default_kv_splits.argtypes = [P]
    lib.fa_default_kv_splits.restype = ctypes.c_int32
    if lib.fa_params_size() != ctypes.sizeof(FaFwdParams):
        raise RuntimeError("fa_fwd_params layout mismatch between the library and this binding")
    _LIB = lib
    return lib


def _check(rc: int, what: str) -> None:
    if rc == FA_OK:
        return
    msg = f"{what}: {_load_library().fa_error_string(rc).decode()} (code {rc})"
    if rc in _ARGUMENT_ERRORS:
        raise ValueError(msg)
    raise RuntimeError(msg)


def kernel_table():
    """All kernel instances in the library: dicts of D, dtype, causal, BLOCK_M, BLOCK_N,
    waves and resident workgroups per CU."""
    lib = _load_library()
    out = (ctypes.c_int32 * 6)()
    rows = []
    for i in range(lib.fa_num_kernels()):
        _check(lib.fa_kernel_info(i, out), "fa_kernel_info")
        wg = lib.fa_kernel_wg_per_cu(i)
        _check(wg if wg < 0 else 0, "fa_kernel_wg_per_cu")
        rows.append({"HEAD_DIM": out[0], "dtype": _DTYPE_NAMES.get(out[1], str(out[1])),
                     "causal": bool(out[2]), "BLOCK_M": out[3], "BLOCK_N": out[4], "waves": out[5],
                     "wg_per_cu": wg})
    return rows


# --------------------------------------------------------------------------
# Tiling policy (flash_attention_forward.py:156-252, 616-644)

def _get_kv_splits():
    """Split-KV factor from $KV_SPLITS (1 = never split), else 0 = the library's choice."""
    raw = os.environ.get("KV_SPLITS")
    if raw is None:
        return DEFAULT_KV_SPLITS
    value = int(raw)
    if not 1 <= value <= 64:
        raise ValueError("KV_SPLITS must be in [1, 64]")
    return value


def _get_persistent_programs():
    """Program count from $PERSISTENT_PROGRAMS (>= 1), else 0 = the library's resident grid.

    Same variable and check as flash_attention_forward.py:616-623.
    """
    raw = os.environ.get("PERSISTENT_PROGRAMS")
    if raw is None:
        return DEFAULT_PERSISTENT_PROGRAMS
    value = int(raw)
    if value < 1:
        raise ValueError("PERSISTENT_PROGRAMS must be >= 1")
    return value


def _shape_params(z, h, n_ctx, head_dim, causal, bm=0, bn=0, dtype=torch.float16, programs=0):
    p = FaFwdParams()
    p.B, p.H, p.Sq, p.Sk, p.D = z, h, n_ctx, n_ctx, head_dim
    p.dtype = FA_DTYPE.get(dtype, -1)
    p.causal = 1 if causal else 0
    p.sm_scale = 1.0
    p.block_m, p.block_n = bm or 0, bn or 0
    p.num_programs = programs
    return p


def _query_config(z, h, n_ctx, head_dim, causal, bm=0, bn=0, dtype=torch.float16, programs=0):
    lib = _load_library()
    out = (ctypes.c_int32 * FA_CFG_COUNT)()
    p = _shape_params(z, h, n_ctx, head_dim, causal, bm, bn, dtype, programs)
    _check(lib.fa_query_config(ctypes.byref(p), out), "fa_query_config")
    return list(out)


# The library's default tiling is a pure function of the shape: asked once per shape.
_FALLBACK_TILING = {}


def _presets_for(dtype):
    """The preset table of an input dtype: the reference's table for float16, a second
    one for bfloat16 (each filled by a sweep in that dtype)."""
    return DEFAULT_TILING_PRESETS_BF16 if dtype == torch.bfloat16 else DEFAULT_TILING_PRESETS


def _default_tiling(z, h, n_ctx, head_dim, causal, dtype=torch.float16):
    """Preset for this exact shape and dtype, else the library's gfx950 default."""
    key = (z, h, n_ctx, head_dim, causal)
    preset = _presets_for(dtype).get(key)
    if preset is not None:
        return preset
    fkey = key + (dtype,)
    tiling = _FALLBACK_TILING.get(fkey)
    if tiling is None:
        cfg = _query_config(z, h, n_ctx, head_dim, causal, dtype=dtype)
        tiling = _FALLBACK_TILING[fkey] = (cfg[0], cfg[1])
    return tiling


def get_tiling(z, h, n_ctx, head_dim, causal, dtype=torch.float16):
    return _default_tiling(z, h, n_ctx, head_dim, causal, dtype)


def get_tiling_source(z, h, n_ctx, head_dim, causal, dtype=torch.float16):
    if (z, h, n_ctx, head_dim, causal) in _presets_for(dtype):
        return "preset"
    return "fallback"


def _resolve_tiling(z, h, n_ctx, head_dim, causal, bm=None, bn=None, dtype=torch.float16):
    if (bm is None) != (bn is None):
        raise ValueError("BM and BN must be provided together")
    if bm is not None:
        return bm, bn, "override"
    return (*get_tiling(z, h, n_ctx, head_dim, causal, dtype),
            get_tiling_source(z, h, n_ctx, head_dim, causal, dtype))


def _describe_runtime(z, h, n_ctx, head_dim, causal, bm=None, bn=None, dtype=torch.float16, v_dtype=None):
    """What a call with this shape would launch (flash_attention_forward.py:634-644).

    dtype is the q/k/o element type and v_dtype V's (None: the same; float8_e5m2 selects
    the fp8-V kernels, as _launch_kernel does).
    """
    block_m, block_n, tiling_source = _resolve_tiling(z, h, n_ctx, head_dim, causal, bm, bn, dtype)
    fp8_v = v_dtype == FP8_V_DTYPE
    if fp8_v and tiling_source != "override":
        block_m, block_n = fp8_v_tiling(head_dim)
    programs = _get_persistent_programs()
    lib = _load_library()
    p = _shape_params(z, h, n_ctx, head_dim, causal, block_m, block_n, dtype, programs)
    if fp8_v:
        p.dtype += FA_DTYPE_V_E5M2_OFFSET
    out = (ctypes.c_int32 * FA_CFG_COUNT)()
    _check(lib.fa_query_config(ctypes.byref(p), out), "fa_query_config")
    cfg = list(out)
    splits = _get_kv_splits()
    if splits == 0:
        splits = int(lib.fa_default_kv_splits(ctypes.byref(p)))
    return {
        "selected_config": {"BLOCK_M": cfg[0], "BLOCK_N": cfg[1]},
        "tiling_source": tiling_source,
        "total_tiles": cfg[4],
        "launched_programs": cfg[3],
        "stage": cfg[6],
        "waves": cfg[2],
        "lds_bytes": cfg[5],
        "kernel_id": cfg[7],
        "kv_splits": splits,
    }


# --------------------------------------------------------------------------
# Operator

def _validate_inputs(q, k, v):
    """The reference's checks (flash_attention_forward.py:1114-1122) plus dtype/device."""
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("q, k, v must all be 4D tensors shaped [Z, H, N_CTX, HEAD_DIM]")
    if q.shape != k.shape or q.shape != v.shape:
        raise ValueError("q, k, v must have the same shape")
    if q.device != k.device or q.device != v.device:
        raise ValueError("q, k, v must be on the same device")
    if q.shape[-1] not in REFERENCE_HEAD_DIMS:
        raise ValueError("HEAD_DIM must be one of {16, 32, 64, 128, 256}")
    if q.shape[-1] not in SUPPORTED_HEAD_DIMS:
        raise ValueError(f"HEAD_DIM={q.shape[-1]} is not supported by this library "
                         f"(supported: {SUPPORTED_HEAD_DIMS})")
    if q.dtype not in FA_DTYPE or k.dtype != q.dtype or (v.dtype != q.dtype and v.dtype != FP8_V_DTYPE):
        raise ValueError("q, k, v must all be float16 or all be bfloat16 (v may also be float8_e5m2)")
    if v.dtype == FP8_V_DTYPE and q.shape[-1] not in FP8_V_HEAD_DIMS:
        raise ValueError(f"a float8_e5m2 v is supported for HEAD_DIM in {FP8_V_HEAD_DIMS}")
    if q.device.type != "cuda":
        raise ValueError(f"q, k, v must be GPU tensors (device 'cuda'), got {q.device}")


def _kernel_ready(t):
    """A view the kernel can read directly: dim stride 1, 16-byte rows, 16B-aligned base.

    Anything else is copied into a fresh dense tensor (whose base the caching allocator
    aligns), including a contiguous view at an odd storage offset: contiguous() would
    return that same misaligned view.
    """
    ptr = t.data_ptr()
    if ptr % 16 == 0 and t.is_contiguous():
        return t  # rows of D >= 16 elements: every stride is a multiple of 16 bytes
    st = t.stride()
    align = 16 // t.element_size()
    if ptr % 16 or st[3] != 1 or any(s % align for s in st[:3]) or (t.shape[2] > 1 and st[2] < t.shape[3]):
        return t.clone(memory_format=torch.contiguous_format)
    return t


class _LaunchPlan:
    """Everything a launch needs that depends only on the call's configuration:
    the parameter block (shape, strides, dtype, mask, tiling, program count), the
    split count and its workspace size.  Built once per configuration."""

    __slots__ = ("params", "splits", "workspace_bytes", "lse_shape")

    def __init__(self, params, splits, workspace_bytes, lse_shape):
        self.params = params
        self.splits = splits
        self.workspace_bytes = workspace_bytes
        self.lse_shape = lse_shape


# Launch plans keyed by (shapes, strides, dtypes, causal, resolved tiling, program
# count, split override): a call only copies the block and sets its pointers and scale.
# Both plan caches are emptied when they reach _MAX_CACHED_PLANS entries (a process that
# sees that many configurations rebuilds them as it goes).
_PLANS = {}
_MAX_CACHED_PLANS = 4096


def _launch_plan(lib, q, k, v, out, causal, bm, bn, programs, split_env):
    key = (q.shape, q.stride(), k.stride(), v.stride(), out.stride(), q.dtype, v.dtype, causal, bm, bn,
           programs, split_env)
    plan = _PLANS.get(key)
    if plan is not None:
        return plan
    z, h, n_ctx, head_dim = q.shape
    p = FaFwdParams()
    p.q_stride[:] = q.stride()
    p.k_stride[:] = k.stride()
    p.v_stride[:] = v.stride()
    p.o_stride[:] = out.stride()
    p.B, p.H, p.Sq, p.Sk, p.D = z, h, n_ctx, n_ctx, head_dim
    p.dtype = FA_DTYPE[q.dtype] + (FA_DTYPE_V_E5M2_OFFSET if v.dtype == FP8_V_DTYPE else 0)
    p.causal = 1 if causal else 0
    p.block_m, p.block_n = int(bm), int(bn)
    p.num_programs = programs
    splits = split_env if split_env else int(lib.fa_default_kv_splits(ctypes.byref(p)))
    nbytes = 0
    if splits > 1:
        nbytes = int(lib.fa_split_workspace_bytes(ctypes.byref(p), splits))
        _check(nbytes if nbytes < 0 else 0, "fa_split_workspace_bytes")
    if len(_PLANS) >= _MAX_CACHED_PLANS:
        _PLANS.clear()
    plan = _PLANS[key] = _LaunchPlan(p, splits, nbytes, (z, h, n_ctx))
    return plan


# Calls whose q, k, v the kernel reads in place, keyed by everything the argument checks,
# the tiling and the launch plan depend on (shapes, strides, dtypes, devices, mask,
# BM/BN override, the two environment variables, the preset tables' identity and change
# count): a repeated call goes straight to
# allocation and launch.  Tensors at a base address that is not 16-byte aligned take
# the full path (and are copied there).
_FAST_PLANS = {}


# The two variables are read on every call.  On POSIX os.environ keeps its entries in a
# plain dict of bytes (shared with os.environb and updated by every change made through
# either): a lookup there costs ~0.1 us, against ~1.5 us through os.environ.get, which
# encodes the key and decodes the value on every access.
_ENV_BYTES = getattr(os.environ, "_data", None) if os.name == "posix" else None
if not isinstance(_ENV_BYTES, dict):
    _ENV_BYTES = None


def _env_key():
    if _ENV_BYTES is not None:
        return _ENV_BYTES.get(b"PERSISTENT_PROGRAMS"), _ENV_BYTES.get(b"KV_SPLITS")
    env = os.environ
    return env.get("PERSISTENT_PROGRAMS"), env.get("KV_SPLITS")


def _call_key(q, k, v, causal, bm, bn):
    return (q.shape, k.shape, v.shape, q.stride(), k.stride(), v.stride(), q.dtype, k.dtype, v.dtype,
            q.get_device(), k.get_device(), v.get_device(), causal, bm, bn, _env_key(),
            _PresetTable.version, id(DEFAULT_TILING_PRESETS), id(DEFAULT_TILING_PRESETS_BF16))


def _launch_kernel(q, k, v, causal, sm_scale, bm=None, bn=None):
    """Validate, resolve tiling, allocate O/LSE, launch; returns (out, lse).

    Same flow and return value as flash_attention_forward.py:1130-1194.
    """
    causal = bool(causal)
    key = _call_key(q, k, v, causal, bm, bn)
    plan = _FAST_PLANS.get(key)
    if plan is not None and not (q.data_ptr() | k.data_ptr() | v.data_ptr()) & 15:
        out = torch.empty_like(q)
        lse = q.new_empty(plan.lse_shape, dtype=torch.float32)
        _launch(plan, q, k, v, out, lse, sm_scale)
        return out, lse
    _validate_inputs(q, k, v)
    z, h, n_ctx, head_dim = q.shape
    bm_r, bn_r, source = _resolve_tiling(z, h, n_ctx, head_dim, causal, bm, bn, q.dtype)
    if v.dtype == FP8_V_DTYPE and source != "override":
        bm_r, bn_r = fp8_v_tiling(head_dim)  # the fp8-V kernels' one tiling; presets are for 16-bit V
    qr, kr, vr = _kernel_ready(q), _kernel_ready(k), _kernel_ready(v)
    out = torch.empty_like(qr)
    lse = torch.empty((z, h, n_ctx), device=q.device, dtype=torch.float32)
    if out.numel() == 0:
        return out, lse
    out_r = _kernel_ready(out)
    lib = _load_library()
    plan = _launch_plan(lib, qr, kr, vr, out_r, causal, bm_r, bn_r, _get_persistent_programs(), _get_kv_splits())
    _launch(plan, qr, kr, vr, out_r, lse, sm_scale)
    if qr is q and kr is k and vr is v and out_r is out:
        if len(_FAST_PLANS) >= _MAX_CACHED_PLANS:
            _FAST_PLANS.clear()
        _FAST_PLANS[key] = plan
    return out_r, lse


def _launch(plan, q, k, v, out, lse, sm_scale):
    sm_scale = float(sm_scale)
    if not math.isfinite(sm_scale):
        raise ValueError("sm_scale must be finite")
    lib = _LIB
    p = FaFwdParams.from_buffer_copy(plan.params)
    p.q, p.k, p.v, p.o, p.lse = q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr()
    p.sm_scale = sm_scale
    dev = q.get_device()
    if dev == _current_device():
        _launch_on(lib, p, plan, dev, q)
    else:
        with torch.cuda.device(dev):
            _launch_on(lib, p, plan, dev, q)


def _launch_on(lib, p, plan, dev, q):
    """Launch on the current stream of device `dev` (the current device, q's)."""
    stream = _current_raw_stream(dev)
    pp = ctypes.byref(p)
    if plan.splits > 1:
        workspace = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=q.device)  # 512 B aligned
        _check(lib.fa_fwd_split(pp, plan.splits, workspace.data_ptr(), plan.workspace_bytes, stream),
               "fa_fwd_split")
    else:
        _check(lib.fa_fwd(pp, stream), "fa_fwd")


# torch's own accessors for the current device and raw stream, resolved once (the
# public torch.cuda.current_device / current_stream(dev).cuda_stream are the fallback).
_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_GET_DEVICE = getattr(torch._C, "_cuda_getDevice", None)


def _current_raw_stream(dev):
    """hipStream_t of torch's current stream on device `dev`, as an int."""
    if _RAW_STREAM is not None:
        return _RAW_STREAM(dev)
    return torch.cuda.current_stream(dev).cuda_stream


def _current_device():
    return _GET_DEVICE() if _GET_DEVICE is not None else torch.cuda.current_device()


def attention(q, k, v, causal, sm_scale, BM=None, BN=None, return_lse=False):
    out, lse = _launch_kernel(q, k, v, causal, sm_scale, bm=BM, bn=BN)
    if return_lse:
        return out, lse
    return out


flash_attention_forward = attention


def _dtype_from_name(name):
    normalized = name.strip().lower()
    if normalized in {"float16", "fp16"}:
        return torch.float16
    if normalized in {"bfloat16", "bf16"}:
        return torch.bfloat16
    raise ValueError(f"Unsupported dtype: {name}")


def _make_inputs(z, h, n_ctx, head_dim, dtype):
    """N(0, 0.5) q, k, v on DEVICE, as flash_attention_forward.py:1308-1312."""
    q = torch.empty((z, h, n_ctx, head_dim), dtype=dtype, device=DEVICE).normal_(mean=0.0, std=0.5)
    k = torch.empty((z, h, n_ctx, head_dim), dtype=dtype, device=DEVICE).normal_(mean=0.0, std=0.5)
    v = torch.empty((z, h, n_ctx, head_dim), dtype=dtype, device=DEVICE).normal_(mean=0.0, std=0.5)
    return q, k, v


__all__ = [
    "DEVICE",
    "RESULT_DIR_NAME",
    "PROFILE_OP_NAME",
    "DEFAULT_TILING_PRESETS",
    "DEFAULT_TILING_PRESETS_BF16",
    "get_tiling",
    "get_tiling_source",
    "attention",
    "flash_attention_forward",
    "kernel_table",
]
