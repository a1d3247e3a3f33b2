"""GPU: the no-allocation split-KV entry point, fa_fwd_split_static.

It runs the kernels of fa_fwd_split with the partial results in the library's
static device buffer instead of a caller workspace, so its outputs must equal
fa_fwd_split's bit for bit (same kernels, same split count, same arithmetic).
Two calls in a row, the second on a smaller input, check that nothing the
first call left in the shared buffer leaks into the second.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

FA_STATIC_SCRATCH_BYTES = 32 * 1024 * 1024
FA_ERR_SCRATCH = -10


def _params(fa, q, k, v, o, lse, causal, scale):
    p = fa.FaFwdParams()
    p.q, p.k, p.v, p.o, p.lse = q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr()
    p.q_stride[:] = q.stride()
    p.k_stride[:] = k.stride()
    p.v_stride[:] = v.stride()
    p.o_stride[:] = o.stride()
    B, H, S, D = q.shape
    p.B, p.H, p.Sq, p.Sk, p.D = B, H, S, S, D
    p.dtype = fa.FA_DTYPE[q.dtype]
    p.causal = 1 if causal else 0
    p.sm_scale = scale
    return p


def _inputs(seed, shape, dtype):
    g = torch.Generator().manual_seed(seed)
    return tuple(torch.randn(shape, generator=g).to(dtype).cuda() for _ in range(3))


def _run_pair(fa, lib, q, k, v, causal, scale, splits):
    """(O, LSE) from fa_fwd_split with a torch workspace and from fa_fwd_split_static."""
    stream = fa._current_raw_stream(q.device.index)
    outs = []
    for static in (False, True):
        o = torch.full_like(q, float("nan"))
        lse = torch.full(q.shape[:3], float("nan"), device=q.device, dtype=torch.float32)
        p = _params(fa, q, k, v, o, lse, causal, scale)
        if static:
            rc = lib.fa_fwd_split_static(ctypes.byref(p), splits, stream)
        else:
            nbytes = int(lib.fa_split_workspace_bytes(ctypes.byref(p), splits))
            ws = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
            rc = lib.fa_fwd_split(ctypes.byref(p), splits, ws.data_ptr(), nbytes, stream)
        assert rc == 0, lib.fa_error_string(rc)
        torch.cuda.synchronize()
        outs.append((o, lse))
    return outs


@pytest.mark.parametrize("dtype,causal,first,second,splits", [
    (torch.bfloat16, True, (2, 4, 1500, 128), (1, 3, 700, 128), 3),
    (torch.float16, False, (1, 8, 2048, 64), (1, 2, 333, 64), 4),
])
def test_static_split_matches_workspace_split(fa, dtype, causal, first, second, splits):
    lib = fa._load_library()
    for seed, shape in ((31, first), (32, second)):
        print(f"[no-alloc] {tuple(shape)} {dtype} causal={causal} splits={splits}", flush=True)
        q, k, v = _inputs(seed, shape, dtype)
        (o_ws, l_ws), (o_st, l_st) = _run_pair(fa, lib, q, k, v, causal, shape[3] ** -0.5, splits)
        assert torch.isfinite(o_st).all() and torch.isfinite(l_st).all()
        assert torch.equal(o_st, o_ws) and torch.equal(l_st, l_ws)


def test_static_split_rejects_oversize(fa):
    lib = fa._load_library()
    shape = (2, 16, 4096, 128)  # 3 splits: 2*16*4096*128*4*3 bytes of partial O, > 32 MiB
    q, k, v = (torch.empty(shape, dtype=torch.bfloat16, device="cuda") for _ in range(3))
    o = torch.empty_like(q)
    lse = torch.empty(shape[:3], device="cuda", dtype=torch.float32)
    p = _params(fa, q, k, v, o, lse, True, 0.088)
    assert lib.fa_split_workspace_bytes(ctypes.byref(p), 3) > FA_STATIC_SCRATCH_BYTES
    assert lib.fa_fwd_split_static(ctypes.byref(p), 3, fa._current_raw_stream(0)) == FA_ERR_SCRATCH
    assert lib.fa_fwd_split_static(ctypes.byref(p), 0, fa._current_raw_stream(0)) == -9


def _capture(lib, p, splits, stream_of):
    """A CUDA/HIP graph holding one fa_fwd_split_static launch."""
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rc = lib.fa_fwd_split_static(ctypes.byref(p), splits, stream_of())
    assert rc == 0, lib.fa_error_string(rc)
    return g


def test_static_split_in_graph_capture(fa):
    # The entry point's launches recorded into a graph (no counters, no
    # allocation, no memset): every replay, with eager calls of the
    # workspace entry point between them, equals the eager result bit for bit.
    lib = fa._load_library()
    dtype, causal, shape, splits = torch.bfloat16, True, (1, 4, 1200, 128), 3
    print(f"[no-alloc graph] {shape} {dtype} causal={causal} splits={splits}", flush=True)
    q, k, v = _inputs(41, shape, dtype)
    scale = shape[3] ** -0.5
    (o_ws, l_ws), _ = _run_pair(fa, lib, q, k, v, causal, scale, splits)
    o = torch.full_like(q, float("nan"))
    lse = torch.full(q.shape[:3], float("nan"), device=q.device, dtype=torch.float32)
    p = _params(fa, q, k, v, o, lse, causal, scale)
    g = _capture(lib, p, splits, lambda: fa._current_raw_stream(q.device.index))
    for r in range(3):
        o.fill_(float("nan"))
        lse.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(o, o_ws) and torch.equal(lse, l_ws), f"replay {r}"
        _run_pair(fa, lib, q, k, v, causal, scale, splits)  # eager work between replays


_CHILD = r"""
import ctypes, sys
import torch
sys.path.insert(0, sys.argv[1])
sys.path.insert(0, sys.argv[1] + "/tests")
from flash_attn_npu_amd import flash_attention_forward as fa
import test_zz_no_alloc as t
lib = fa._load_library()
q, k, v = t._inputs(43, (1, 2, 900, 64), torch.float16)
o = torch.empty_like(q)
lse = torch.empty(q.shape[:3], device="cuda", dtype=torch.float32)
p = t._params(fa, q, k, v, o, lse, False, 0.125)
# The first call of the library on this device is the captured one.
g = t._capture(lib, p, 2, lambda: fa._current_raw_stream(0))
g.replay(); g.replay()
torch.cuda.synchronize()
(o_ws, l_ws), _ = t._run_pair(fa, lib, q, k, v, False, 0.125, 2)
assert torch.equal(o, o_ws) and torch.equal(lse, l_ws)
print("CAPTURE-FIRST-OK", flush=True)
"""


def test_static_split_first_call_inside_capture():
    # In a fresh process the entry point resolves its device buffer on its
    # first call on a device; here that call is being captured.
    import subprocess
    import sys
    from pathlib import Path
    repo = str(Path(__file__).resolve().parent.parent)
    print("[no-alloc graph] first library call inside a capture (child process)", flush=True)
    proc = subprocess.run([sys.executable, "-c", _CHILD, repo], capture_output=True, text=True, timeout=300)
    assert proc.returncode == 0 and "CAPTURE-FIRST-OK" in proc.stdout, proc.stdout[-2000:] + proc.stderr[-3000:]
