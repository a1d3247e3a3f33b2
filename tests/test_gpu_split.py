"""GPU: split-KV (fa_fwd_split + the merge kernel) against float64 and the oracle.

Split-KV has no counterpart in the reference; its arithmetic is pinned in
the oracle by the partition identity (tests/test_oracle.py).  Here the HIP
path, with forced split counts, must meet the same gates as the unsplit
kernel: max|dO| <= 5e-3 (fp16) / 2e-2 (bf16), max|dLSE| <= 1e-3.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from flash_attn_npu_amd import workloads as W
from oracle.attention_oracle import attention_partial, attention_ref, merge_partials
from tests.gpu_reference import attention_fp64

pytestmark = pytest.mark.gpu

O_TOL = {torch.float16: 5e-3, torch.bfloat16: 2e-2}


def _inputs(seed, shape, dtype):
    g = torch.Generator().manual_seed(seed)
    return tuple((torch.randn(shape, generator=g) * 0.7).to(dtype).cuda() for _ in range(3))


@pytest.mark.parametrize("splits", [2, 3, 7, 64])
@pytest.mark.parametrize("d", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
def test_forced_splits_vs_fp64(fa, monkeypatch, splits, d, causal):
    dtype = torch.bfloat16 if d in (128, 256) else torch.float16
    print(f"[split] splits={splits} D={d} causal={causal}", flush=True)
    q, k, v = _inputs(31 + d + splits, (1, 3, 1000, d), dtype)
    monkeypatch.setenv("KV_SPLITS", str(splits))
    out, lse = fa.attention(q, k, v, causal, 0.2, return_lse=True)
    o64, l64 = attention_fp64(q, k, v, causal, 0.2)
    assert (out.float() - o64.to(dtype).float()).abs().max().item() <= O_TOL[dtype]
    assert (lse.double() - l64).abs().max().item() <= 1e-3


def test_split_matches_oracle_merge(fa, monkeypatch):
    """The kernel's split result against the oracle's own partial + merge path."""
    q, k, v = _inputs(41, (1, 2, 300, 64), torch.float16)
    monkeypatch.setenv("KV_SPLITS", "3")
    out, lse = fa.attention(q, k, v, True, 0.125, return_lse=True)
    bn = 64                                   # BLOCK_N of the D = 64 kernel
    kv_tiles = (300 + bn - 1) // bn           # 5
    run = (kv_tiles + 2) // 3 * bn            # split_tiles (ceil(5 / 3) = 2) * BN keys per run
    for h in range(2):
        qh, kh, vh = (t[0, h].float().cpu().numpy() for t in (q, k, v))
        parts = [attention_partial(qh, kh, vh, True, 0.125, lo, lo + run) for lo in range(0, 300, run)]
        o_m, l_m = merge_partials(parts)
        o_full, l_full = attention_ref(qh, kh, vh, True, 0.125)
        assert np.abs(o_m - o_full).max() < 1e-5 and np.abs(l_m - l_full).max() < 1e-5
        assert np.abs(out[0, h].float().cpu().numpy() - o_full).max() <= 5e-3
        assert np.abs(lse[0, h].cpu().numpy() - l_full).max() <= 1e-3


def test_default_split_choice(fa):
    """A one-head, long-sequence shape leaves the grid mostly empty: the library splits it."""
    q, k, v = _inputs(43, (1, 1, 4096, 128), torch.bfloat16)
    rt = fa._describe_runtime(1, 1, 4096, 128, False)
    assert rt["kv_splits"] > 1 and rt["total_tiles"] == 32
    out, lse = fa.attention(q, k, v, False, 0.09, return_lse=True)
    o64, l64 = attention_fp64(q, k, v, False, 0.09)
    assert (out.float() - o64.to(torch.bfloat16).float()).abs().max().item() <= 2e-2
    assert (lse.double() - l64).abs().max().item() <= 1e-3


def test_small_grids_are_not_split(fa):
    """Config 1 (B1 H8 S512 D64, 32 tiles) and similar small grids stay unsplit: split
    into 2, 4 or 8 runs they measured 11.2 -> 15.1-15.5 us back to back on MI355X (the
    merge launch costs more than the shorter runs save; the other four shapes: 11.1-14.8
    -> 15.2-22.5 us).  The shape's preset (128-key tiles) is the fastest by HIP-graph
    replay."""
    w = next(c for c in W.CONFIGS if c.name == "small-fp16")
    rt = fa._describe_runtime(w.B, w.H, w.S, w.D, w.causal, dtype=w.dtype)
    assert rt["kv_splits"] == 1 and rt["tiling_source"] == "preset"
    assert rt["selected_config"] == {"BLOCK_M": 128, "BLOCK_N": 128}
    for shape in ((1, 8, 512, 128), (1, 4, 1024, 64), (2, 8, 256, 64), (1, 16, 512, 64)):
        assert fa._describe_runtime(*shape, False, dtype=torch.float16)["kv_splits"] == 1, shape
    q, k, v = _inputs(44, (w.B, w.H, w.S, w.D), w.dtype)
    out, lse = fa.attention(q, k, v, w.causal, w.sm_scale, return_lse=True)
    o64, l64 = attention_fp64(q, k, v, w.causal, w.sm_scale)
    assert (out.float() - o64.to(w.dtype).float()).abs().max().item() <= 5e-3
    assert (lse.double() - l64).abs().max().item() <= 1e-3


def _params(fa, q, k, v, out, lse, causal=1, bm=0, bn=0):
    p = fa.FaFwdParams()
    p.q, p.k, p.v, p.o = q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr()
    p.lse = lse.data_ptr() if lse is not None else None
    for arr, t in ((p.q_stride, q), (p.k_stride, k), (p.v_stride, v), (p.o_stride, out)):
        for i, s in enumerate(t.stride()):
            arr[i] = s
    p.B, p.H, p.Sq, p.Sk, p.D = q.shape[0], q.shape[1], q.shape[2], q.shape[2], q.shape[3]
    p.dtype = 1 if q.dtype == torch.bfloat16 else 0
    p.causal, p.sm_scale, p.block_m, p.block_n = causal, 0.1, bm, bn
    return p


def test_c_abi_split_and_errors(fa):
    lib = fa._load_library()
    q, k, v = _inputs(44, (2, 2, 700, 128), torch.bfloat16)
    out = torch.empty_like(q)
    want = fa.attention(q, k, v, True, 0.1)
    p = _params(fa, q, k, v, out, None)
    nbytes = lib.fa_split_workspace_bytes(ctypes.byref(p), 4)
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib.fa_fwd_split(ctypes.byref(p), 4, ctypes.c_void_p(ws.data_ptr()), nbytes, stream) == 0
    torch.cuda.synchronize()
    assert (out.float() - want.float()).abs().max().item() <= 2e-2   # LSE = NULL path
    bad = [
        (4, None, nbytes, -1),                            # no workspace
        (4, ws.data_ptr(), nbytes - 1, -2),               # too small
        (4, ws.data_ptr() + 64, nbytes - 64, -6),         # misaligned
        (0, ws.data_ptr(), nbytes, -9),                   # kv_splits out of range
        (65, ws.data_ptr(), nbytes, -9),
    ]
    for splits, ptr, size, code in bad:
        assert lib.fa_fwd_split(ctypes.byref(p), splits, ctypes.c_void_p(ptr), size, stream) == code
    p8 = _params(fa, q, k, v, out, None, bm=256, bn=64)   # the 8-wave ping-pong kernel does not split
    assert lib.fa_fwd_split(ctypes.byref(p8), 4, ctypes.c_void_p(ws.data_ptr()), nbytes, stream) == -7


def test_split_graph_replays(fa, monkeypatch):
    monkeypatch.setenv("KV_SPLITS", "5")
    q, k, v = _inputs(45, (1, 4, 2000, 64), torch.float16)
    want_o, want_l = fa.attention(q, k, v, True, 0.1, return_lse=True)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fa.attention(q, k, v, True, 0.1, return_lse=True)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out, lse = fa.attention(q, k, v, True, 0.1, return_lse=True)
    for rep in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want_o) and torch.equal(lse, want_l), rep
