"""GPU: the fp8-e5m2 V path (reference flash_attention_forward.py:704, :737,
:996) against the CPU oracle.

With V in float8_e5m2 the kernel, like the reference, rounds the unnormalised
probabilities of each KV tile to e5m2 before P.V (and sums the unrounded ones
into l).  Where that rounding lands depends on the tiling and on when the
running max moves, so the oracle replays the kernel's schedule
(`attention_fp8v`: 64-key tiles, 128 at D = 16; at D = 32, 64 and 128 the
first tile's row max, moved for a wavefront's 32 rows only when a lane's sum
of p over a tile passes 2^14; at D = 16 and 256 the max moved only past a
2^8 margin).  Gates:

* LSE: max|dLSE| <= 1e-3 against both the replay and the fp32 formula (l uses
  unrounded p, so the fp8 cast does not touch it).
* O against the replay: every row within the output tolerance (5e-3 fp16,
  2e-2 bf16), except rows where a logit that differs by an fp32 ulp (MFMA
  summation order, v_exp_f32) rounds to the other e5m2 neighbour.  One such
  flip moves row i by at most 2^-2 p_ij/l_i |v_j|; at most 5% of the rows (or
  2) may exceed the tolerance, each by no more than two flips' worth.
* O against the fp32 formula with the dequantised V: within
  2^-2 sum_j p_ij/l_i |v_j| + tolerance (rounding to either e5m2 neighbour).
* The kernel follows the replayed schedule: its mean distance to it is below
  3/4 of its distance to the reference's always-move schedule
  (lazy_threshold = 0) wherever the two differ.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.attention_oracle import attention_fp8v, attention_ref

pytestmark = pytest.mark.gpu

O_TOL = {torch.float16: 5e-3, torch.bfloat16: 2e-2}
LSE_TOL = 1e-3
DT_ORACLE = {torch.float16: "float16", torch.bfloat16: "bfloat16"}


def _inputs(seed, shape, dtype, v_scale=1.0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(shape, generator=g).to(dtype)
    k = torch.randn(shape, generator=g).to(dtype)
    v = (torch.randn(shape, generator=g) * v_scale).to(torch.float8_e5m2)
    return q, k, v


def _probs(q, k, causal, scale):
    s = (q.astype(np.float64) @ k.astype(np.float64).T) * scale
    if causal:
        s = np.where(np.triu(np.ones(s.shape, dtype=bool), k=1), -np.inf, s)
    e = np.exp(s - s.max(axis=1, keepdims=True))
    return e / e.sum(axis=1, keepdims=True)


def _check_head(qh, kh, vh, og, lg, causal, scale, dtype, schedule_check=True):
    """Gates for one (b, h); returns (max|dO| vs replay, rows over tol, max|dLSE|)."""
    dt = DT_ORACLE[dtype]
    tol = O_TOL[dtype]
    d = qh.shape[-1]
    bn = 128 if d == 16 else 64  # the fp8-V kernels' key tile
    schedule = "sum" if d in (32, 64, 128) else "max"  # the kernels' running-max rule
    r8, rl8 = attention_fp8v(qh, kh, vh, causal, scale, out_dtype=dt, block_n=bn, schedule=schedule)
    ref, rl = attention_ref(qh, kh, vh, causal, scale, out_dtype=dt)
    p = _probs(qh, kh, causal, scale)
    av = np.abs(vh).astype(np.float64)
    flip = 2.0 ** -2 * (p * av.max(axis=1)[None, :]).max(axis=1)  # one flip, worst key of the row
    d8 = np.abs(og - r8)
    over = d8.max(axis=1) > tol
    assert over.sum() <= max(2, int(0.05 * len(over))), f"{over.sum()} rows off the replay"
    assert np.all(d8 <= tol + 2.0 * flip[:, None] + 1e-6)
    bound = 2.0 ** -2 * (p @ av) + tol
    assert np.all(np.abs(og - ref) <= bound)
    dl = max(float(np.abs(lg - rl8).max()), float(np.abs(lg - rl).max()))
    assert dl <= LSE_TOL
    if schedule_check:
        r0, _ = attention_fp8v(qh, kh, vh, causal, scale, out_dtype=dt, block_n=bn, lazy_threshold=0.0)
        gap = np.abs(r0 - r8).mean()
        if gap > 1e-4:
            # Both distances share the output-rounding floor (~1e-3 for bf16
            # at 2048 keys), which dilutes the ratio: ask for a clear margin.
            assert np.abs(og - r8).mean() < 0.75 * np.abs(og - r0).mean()
    return float(d8.max()), int(over.sum()), dl


def _run(fa, q, k, v, causal, scale, **kw):
    out, lse = fa.attention(q.cuda(), k.cuda(), v.cuda(), causal, scale, return_lse=True, **kw)
    torch.cuda.synchronize()
    assert out.dtype == q.dtype and out.shape == q.shape and lse.shape == q.shape[:3]
    assert torch.isfinite(out).all() and torch.isfinite(lse).all()
    return out.float().cpu().numpy(), lse.cpu().numpy()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
@pytest.mark.parametrize("s", [1, 64, 130, 257])
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("d", [16, 32, 64, 128, 256])
def test_fp8v_matches_replay(fa, d, causal, s, dtype):
    print(f"[fp8v] D={d} causal={causal} S={s} {dtype}", flush=True)
    q, k, v = _inputs(100 + d + s + causal, (1, 2, s, d), dtype)
    scale = d ** -0.5
    out, lse = _run(fa, q, k, v, causal, scale)
    for h in range(2):
        _check_head(q[0, h].float().numpy(), k[0, h].float().numpy(), v[0, h].float().numpy(),
                    out[0, h], lse[0, h], causal, scale, dtype)


def test_fp8v_headline_heads(fa):
    # The headline per-head shape (S 2048, D 128, causal, bf16) on four heads.
    print("[fp8v] B1 H4 S2048 D128 causal bf16", flush=True)
    q, k, v = _inputs(7, (1, 4, 2048, 128), torch.bfloat16)
    out, lse = _run(fa, q, k, v, True, 128 ** -0.5)
    for h in range(4):
        _check_head(q[0, h].float().numpy(), k[0, h].float().numpy(), v[0, h].float().numpy(),
                    out[0, h], lse[0, h], True, 128 ** -0.5, torch.bfloat16, schedule_check=(h == 0))


def test_fp8v_strided_negative_scale_ragged(fa):
    # v as a [B, S, H, D] tensor viewed [B, H, S, D] (row stride H*D), a
    # negative scale (Q negated in registers) and a ragged key tail.
    print("[fp8v] strided v, scale -0.11, S 333", flush=True)
    q, k, _ = _inputs(8, (1, 2, 333, 64), torch.float16)
    g = torch.Generator().manual_seed(9)
    v_bshd = torch.randn((1, 333, 2, 64), generator=g).to(torch.float8_e5m2)
    v = v_bshd.permute(0, 2, 1, 3)
    assert not v.is_contiguous()
    out, lse = _run(fa, q, k, v, False, -0.11)
    for h in range(2):
        _check_head(q[0, h].float().numpy(), k[0, h].float().numpy(), v[0, h].float().numpy(),
                    out[0, h], lse[0, h], False, -0.11, torch.float16)


@pytest.mark.parametrize("splits", [3, 8])
def test_fp8v_split_kv(fa, monkeypatch, splits):
    # Each KV run rounds p against its own running max, so the split result is
    # checked against the fp32 formula's e5m2 bound, not the unsplit replay.
    print(f"[fp8v] split-KV {splits}", flush=True)
    q, k, v = _inputs(10 + splits, (1, 2, 3000, 128), torch.bfloat16)
    monkeypatch.setenv("KV_SPLITS", str(splits))
    out, lse = _run(fa, q, k, v, True, 128 ** -0.5)
    for h in range(2):
        qh, kh, vh = q[0, h].float().numpy(), k[0, h].float().numpy(), v[0, h].float().numpy()
        ref, rl = attention_ref(qh, kh, vh, True, 128 ** -0.5, out_dtype="bfloat16")
        p = _probs(qh, kh, True, 128 ** -0.5)
        bound = 2.0 ** -2 * (p @ np.abs(vh).astype(np.float64)) + O_TOL[torch.bfloat16]
        assert np.all(np.abs(out[0, h] - ref) <= bound)
        assert np.abs(lse[0, h] - rl).max() <= LSE_TOL


def test_fp8v_tiling_override_rejected(fa):
    q, k, v = _inputs(11, (1, 1, 128, 128), torch.bfloat16)
    with pytest.raises(ValueError, match="BLOCK_M/BLOCK_N"):
        fa.attention(q.cuda(), k.cuda(), v.cuda(), False, 0.1, BM=128, BN=32)
