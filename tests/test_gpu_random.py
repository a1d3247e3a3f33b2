"""GPU: a seeded random sweep of the operator surface against float64.

Each case draws batch and heads, a length from 1 to 2600, the head dim, the
dtype, the mask, the scale (negative now and then), a memory layout per
tensor (dense [B,H,S,D]; a [B,S,H,D] buffer viewed as [B,H,S,D]; rows with
a wider pitch), the input magnitude, the tiling (the library's choice or an
explicit BLOCK_M/BLOCK_N the library has a kernel for) and the KV split
count (the library's choice or a forced one), and compares O and LSE with
the float64 restatement of evaluate_attention.py:134-143
(tests/gpu_reference.py):

    |O - O64| <= O_TOL + REL * |O64|   (fp16: 5e-3 + 2^-11 |O64|; bf16: 2e-2 + 2^-8 |O64|)
    |LSE - LSE64| <= 1e-3

O_TOL is the gate of the other parity tests; the relative term covers the
final rounding of O to the dtype where |O| exceeds ~2 (large inputs with a
peaked softmax).  Cases are printed before they run.
"""

from __future__ import annotations

import math
import random

import pytest
import torch

from tests.gpu_reference import attention_fp64

pytestmark = pytest.mark.gpu

O_TOL = {torch.float16: 5e-3, torch.bfloat16: 2e-2}
REL = {torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8}
LSE_TOL = 1e-3
N_CASES = 160
CHUNK = 20
SEED = 20261202


def _draw(i, table):
    rng = random.Random(SEED + i)
    d = rng.choice([16, 32, 64, 64, 128, 128, 128, 256])
    dtype = rng.choice([torch.float16, torch.bfloat16])
    causal = rng.random() < 0.5
    r = rng.random()
    s = rng.randint(1, 130) if r < 0.35 else rng.randint(131, 1200) if r < 0.85 else rng.randint(1201, 2600)
    b, h = rng.randint(1, 3), rng.randint(1, 4)
    scale = math.exp(rng.uniform(math.log(0.02), math.log(1.0))) * (-1.0 if rng.random() < 0.1 else 1.0)
    layouts = [rng.choice(["bhsd", "bhsd", "bshd", "pitch"]) for _ in range(3)]
    qk_mag = rng.choice([0.5, 1.0, 2.0])
    tiling = None
    if rng.random() < 0.3:
        name = "float16" if dtype == torch.float16 else "bfloat16"
        rows = [t for t in table if t["HEAD_DIM"] == d and t["dtype"] == name and t["causal"] == causal]
        if rows:
            row = rng.choice(rows)
            tiling = (row["BLOCK_M"], row["BLOCK_N"])
    splits = None
    if rng.random() < 0.3 and not (tiling is not None and tiling[0] == 256):  # the 8-wave kernel does not split
        splits = rng.choice([2, 3, 5])
    return dict(d=d, dtype=dtype, causal=causal, s=s, b=b, h=h, scale=scale, layouts=layouts, qk_mag=qk_mag,
                tiling=tiling, splits=splits, seed=SEED + i)


def _tensor(shape, layout, dtype, mag, g, pad):
    b, h, s, d = shape
    if layout == "bshd":
        base = (torch.randn((b, s, h, d), generator=g) * mag).to(dtype).cuda()
        return base.permute(0, 2, 1, 3)
    if layout == "pitch":
        base = (torch.randn((b, h, s, d + pad), generator=g) * mag).to(dtype).cuda()
        return base[..., :d]
    return (torch.randn((b, h, s, d), generator=g) * mag).to(dtype).cuda()


@pytest.mark.parametrize("chunk", range(N_CASES // CHUNK))
def test_random_cases_vs_fp64(fa, monkeypatch, chunk):
    table = [t for t in fa.kernel_table() if "float8" not in t["dtype"]]
    for i in range(chunk * CHUNK, (chunk + 1) * CHUNK):
        c = _draw(i, table)
        print(f"[random] case {i}: " + ", ".join(f"{k}={v}" for k, v in c.items()), flush=True)
        g = torch.Generator().manual_seed(c["seed"])
        shape = (c["b"], c["h"], c["s"], c["d"])
        pad = 8 * (1 + c["seed"] % 3)
        q = _tensor(shape, c["layouts"][0], c["dtype"], c["qk_mag"], g, pad)
        k = _tensor(shape, c["layouts"][1], c["dtype"], c["qk_mag"], g, pad)
        v = _tensor(shape, c["layouts"][2], c["dtype"], 1.0, g, pad)
        if c["splits"] is None:
            monkeypatch.delenv("KV_SPLITS", raising=False)
        else:
            monkeypatch.setenv("KV_SPLITS", str(c["splits"]))
        bm, bn = c["tiling"] if c["tiling"] is not None else (None, None)
        out, lse = fa.attention(q, k, v, c["causal"], c["scale"], BM=bm, BN=bn, return_lse=True)
        o64, l64 = attention_fp64(q, k, v, c["causal"], c["scale"])
        err = (out.double() - o64).abs()
        bound = O_TOL[c["dtype"]] + REL[c["dtype"]] * o64.abs()
        excess = (err - bound).max().item()
        assert excess <= 0.0 and not torch.isnan(out).any(), (i, err.max().item(), excess)
        d_lse = (lse.double() - l64).abs().max().item()
        assert d_lse <= LSE_TOL, (i, d_lse)
    monkeypatch.delenv("KV_SPLITS", raising=False)


# ---------------------------------------------------------------------------
# fp8-e5m2 V: the same kind of draw (no tiling override: the fp8-V kernels have
# one tiling each), checked per head with the gates of tests/test_gpu_fp8v.py
# (the CPU replay of the kernel's e5m2 rounding, the fp32 formula's e5m2
# bound, LSE); with forced splits only the e5m2 bound and LSE apply, since
# each KV run rounds p against its own running max.

N_FP8 = 48


def _draw_fp8(i):
    rng = random.Random(SEED + 7919 + i)
    d = rng.choice([16, 32, 64, 128, 128, 256])
    return dict(d=d, dtype=rng.choice([torch.float16, torch.bfloat16]), causal=rng.random() < 0.5,
                s=rng.randint(1, 130) if rng.random() < 0.4 else rng.randint(131, 900),
                b=rng.randint(1, 2), h=rng.randint(1, 2),
                scale=d ** -0.5 * rng.choice([0.5, 1.0, 2.0]) * (-1.0 if rng.random() < 0.15 else 1.0),
                layouts=[rng.choice(["bhsd", "bshd", "pitch"]) for _ in range(3)],
                splits=rng.choice([None, None, None, 2, 5]), seed=SEED + 7919 + i)


@pytest.mark.parametrize("chunk", range(N_FP8 // 12))
def test_random_fp8v_cases(fa, monkeypatch, chunk):
    import numpy as np
    from oracle.attention_oracle import attention_ref
    from tests.test_gpu_fp8v import _check_head, _probs

    for i in range(chunk * 12, (chunk + 1) * 12):
        c = _draw_fp8(i)
        print(f"[random-fp8v] case {i}: " + ", ".join(f"{k}={v}" for k, v in c.items()), flush=True)
        g = torch.Generator().manual_seed(c["seed"])
        shape = (c["b"], c["h"], c["s"], c["d"])
        q = _tensor(shape, c["layouts"][0], c["dtype"], 1.0, g, 8)
        k = _tensor(shape, c["layouts"][1], c["dtype"], 1.0, g, 16)
        v = _tensor(shape, c["layouts"][2], torch.float8_e5m2, 1.0, g, 16)  # fp8 rows: 16-element pitch
        if c["splits"] is None:
            monkeypatch.delenv("KV_SPLITS", raising=False)
            # The library's own split choice applies to fp8 V as well (e.g. B1 H2 S560 D256).
            splits = fa._describe_runtime(*shape, c["causal"], dtype=c["dtype"],
                                          v_dtype=torch.float8_e5m2)["kv_splits"]
        else:
            monkeypatch.setenv("KV_SPLITS", str(c["splits"]))
            splits = c["splits"]
        out, lse = fa.attention(q, k, v, c["causal"], c["scale"], return_lse=True)
        assert torch.isfinite(out).all() and torch.isfinite(lse).all(), i
        out, lse = out.float().cpu().numpy(), lse.cpu().numpy()
        for bi in range(c["b"]):
            for hi in range(c["h"]):
                qh, kh, vh = (t[bi, hi].float().cpu().numpy() for t in (q, k, v))
                if splits == 1:
                    _check_head(qh, kh, vh, out[bi, hi], lse[bi, hi], c["causal"], c["scale"], c["dtype"],
                                schedule_check=False)
                else:
                    dt = "float16" if c["dtype"] == torch.float16 else "bfloat16"
                    ref, rl = attention_ref(qh, kh, vh, c["causal"], c["scale"], out_dtype=dt)
                    p = _probs(qh, kh, c["causal"], c["scale"])
                    bound = 2.0 ** -2 * (p @ np.abs(vh).astype(np.float64)) + O_TOL[c["dtype"]]
                    assert np.all(np.abs(out[bi, hi] - ref) <= bound), i
                    assert np.abs(lse[bi, hi] - rl).max() <= LSE_TOL, i
    monkeypatch.delenv("KV_SPLITS", raising=False)
