"""GPU: long sequences (S = 16384 and 32768) on sampled query rows against float64.

A full float64 reference needs S x S scores per head (8.6 GB at S = 32768), so
these cases check 192 query rows per head, drawn with a fixed seed (plus the
first and the last row), against the float64 formula of
evaluate_attention.py:134-143 evaluated for those rows only: O within 5e-3
(fp16) / 2e-2 (bf16), LSE within 1e-3.  Long units (256 and 512 KV tiles of
one m-tile), the causal diagonal at the far end of the sequence and, with few
heads, the library's split choice are what these shapes add to the other
parity tests.
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

O_TOL = {torch.float16: 5e-3, torch.bfloat16: 2e-2}
LSE_TOL = 1e-3


def _rows_fp64(q, k, v, rows, causal, scale):
    """O and LSE (float64) of query rows `rows` of one head."""
    qs = q[rows].double()
    s = (qs @ k.double().T) * scale
    if causal:
        keys = torch.arange(k.shape[0], device=q.device)
        s = s.masked_fill(keys[None, :] > rows[:, None], float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    return torch.softmax(s, dim=-1) @ v.double(), lse


@pytest.mark.parametrize("shape,causal,dtype", [
    ((1, 2, 32768, 128), True, torch.bfloat16),
    ((1, 2, 16384, 64), False, torch.float16),
    ((1, 1, 32768, 256), True, torch.bfloat16),
    ((1, 1, 16384, 128), False, torch.bfloat16),   # 128 tiles: the library splits into 2 runs
    ((1, 1, 16384, 64), True, torch.float16),      # causal, 128 tiles: 4 runs
], ids=["S32768-D128-causal-bf16", "S16384-D64-fp16", "S32768-D256-causal-bf16", "S16384-D128-split2-bf16",
        "S16384-D64-causal-split4-fp16"])
def test_long_sequence_sampled_rows(fa, shape, causal, dtype):
    b, h, s, d = shape
    scale = d ** -0.5
    splits = fa._describe_runtime(b, h, s, d, causal, dtype=dtype)["kv_splits"]
    print(f"[long] {shape} causal={causal} {dtype} kv_splits={splits}", flush=True)
    assert splits == {(1, 1, 16384, 128): 2, (1, 1, 16384, 64): 4}.get(shape, 1)
    g = torch.Generator().manual_seed(s + d)
    q, k, v = ((torch.randn(shape, generator=g) * 0.8).to(dtype).cuda() for _ in range(3))
    out, lse = fa.attention(q, k, v, causal, scale, return_lse=True)
    torch.cuda.synchronize()
    rows = torch.unique(torch.cat([torch.tensor([0, s - 1]), torch.randint(0, s, (190,), generator=g)])).cuda()
    for hi in range(h):
        o64, l64 = _rows_fp64(q[0, hi], k[0, hi], v[0, hi], rows, causal, scale)
        d_o = (out[0, hi, rows].double() - o64).abs().max().item()
        d_l = (lse[0, hi, rows].double() - l64).abs().max().item()
        assert d_o <= O_TOL[dtype] and d_l <= LSE_TOL, (hi, d_o, d_l)
