"""Device-side float64 attention, used as the full-size reference in GPU tests.

The CPU oracle (oracle/attention_oracle.py) is the primary reference; at the
full sizes of the measured configurations it runs on sampled heads only, and
this float64 restatement of the same formula (evaluate_attention.py:134-143)
covers every head on the GPU.  Float64 keeps it clear of any reduced-precision
GEMM mode; K^T is made contiguous before the batched product.
"""

from __future__ import annotations

import torch


def attention_fp64(q, k, v, causal: bool, sm_scale: float, heads_per_chunk: int = 8):
    """Returns (out float64 [B,H,S,D], lse float64 [B,H,S]) on q's device."""
    B, H, S, D = q.shape
    Sk = k.shape[2]
    qf = q.reshape(B * H, S, D)
    kf = k.reshape(B * H, Sk, D)
    vf = v.reshape(B * H, Sk, D)
    out = torch.empty((B * H, S, D), dtype=torch.float64, device=q.device)
    lse = torch.empty((B * H, S), dtype=torch.float64, device=q.device)
    mask = None
    if causal:
        mask = torch.triu(torch.ones((S, Sk), dtype=torch.bool, device=q.device), diagonal=1)
    for i in range(0, B * H, heads_per_chunk):
        qs = qf[i:i + heads_per_chunk].to(torch.float64)
        kt = kf[i:i + heads_per_chunk].to(torch.float64).transpose(1, 2).contiguous()
        vs = vf[i:i + heads_per_chunk].to(torch.float64).contiguous()
        s = torch.bmm(qs, kt) * sm_scale
        if mask is not None:
            s = s.masked_fill(mask, float("-inf"))
        lse[i:i + heads_per_chunk] = torch.logsumexp(s, dim=-1)
        p = torch.softmax(s, dim=-1)
        out[i:i + heads_per_chunk] = torch.bmm(p, vs)
        del s, p, qs, kt, vs
    return out.reshape(B, H, S, D), lse.reshape(B, H, S)
