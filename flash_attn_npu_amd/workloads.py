"""Seeded attention workloads: the five measured configurations and the
reference evaluator's shape lists.

Inputs are drawn from a CPU `torch.Generator` in fp32, transformed, cast to the
element type and only then moved to the device, so the GPU kernel and the CPU
oracle see bit-identical tensors.

The reference's own shape lists are restated from evaluate_attention.py:15-43
(18 correctness cases, 6 performance cases, as (Z, H, N_CTX, HEAD_DIM, causal))
with its defaults sm_scale=0.5 (:46), atol=rtol=1e-2 (:47-48) and N(0, 0.5)
inputs seeded with torch.manual_seed(seed) (:90-95).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class Workload:
    name: str
    B: int
    H: int
    S: int
    D: int
    dtype: torch.dtype
    causal: bool
    sm_scale: float
    qk: str          # "normal", "normal_half", "normal_outliers"
    v: str           # "normal", "normal_half", "uniform"
    with_lse: bool
    seed: int

    @property
    def flops(self) -> float:
        f = 4.0 * self.B * self.H * self.S * self.S * self.D
        return f / 2.0 if self.causal else f

    @property
    def io_bytes(self) -> int:
        """Q, K, V read once, O written once, plus the fp32 LSE."""
        elem = 2
        return 4 * self.B * self.H * self.S * self.D * elem + 4 * self.B * self.H * self.S

    @property
    def tolerance(self) -> float:
        """Max-abs tolerance on O: 5e-3 for fp16, 2e-2 for bf16 outputs."""
        return 5e-3 if self.dtype == torch.float16 else 2e-2

    LSE_TOLERANCE = 1e-3

    def describe(self) -> str:
        dt = "fp16" if self.dtype == torch.float16 else "bf16"
        return (f"{self.name}: B{self.B} H{self.H} S{self.S} D{self.D} {dt} "
                f"{'causal' if self.causal else 'non-causal'}")


# The five measured configurations (seed = position 1..5).
CONFIGS = [
    Workload("small-fp16", 1, 8, 512, 64, torch.float16, False, 1 / math.sqrt(64),
             "normal", "normal", False, 1),
    Workload("llama-b4h32s2048d128-causal", 4, 32, 2048, 128, torch.bfloat16, True,
             1 / math.sqrt(128), "normal", "normal", True, 2),
    Workload("long-b2h16s8192d128-causal", 2, 16, 8192, 128, torch.bfloat16, True,
             1 / math.sqrt(128), "normal_half", "normal_half", True, 3),
    Workload("many-heads-b16h16s1024d64", 16, 16, 1024, 64, torch.float16, False,
             1 / math.sqrt(64), "normal", "normal", True, 4),
    Workload("ragged-b8h32s3000d128-causal", 8, 32, 3000, 128, torch.bfloat16, True,
             1 / math.sqrt(128), "normal_outliers", "uniform", True, 5),
]

# The headline workload (bench.py's default).
HEADLINE = CONFIGS[1]

# evaluate_attention.py:15-34
REFERENCE_CORRECTNESS_CASES = [
    (1, 1, 64, 64, False),
    (1, 1, 64, 64, True),
    (1, 1, 128, 128, False),
    (1, 1, 128, 128, True),
    (1, 2, 1024, 64, False),
    (1, 2, 1024, 64, True),
    (4, 32, 64, 64, False),
    (4, 32, 64, 64, True),
    (4, 32, 128, 128, False),
    (4, 32, 256, 128, True),
    (4, 32, 512, 64, True),
    (4, 32, 1024, 64, False),
    (4, 32, 1024, 64, True),
    (4, 32, 1024, 128, False),
    (4, 32, 2048, 64, True),
    (4, 32, 2048, 128, False),
    (4, 32, 4096, 64, False),
    (128, 8, 1024, 64, False),
]

# evaluate_attention.py:36-43
REFERENCE_PERFORMANCE_CASES = [
    (128, 8, 1024, 128, True),
    (128, 8, 1024, 256, True),
    (128, 8, 2048, 128, True),
    (128, 8, 2048, 256, False),
    (128, 8, 4096, 128, False),
    (128, 8, 8192, 64, False),
]
REFERENCE_SM_SCALE = 0.5
REFERENCE_ATOL = 1e-2
REFERENCE_RTOL = 1e-2


def _draw(g: torch.Generator, shape, kind: str) -> torch.Tensor:
    if kind == "normal":
        return torch.randn(shape, generator=g, dtype=torch.float32)
    if kind == "normal_half":
        return torch.randn(shape, generator=g, dtype=torch.float32) * 0.5
    if kind == "normal_outliers":
        x = torch.randn(shape, generator=g, dtype=torch.float32)
        hit = torch.rand(shape, generator=g, dtype=torch.float32) < 0.01
        return torch.where(hit, x * 8.0, x)
    if kind == "uniform":
        return torch.rand(shape, generator=g, dtype=torch.float32) * 2.0 - 1.0
    raise ValueError(kind)


def make_inputs(w: Workload, device=None, batch_slice: slice | None = None):
    """q, k, v for workload `w` (CPU generator seeded with w.seed).

    `batch_slice` keeps only some batch entries after drawing the full tensors
    (so a subset is bit-identical to the same entries of the full draw).
    """
    g = torch.Generator(device="cpu").manual_seed(w.seed)
    shape = (w.B, w.H, w.S, w.D)
    q = _draw(g, shape, w.qk)
    k = _draw(g, shape, w.qk)
    v = _draw(g, shape, w.v)
    out = []
    for t in (q, k, v):
        if batch_slice is not None:
            t = t[batch_slice]
        t = t.to(w.dtype).contiguous()
        out.append(t.to(device) if device is not None else t)
    return tuple(out)


def make_reference_inputs(shape, dtype, seed, device=None):
    """N(0, 0.5) inputs for a reference evaluator case, drawn on the CPU.

    The reference draws on the NPU after torch.manual_seed(seed)
    (evaluate_attention.py:90-95); device RNG streams differ between vendors,
    so bit-identical inputs are not reproducible anyway.  The distribution,
    shape, dtype and seed are the same.
    """
    z, h, n_ctx, head_dim = shape[:4]
    g = torch.Generator(device="cpu").manual_seed(seed)
    ts = []
    for _ in range(3):
        t = (torch.randn((z, h, n_ctx, head_dim), generator=g, dtype=torch.float32) * 0.5).to(dtype)
        ts.append(t.to(device) if device is not None else t)
    return tuple(ts)
