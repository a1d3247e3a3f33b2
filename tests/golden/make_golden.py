"""Write tests/golden/attention_golden.npz: small seeded attention cases with
their expected outputs.

Inputs are drawn from a CPU torch.Generator in fp32 and rounded to the case's
element type (stored as raw 16-bit patterns, so they are bit-exact); expected
O (rounded to the element type, as float32) and LSE come from the CPU oracle,
and each case was also checked against the float64 brute-force loops before
being written.  The reference repository holds no tensors of its own for this
path (no fixtures, no known-answer tests), so these vectors pin our oracle
against drift and give the GPU kernel committed vectors to match.

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

REPO = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(REPO))

from oracle.attention_oracle import attention_bruteforce, attention_ref  # noqa: E402

OUT = Path(__file__).resolve().parent / "attention_golden.npz"

# (name, H, S, D, dtype, causal, sm_scale)
CASES = [
    ("s37_d64_fp16_full", 2, 37, 64, torch.float16, False, 0.125),
    ("s37_d64_bf16_causal", 2, 37, 64, torch.bfloat16, True, 0.125),
    ("s64_d128_bf16_causal", 1, 64, 128, torch.bfloat16, True, 128 ** -0.5),
    ("s130_d128_fp16_full", 1, 130, 128, torch.float16, False, 128 ** -0.5),
    ("s130_d128_bf16_causal", 1, 130, 128, torch.bfloat16, True, 0.5),
    ("s1_d64_bf16_causal", 1, 1, 64, torch.bfloat16, True, 0.125),
]


def bits16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def main():
    arrays = {}
    for idx, (name, h, s, d, dtype, causal, scale) in enumerate(CASES):
        g = torch.Generator().manual_seed(1000 + idx)
        q, k, v = (torch.randn((1, h, s, d), generator=g).to(dtype) for _ in range(3))
        dt = "bfloat16" if dtype == torch.bfloat16 else "float16"
        qf, kf, vf = (t.float().numpy() for t in (q, k, v))
        o, lse = attention_ref(qf, kf, vf, causal, scale, out_dtype=dt)
        for hh in range(h):
            ob, lb = attention_bruteforce(qf[0, hh], kf[0, hh], vf[0, hh], causal, scale)
            o32, _ = attention_ref(qf[0, hh], kf[0, hh], vf[0, hh], causal, scale)
            assert np.abs(o32 - ob).max() < 1e-5 and np.abs(lse[0, hh] - lb).max() < 1e-5, name
        arrays[f"{name}__q"] = bits16(q)
        arrays[f"{name}__k"] = bits16(k)
        arrays[f"{name}__v"] = bits16(v)
        arrays[f"{name}__o"] = o
        arrays[f"{name}__lse"] = lse
        arrays[f"{name}__meta"] = np.array([h, s, d, 1 if dtype == torch.bfloat16 else 0,
                                            1 if causal else 0], np.int64)
        arrays[f"{name}__scale"] = np.array([scale], np.float64)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(CASES)} cases)")


def load_cases(path: Path = OUT):
    """Yield (name, q, k, v, causal, scale, dtype_name, o, lse) with torch inputs."""
    data = np.load(path, allow_pickle=False)
    names = sorted({key.split("__")[0] for key in data.files})
    for name in names:
        h, s, d, is_bf16, causal = (int(x) for x in data[f"{name}__meta"])
        dtype = torch.bfloat16 if is_bf16 else torch.float16
        qkv = [torch.from_numpy(data[f"{name}__{t}"].view(np.int16).copy()).view(dtype) for t in "qkv"]
        yield (name, *qkv, bool(causal), float(data[f"{name}__scale"][0]),
               "bfloat16" if is_bf16 else "float16", data[f"{name}__o"], data[f"{name}__lse"])


if __name__ == "__main__":
    main()
