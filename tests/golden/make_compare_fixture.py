"""Writes tests/golden/compare_results/comparison.txt: the reference's own
comparison tool, compare_results_plus.py, run unmodified on two profile
summaries that flash_attn_npu_amd.rocprof wrote on an MI355X (config 2,
B4 H32 S2048 D128 bf16 causal, with BLOCK_M x BLOCK_N = 128 x 64 and 128 x 32;
`python -m flash_attn_npu_amd.rocprof run --out DIR -- python3 bench.py
--config 2 --block-m 128 --block-n N --cpu-seconds 0 --calibrate-copy
--steps 20`, profiler_output paths shortened to <dir>/).

Runs only where the reference tree is mounted (the build container): the tool
is imported from /root/reference/compare_results_plus.py (stdlib only) and its
stdout is the fixture.  tests/test_compare_fixture.py reads the fixture.

    python tests/golden/make_compare_fixture.py
"""

from __future__ import annotations

import contextlib
import importlib.util
import io
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent / "compare_results"
TOOL = Path("/root/reference/compare_results_plus.py")
A, B = "config2_128x64", "config2_128x32"


def main() -> int:
    spec = importlib.util.spec_from_file_location("compare_results_plus", TOOL)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    out = io.StringIO()
    argv = sys.argv
    sys.argv = ["compare_results_plus.py", str(HERE / A), str(HERE / B), "--name-a", "128x64", "--name-b", "128x32"]
    try:
        with contextlib.redirect_stdout(out):
            mod.main()
    finally:
        sys.argv = argv
    # The input paths are the only machine-specific lines.
    text = out.getvalue().replace(str(HERE), "tests/golden/compare_results")
    (HERE / "comparison.txt").write_text(text)
    print(f"wrote {HERE / 'comparison.txt'} ({len(text.splitlines())} lines)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
