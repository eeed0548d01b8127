"""The bench.py contract pieces that run without a GPU: the single-GPU refusal and the
analytic FLOP count it divides by."""

import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_bench_refuses_more_than_one_gpu():
    proc = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                          timeout=120, cwd=ROOT)
    assert proc.returncode != 0
    assert "one GPU" in proc.stderr and proc.stdout == ""


def test_srnl_flops_matches_the_reference_formula_by_hand():
    """analysis/operation_count.py:36-44 for one direction, B = 1, 2 x 2 tokens, C = d = 4,
    chunk 2: two chunks of 2 tokens, (6 d^2 + 20 d) MAC per token and 3 d^3 + 2 d^2 per
    chunk boundary, FLOP = 2 MAC."""
    sys.path.insert(0, str(ROOT))
    import bench

    d = 4
    token, boundary = 6 * d * d + 20 * d, 3 * d ** 3 + 2 * d * d
    assert bench.srnl_flops(1, 2, 2, 4, 4, [2]) == 2 * (2 * 2 * token + 2 * boundary)
    # four directions count four times; batch and heads scale linearly
    assert bench.srnl_flops(3, 2, 2, 8, 4, [2] * 4) == 4 * 3 * 2 * bench.srnl_flops(1, 2, 2, 4, 4, [2])
