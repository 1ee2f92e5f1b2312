"""bench.py's contract pieces that need no GPU: the refusal of more than one
GPU, and the HBM traffic it reads from the committed PMC summaries."""

from __future__ import annotations

import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused():
    run = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, timeout=120)
    assert run.returncode == 2
    assert "one GPU" in run.stderr and run.stdout == ""


def test_pmc_traffic_figures_parse():
    sys.path.insert(0, ROOT)
    import bench

    gemm = bench.pmc_traffic("k_gemm_512x6144x1536_pmc.txt")
    gemv = bench.pmc_traffic("k_gemv_262144x1536_pmc.txt")
    # at least the algorithmic bytes of each launch: the GEMM's 23,150,592
    # (weights, scales, activations, fp32 output) and the lm_head GEMV's
    # weights and scales (262144 x 1536 x (1 + 1/32) bytes)
    assert gemm is not None and gemm >= 23150592
    assert gemv is not None and gemv >= 262144 * 1536 * 33 // 32
    assert bench.pmc_traffic("no_such_profile.txt") is None
