"""CPU checks of bench.py's contract pieces that need no GPU: the one-GPU guard and the HBM-traffic figures it reads
from the committed rocprofv3 summaries."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and not r.stdout


def test_traffic_figures_from_profiles():
    K, N = 5120, 17408
    gemv_alg = N * K + K + 2 * N + 4 * N + 4                        # M = 1
    t = bench.traffic_from_profiles("gemv_m1")
    assert t is not None and gemv_alg <= t < 1.05 * gemv_alg        # weights read once
    Mg, Ng = 4096, 12288
    gemm_alg = Mg * K + Ng * K + 2 * Mg * Ng
    t = bench.traffic_from_profiles("gemm_m4096")
    assert t is not None and t >= gemm_alg
    assert bench.traffic_from_profiles("no_such_kernel") is None
