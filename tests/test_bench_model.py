"""bench.py on the CPU: the algorithmic-bytes model behind roofline.achieved
reproduces the per-problem figures it is quoted from (F = factorization, I =
one ADMM iteration: config 3 195.6 / 122.4 KiB, config 4 97.8 / 86.0 KiB, fp32),
and a multi-GPU request exits with a message before touching a device."""
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


@pytest.mark.parametrize("args, F_kib, I_kib", [
    ((41, 17, 13, 13, 4, 20, 4), 195.6, 122.4),          # config 3: box rows only
    ((61, 9, 6, 6, 11, 30, 4, 8), 97.8, 86.0),           # config 4: 8 data-carrying obstacle rows
])
def test_bytes_model_matches_quoted_figures(args, F_kib, I_kib):
    per_qp, F, I = bench.bytes_per_qp(*args)
    assert round(F / 1024, 1) == F_kib
    assert round(I / 1024, 1) == I_kib
    K = args[5]
    assert per_qp == F + K * I


def test_multi_gpu_request_exits_with_message():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_traffic_is_reported_only_for_the_profiled_shape():
    # the committed --pmc summary profiled B = 4096, 20 ADMM iterations: its
    # figure is the one reported, and it lies within a factor of two of the
    # algorithmic bytes of that launch (the kernel streams its records once
    # or twice per iteration, never many times)
    import re

    text = bench.TRAFFIC_FILE.read_text()
    want = float(re.search(r"^traffic_bytes_per_launch = (\d+)", text, re.M).group(1))
    assert bench.measured_traffic(4096, 20) == want
    _, F, I = bench.bytes_per_qp(41, 17, 13, 13, 4, 20, 4)
    algorithmic = 20 * I * 4096
    assert 0.5 * algorithmic < want < 2.0 * algorithmic
    assert bench.measured_traffic(2048, 20) is None
    assert bench.measured_traffic(4096, 10) is None


def test_pcg_flop_model():
    # one block row of S (or Phiinv) has 3 n x n blocks, the end rows 2:
    # (3T - 2) n^2 entries, 2 flop each, for both products; 2 dots + 3 updates
    T, n = 51, 16
    assert bench.flops_pcg_iteration(T, n) == 2 * 2 * (3 * T - 2) * n * n + (2 * 2 + 3 * 2) * T * n
