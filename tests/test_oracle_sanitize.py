"""The CPU oracle under AddressSanitizer and UndefinedBehaviorSanitizer:
`make -C oracle asan` builds oracle/sanitize_main.cpp with oracle.cpp, which
drives every entry point (ADMM with the direct and PCG Schur solves, hard and
soft constraints, S/Phiinv, PCG, the block solve, the adjoint KKT, the
quadrotor RK4 Jacobian) in fp32 and fp64 on small random problems.  The
sanitizers abort on their first finding; the driver also checks return codes
and finiteness."""
import os
import shutil
import subprocess
from pathlib import Path

import pytest

ORACLE = Path(__file__).resolve().parents[1] / "oracle"


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++ with libasan/libubsan")
def test_oracle_runs_clean_under_address_and_ub_sanitizers():
    b = subprocess.run(["make", "-C", str(ORACLE), "asan"], capture_output=True, text=True)
    assert b.returncode == 0, b.stdout + b.stderr
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1",
               OMP_NUM_THREADS="2")
    r = subprocess.run([str(ORACLE / "_asan" / "oracle_sanitize")], capture_output=True, text=True, env=env,
                       timeout=600)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out
    assert "oracle sanitize: ok" in out
    assert "AddressSanitizer" not in out and "runtime error" not in out
