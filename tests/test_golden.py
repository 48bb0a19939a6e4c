"""The committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_fixtures.py from the CPU restatement) are re-derived on the
CPU: a change of the oracle, or of the seeded problem generators the fixtures
were made from, shows up here.  The GPU side is tests/test_gpu_golden.py."""
import sys
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))

import make_fixtures  # noqa: E402

# the restatement is deterministic per problem; the bar leaves room for a
# different host compiler's contraction of a*b+c into one rounding
BAR = 1e-10


@pytest.mark.parametrize("name", sorted(make_fixtures.FIXTURES))
def test_fixture_is_reproduced_by_the_oracle(name):
    stored = np.load(GOLDEN / f"{name}.npz")
    fresh = make_fixtures.FIXTURES[name]()
    assert sorted(stored.files) == sorted(fresh), name
    for k in stored.files:
        a, b = np.asarray(fresh[k], dtype=np.float64), stored[k].astype(np.float64)
        assert a.shape == b.shape, (name, k)
        scale = max(float(np.max(np.abs(b))) if b.size else 0.0, 1e-300)
        err = float(np.max(np.abs(a - b))) / scale if b.size else 0.0
        assert err <= BAR, (name, k, err)


def test_fixtures_are_small_and_finite():
    for p in sorted(GOLDEN.glob("*.npz")):
        assert p.stat().st_size < 200_000, p.name
        z = np.load(p)
        for k in z.files:
            assert np.all(np.isfinite(z[k])), (p.name, k)
