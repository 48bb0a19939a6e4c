"""The C-ABI boundary without a GPU: libtmpc_hip.so loads, exports every entry
point include/tmpc.h declares, the Python mirror binds each of them, and the
host-side parts (workspace queries, status strings, argument validation that
returns before any HIP call) behave as documented."""
import ctypes
import re
from pathlib import Path

import pytest

from turbompc_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "tmpc.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(tmpc_[a-z0-9_]+)\s*\(", text)) - {"tmpc_dims", "tmpc_qp", "tmpc_state"})


@pytest.fixture(scope="module")
def lib():
    try:
        return _lib.load()
    except FileNotFoundError:
        pytest.fail("libtmpc_hip.so is not built (run __graft_entry__.build())")


def test_every_declared_entry_point_is_exported_and_bound(lib):
    names = declared_functions()
    assert len(names) >= 28, names
    missing = [nm for nm in names if not hasattr(lib, nm)]
    assert not missing, missing
    unbound = [nm for nm in names if nm not in _lib.SIGNATURES]
    assert not unbound, unbound
    extra = [nm for nm in _lib.SIGNATURES if nm not in names]
    assert not extra, extra


def test_version_and_status_strings(lib):
    assert lib.tmpc_version() >= 100
    codes = sorted(int(c) for c in re.findall(r"TMPC_[A-Z]+ = (\d+)", HEADER.read_text()))
    assert codes == list(range(len(codes))) and len(codes) >= 7, codes
    for code in codes:
        # the Python mirror names every status the header declares, as the library does
        assert lib.tmpc_status_string(code).decode() == _lib._STATUS[code], code
    assert lib.tmpc_status_string(99) == b"unknown status"


def test_workspace_queries_grow_with_the_batch(lib):
    d1 = _lib.Dims(64, 41, 17, 13, 13, 4)
    d2 = _lib.Dims(128, 41, 17, 13, 13, 4)
    for fn in ("tmpc_admm_direct_workspace_bytes", "tmpc_admm_pcg_workspace_bytes", "tmpc_adjoint_kkt_workspace_bytes"):
        f = getattr(lib, fn)
        a, b = f(4, ctypes.byref(d1)), f(4, ctypes.byref(d2))
        assert 0 < a < b, fn
        assert f(8, ctypes.byref(d1)) > a  # fp64 needs more
        assert a % 256 == 0
    assert 0 < lib.tmpc_blktri_workspace_bytes(4, 64, 41, 17) < lib.tmpc_blktri_workspace_bytes(8, 64, 41, 17)
    assert lib.tmpc_schur_pcg_workspace_bytes(4, 64, 41, 17) > 0


def test_shape_and_argument_errors_return_before_any_launch(lib):
    cfg = _lib.AdmmCfg()
    bad = _lib.Dims(4, 1, 17, 13, 13, 4)  # T < 2
    too_wide = _lib.Dims(4, 10, 65, 13, 13, 4)  # n > 64
    for d in (bad, too_wide):
        st = lib.tmpc_admm_direct_f32(None, ctypes.byref(d), None, None, None, None, ctypes.byref(cfg), None, 0)
        assert st == 1  # TMPC_EBADSHAPE
    ok = _lib.Dims(4, 10, 17, 13, 13, 4)
    st = lib.tmpc_admm_direct_f32(None, ctypes.byref(ok), None, None, None, None, ctypes.byref(cfg), None, 0)
    assert st == 2  # TMPC_EBADARG: null QP / state pointers
    assert lib.tmpc_blktri_factor_f32(None, 4, 1, 17, None, None, 0) == 1
    assert lib.tmpc_blktri_factor_f32(None, 4, 10, 17, None, None, 0) == 2
    # obstacle rows: dim <= nx, row0 + K <= m, n = nx + nu <= 64, then pointers
    obst = lambda nx, nu, dim, K, m, row0: lib.tmpc_obstacle_linearize_f32(  # noqa: E731
        None, 4, 10, nx, nu, dim, K, None, None, None, m, row0, None, None, None)
    assert obst(6, 3, 7, 8, 11, 3) == 1
    assert obst(6, 3, 3, 8, 10, 3) == 1
    assert obst(40, 25, 3, 8, 11, 3) == 1
    assert obst(6, 3, 3, 8, 11, 3) == 2


def test_noalloc_entry_rejects_on_the_host(lib):
    """tmpc_admm_direct_noalloc: checks that return before any HIP call."""
    cfg = _lib.AdmmCfg()
    ok = _lib.Dims(4, 10, 17, 13, 13, 4)
    assert lib.tmpc_admm_direct_noalloc(None, 2, ctypes.byref(ok), None, None, None, None, ctypes.byref(cfg)) == 2
    bad = _lib.Dims(4, 1, 17, 13, 13, 4)
    assert lib.tmpc_admm_direct_noalloc(None, 4, ctypes.byref(bad), None, None, None, None, ctypes.byref(cfg)) == 1
    warm = _lib.AdmmCfg()
    warm.flags = _lib.FLAG_STD_DYNAMICS | _lib.FLAG_WARM_RECORDS
    assert lib.tmpc_admm_direct_noalloc(None, 4, ctypes.byref(ok), None, None, None, None, ctypes.byref(warm)) == 2
    # the smallest batch whose workspace exceeds the scratch array
    B = 1
    while lib.tmpc_admm_direct_workspace_bytes(4, ctypes.byref(_lib.Dims(B, 41, 17, 13, 13, 4))) \
            <= _lib.NOALLOC_SCRATCH_BYTES:
        B *= 2
    big = _lib.Dims(B, 41, 17, 13, 13, 4)
    st = lib.tmpc_admm_direct_noalloc(None, 4, ctypes.byref(big), None, None, None, None, ctypes.byref(cfg))
    assert st == 5  # TMPC_ESCRATCH
    assert b"scratch" in lib.tmpc_status_string(st)


def test_iteration_words_split_into_counts_and_nonfinite_flags():
    import torch

    from turbompc_amd.solvers.admm.admm import _split_iters

    words = torch.tensor([0, 12, 0x7FFFFFFF, -(2 ** 31) + 12, -(2 ** 31)], dtype=torch.int32)  # bit 31 = flag
    counts, bad = _split_iters(words)
    assert counts.tolist() == [0, 12, 0x7FFFFFFF, 12, 0]
    assert bad.tolist() == [False, False, False, True, True]


def test_fill_zero_checks_alignment_before_any_launch(lib):
    assert lib.tmpc_fill_zero(None, None, 0) == 0  # nothing to fill
    assert lib.tmpc_fill_zero(None, None, 16) == 2  # null pointer
    assert lib.tmpc_fill_zero(None, ctypes.c_void_p(0x1002), 16) == 2  # misaligned pointer
    assert lib.tmpc_fill_zero(None, ctypes.c_void_p(0x1000), 6) == 2  # not whole words
