"""tmpc_admm_direct_noalloc (the allocation-free variant of tmpc_admm_direct_*,
whose workspace is the library's per-GPU scratch array) against
tmpc_admm_direct_f32/_f64 with a caller workspace, through the C ABI.

Both run the same kernels with the same launch shapes, so their outputs must
agree bit for bit.  Each case makes two calls in a row, the second on a smaller
batch, so the second call runs on a scratch array that still holds the first
call's contents.  Also checked on the host (no kernel runs): a batch whose
workspace exceeds the scratch is rejected with TMPC_ESCRATCH, warm stage
records with TMPC_EBADARG, an unknown element size with TMPC_EBADARG.
"""
import ctypes

import pytest
import torch

from helpers import random_qp
from turbompc_amd import _lib
from turbompc_amd.problems.quadrotor import make_quadrotor_config
from turbompc_amd.solvers.admm.admm_hip_backend import cfg_struct, qp_struct, state_struct
from turbompc_amd.solvers.qp_data import QPData

pytestmark = pytest.mark.gpu
DEV = "cuda"
ESCRATCH, EBADARG = 5, 2


def _cfg(flags, max_iter=30, adapt=0, check=10):
    return cfg_struct(max_iter=max_iter, check_every=check, adapt_rho_every=adapt, pcg_max_iter=0, use_slack=False,
                      flags=flags, sigma=1e-6, eps_abs=1e-30, eps_rel=1e-30, rho_min=1e-6, rho_max=1e6,
                      adaptive_rho_tolerance=5.0, rho_f_factor=1000.0, alpha=1.6, pcg_eps=0.0)


def _state(qp, rho):
    """The reference initial state (x = 0, z = clip(0, l, u), zero duals) on the device."""
    B, T, n, nx, n0, m = qp.dims
    z = lambda *s: torch.zeros(s, dtype=qp.dtype, device=DEV)  # noqa: E731
    zg = torch.clamp(z(B, T, m), qp.ineq.l.to(DEV), qp.ineq.u.to(DEV)).contiguous()
    return [z(B, T, n), zg, z(B, T, m), z(B, n0), z(B, T - 1, nx), z(B, T, m),
            torch.full((B,), float(rho), dtype=qp.dtype, device=DEV)]


def _slice(qp: QPData, B: int) -> QPData:
    f = lambda t: t[:B].contiguous()  # noqa: E731
    from turbompc_amd.solvers.qp_data import QPCostBlocks, QPEqualityBlocks, QPInequalityBlocks

    return QPData(
        cost=QPCostBlocks(f(qp.cost.D), f(qp.cost.E), f(qp.cost.q)),
        eq=QPEqualityBlocks(f(qp.eq.A0), f(qp.eq.A_minus), f(qp.eq.A_plus), f(qp.eq.c0), f(qp.eq.c)),
        ineq=QPInequalityBlocks(f(qp.ineq.G), f(qp.ineq.l), f(qp.ineq.u), qp.ineq.slack_penalization_weight,
                                qp.ineq.use_slack_variables),
    )


def _run(qp, cfg, noalloc: bool):
    lib = _lib.load()
    B, T, n, nx, n0, m = qp.dims
    dims = _lib.Dims(B, T, n, nx, n0, m)
    cq, keep = qp_struct(qp, None)
    outs = _state(qp, 0.1)
    sv = state_struct(*outs)
    iters = torch.zeros(B, dtype=torch.int32, device=DEV)
    stream = _lib.stream_handle(torch.device(DEV))
    eb = 8 if qp.dtype == torch.float64 else 4
    if noalloc:
        st = lib.tmpc_admm_direct_noalloc(stream, eb, ctypes.byref(dims), ctypes.byref(cq), ctypes.byref(sv),
                                          ctypes.byref(sv), _lib.ptr(iters), ctypes.byref(cfg))
        _lib.check("tmpc_admm_direct_noalloc", st)
    else:
        nbytes = lib.tmpc_admm_direct_workspace_bytes(eb, ctypes.byref(dims))
        ws = _lib.workspace(nbytes, torch.device(DEV))
        sfx = _lib.suffix(qp.dtype)
        st = getattr(lib, f"tmpc_admm_direct_{sfx}")(stream, ctypes.byref(dims), ctypes.byref(cq), ctypes.byref(sv),
                                                    ctypes.byref(sv), _lib.ptr(iters), ctypes.byref(cfg),
                                                    _lib.ptr(ws), nbytes)
        _lib.check(f"tmpc_admm_direct_{sfx}", st)
    torch.cuda.synchronize()
    del keep
    return outs, iters


def _assert_same(qp, cfg):
    ref, it_ref = _run(qp, cfg, noalloc=False)
    got, it_got = _run(qp, cfg, noalloc=True)
    assert torch.equal(it_ref, it_got)
    for a, b in zip(ref, got):
        assert torch.equal(a, b)
    assert all(bool(torch.isfinite(a).all()) for a in got)


def _quad_qp(B, dtype):
    prob = make_quadrotor_config(B=B, seed=3, dtype=dtype, device=DEV)
    return prob.build_qp(*prob.initial_guess())


def _ws_bytes(qp):
    B, T, n, nx, n0, m = qp.dims
    eb = 8 if qp.dtype == torch.float64 else 4
    return _lib.load().tmpc_admm_direct_workspace_bytes(eb, ctypes.byref(_lib.Dims(B, T, n, nx, n0, m)))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_noalloc_streaming_quadrotor_matches_workspace_entry(dtype):
    flags = _lib.FLAG_STD_DYNAMICS | _lib.FLAG_DIAG_COST
    big = _quad_qp(128, dtype)
    assert _ws_bytes(big) <= _lib.NOALLOC_SCRATCH_BYTES
    print(f"noalloc streaming: quadrotor B=128 then B=37, {dtype}", flush=True)
    _assert_same(big, _cfg(flags))
    # second call on a smaller batch, with adaptive rho (refactorization
    # between chunks reads control words the first chunk wrote)
    _assert_same(_slice(big, 37), _cfg(flags, max_iter=60, adapt=25, check=5))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_noalloc_generic_matches_workspace_entry(dtype):
    qp = random_qp(9, 13, 9, 6, 5, seed=11, std=False, dtype=dtype).to(DEV, dtype)
    print(f"noalloc generic: random QP B=9 then B=4, {dtype}", flush=True)
    _assert_same(qp, _cfg(0))
    _assert_same(_slice(qp, 4), _cfg(0, max_iter=17, check=3))


def test_noalloc_rejects_on_host():
    """Argument checks that return before any kernel is launched."""
    lib = _lib.load()
    qp = _quad_qp(2, torch.float32)
    B, T, n, nx, n0, m = qp.dims
    cq, keep = qp_struct(qp, None)
    outs = _state(qp, 0.1)
    sv = state_struct(*outs)
    iters = torch.zeros(B, dtype=torch.int32, device=DEV)
    stream = _lib.stream_handle(torch.device(DEV))
    flags = _lib.FLAG_STD_DYNAMICS | _lib.FLAG_DIAG_COST
    # a batch whose workspace exceeds the scratch: rejected before reading any buffer
    Bbig = 1
    while lib.tmpc_admm_direct_workspace_bytes(4, ctypes.byref(_lib.Dims(Bbig, T, n, nx, n0, m))) \
            <= _lib.NOALLOC_SCRATCH_BYTES:
        Bbig *= 2
    big = _lib.Dims(Bbig, T, n, nx, n0, m)
    st = lib.tmpc_admm_direct_noalloc(stream, 4, ctypes.byref(big), ctypes.byref(cq), ctypes.byref(sv),
                                      ctypes.byref(sv), _lib.ptr(iters), ctypes.byref(_cfg(flags)))
    assert st == ESCRATCH
    assert b"scratch" in lib.tmpc_status_string(st)
    dims = _lib.Dims(B, T, n, nx, n0, m)
    st = lib.tmpc_admm_direct_noalloc(stream, 4, ctypes.byref(dims), ctypes.byref(cq), ctypes.byref(sv),
                                      ctypes.byref(sv), _lib.ptr(iters),
                                      ctypes.byref(_cfg(flags | _lib.FLAG_WARM_RECORDS)))
    assert st == EBADARG
    st = lib.tmpc_admm_direct_noalloc(stream, 2, ctypes.byref(dims), ctypes.byref(cq), ctypes.byref(sv),
                                      ctypes.byref(sv), _lib.ptr(iters), ctypes.byref(_cfg(flags)))
    assert st == EBADARG
    del keep
