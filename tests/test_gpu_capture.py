"""tmpc_admm_direct_* captured in a HIP graph, and called from two host
threads at once.

On the streaming path with the AINV form the call forks a library-owned
stream (the invariant-entry detection runs there beside the factorization)
and joins it back with events; a stream capture records that fork and join
as graph dependencies.  The graph (state reset, iteration-word reset, the
call) is replayed several times, with eager work and synchronisations of the
program between the replays, and every replay must equal the eager call bit
for bit.  The call itself records no memset (the workspace words it reads
are written by its kernels).  Each host thread forks its own side stream, so
calls from two threads on two streams do not order each other's work through
shared events.
"""
import ctypes

import pytest
import torch

from turbompc_amd import _lib
from turbompc_amd.problems.quadrotor import make_quadrotor_config
from turbompc_amd.solvers.admm.admm_hip_backend import cfg_struct, qp_struct, state_struct

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _initial_state(qp, rho):
    B, T, n, nx, n0, m = qp.dims
    z = lambda *s: torch.zeros(s, dtype=qp.dtype, device=DEV)  # noqa: E731
    zg = torch.clamp(z(B, T, m), qp.ineq.l, qp.ineq.u).contiguous()
    return [z(B, T, n), zg, z(B, T, m), z(B, n0), z(B, T - 1, nx), z(B, T, m),
            torch.full((B,), float(rho), dtype=qp.dtype, device=DEV)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_admm_direct_ainv_call_replays_in_a_graph(dtype):
    prob = make_quadrotor_config(B=96, seed=5, dtype=dtype, device=DEV)
    qp = prob.build_qp(*prob.initial_guess())
    B, T, n, nx, n0, m = qp.dims
    flags = _lib.FLAG_STD_DYNAMICS | _lib.FLAG_DIAG_COST | _lib.FLAG_CONST_G | _lib.FLAG_INVARIANT_A
    cfg = cfg_struct(max_iter=20, check_every=10, adapt_rho_every=0, pcg_max_iter=0, use_slack=False, flags=flags,
                     sigma=1e-6, eps_abs=1e-30, eps_rel=1e-30, rho_min=1e-6, rho_max=1e6,
                     adaptive_rho_tolerance=5.0, rho_f_factor=1000.0, alpha=1.6, pcg_eps=0.0)
    lib = _lib.load()
    sfx = _lib.suffix(dtype)
    fn = getattr(lib, f"tmpc_admm_direct_{sfx}")
    dims = _lib.Dims(B, T, n, nx, n0, m)
    eb = 8 if dtype == torch.float64 else 4
    nbytes = lib.tmpc_admm_direct_workspace_bytes(eb, ctypes.byref(dims))
    cq, keep = qp_struct(qp, None)

    def call(outs, iters, ws):
        sv = state_struct(*outs)
        st = fn(_lib.stream_handle(torch.device(DEV)), ctypes.byref(dims), ctypes.byref(cq), ctypes.byref(sv),
                ctypes.byref(sv), _lib.ptr(iters), ctypes.byref(cfg), _lib.ptr(ws), nbytes)
        _lib.check(f"tmpc_admm_direct_{sfx}", st)

    # the eager call (it also creates this thread's side stream)
    print(f"eager call: quadrotor B={B}, {dtype}", flush=True)
    ref = _initial_state(qp, 0.1)
    it_ref = torch.zeros(B, dtype=torch.int32, device=DEV)
    call(ref, it_ref, _lib.workspace(nbytes, torch.device(DEV)))
    torch.cuda.synchronize()
    assert all(bool(torch.isfinite(t).all()) for t in ref)

    src = _initial_state(qp, 0.1)
    outs = [torch.empty_like(t) for t in src]
    iters = torch.zeros(B, dtype=torch.int32, device=DEV)
    ws = _lib.workspace(nbytes, torch.device(DEV))
    torch.cuda.synchronize()
    print("capture", flush=True)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for o, s0 in zip(outs, src):
            o.copy_(s0)
        iters.zero_()
        call(outs, iters, ws)
    torch.cuda.synchronize()
    for k in range(3):
        # eager work of the program between the replays
        for o in outs:
            o.fill_(float("nan"))
        iters.fill_(-1)
        torch.cuda.synchronize()
        print(f"replay {k}", flush=True)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(iters, it_ref), k
        for a, b in zip(outs, ref):
            assert torch.equal(a, b), k
    del keep


def test_admm_direct_ainv_calls_from_two_threads():
    """Two host threads, each with its own stream and workspace, call the
    forking solve at the same time (each thread forks its own side stream):
    every call equals the same call made alone, bit for bit."""
    import threading

    dtype = torch.float32
    probs = [make_quadrotor_config(B=64 + 32 * k, seed=7 + k, dtype=dtype, device=DEV) for k in range(2)]
    qps = [p.build_qp(*p.initial_guess()) for p in probs]
    flags = _lib.FLAG_STD_DYNAMICS | _lib.FLAG_DIAG_COST | _lib.FLAG_CONST_G | _lib.FLAG_INVARIANT_A
    cfg = cfg_struct(max_iter=20, check_every=10, adapt_rho_every=0, pcg_max_iter=0, use_slack=False, flags=flags,
                     sigma=1e-6, eps_abs=1e-30, eps_rel=1e-30, rho_min=1e-6, rho_max=1e6,
                     adaptive_rho_tolerance=5.0, rho_f_factor=1000.0, alpha=1.6, pcg_eps=0.0)
    lib = _lib.load()

    def solve(qp, stream, reps):
        B, T, n, nx, n0, m = qp.dims
        dims = _lib.Dims(B, T, n, nx, n0, m)
        nbytes = lib.tmpc_admm_direct_workspace_bytes(4, ctypes.byref(dims))
        cq, keep = qp_struct(qp, None)
        outs = []
        with torch.cuda.stream(stream):
            ws = _lib.workspace(nbytes, torch.device(DEV))
            for _ in range(reps):
                st = _initial_state(qp, 0.1)
                it = torch.zeros(B, dtype=torch.int32, device=DEV)
                sv = state_struct(*st)
                code = lib.tmpc_admm_direct_f32(_lib.stream_handle(torch.device(DEV)), ctypes.byref(dims),
                                                ctypes.byref(cq), ctypes.byref(sv), ctypes.byref(sv), _lib.ptr(it),
                                                ctypes.byref(cfg), _lib.ptr(ws), nbytes)
                _lib.check("tmpc_admm_direct_f32", code)
                outs.append((st, it))
            stream.synchronize()
        del keep
        return outs

    print("alone", flush=True)
    alone = [solve(qp, torch.cuda.Stream(), 1)[0] for qp in qps]
    print("two threads", flush=True)
    res = [None, None]
    errs = []

    def work(k):
        try:
            res[k] = solve(qps[k], torch.cuda.Stream(), 4)
        except Exception as e:  # reported below
            errs.append(e)

    th = [threading.Thread(target=work, args=(k,)) for k in range(2)]
    for t in th:
        t.start()
    for t in th:
        t.join()
    torch.cuda.synchronize()
    assert not errs, errs
    for k in range(2):
        st_ref, it_ref = alone[k]
        for st, it in res[k]:
            assert torch.equal(it, it_ref), k
            for a, b in zip(st, st_ref):
                assert torch.equal(a, b), k
