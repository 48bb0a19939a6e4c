"""tmpc_admm_direct_* captured in a HIP graph.

On the streaming path with the AINV form the call forks a library-owned
stream (the invariant-entry detection runs there beside the factorization)
and joins it back with events; a stream capture records that fork and join
as graph dependencies.  The graph (state reset, iteration-word reset, the
call) is replayed several times, with eager work and synchronisations of the
program between the replays, and every replay must equal the eager call bit
for bit.  The call itself records no memset (the workspace words it reads
are written by its kernels).
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
