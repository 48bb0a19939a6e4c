"""GPU parity of the Schur-level kernels against the CPU oracle (via the C ABI).

Tolerances: normwise relative error (helpers.rel_err) 1e-9 in fp64 and 1e-4 in
fp32 unless a test says otherwise.
"""
import numpy as np
import pytest
import torch

import oracle
from helpers import TOL, blocks_to_dense, random_qp, rel_err
from turbompc_amd.solvers.admm.admm import compute_S_Phiinv
from turbompc_amd.solvers.linear_systems_solvers.hip_backend import BlockTriFactor, hip_blktri_solve, hip_pcg_solve

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("std,shape", [(True, (5, 21, 6, 4, 2)), (False, (7, 11, 17, 13, 4)), (False, (3, 9, 5, 3, 7))])
def test_schur_build_matches_oracle(dtype, std, shape):
    B, T, n, nx, m = shape
    qp = random_qp(B, T, n, nx, m, seed=31, std=std)
    S0, P0 = oracle.schur_build(qp, 0.2, 1e-6, 100.0)
    sp = compute_S_Phiinv(qp.to(DEV, dtype), 0.2 * 100.0, 1e-6, rho_ineq=0.2)
    assert rel_err(sp.S, S0) < TOL[dtype]
    assert rel_err(sp.preconditioner_Phiinv, P0) < (TOL[dtype] if dtype == torch.float64 else 1e-3)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("shape", [(4, 21, 6, 4, 2), (10, 41, 17, 13, 4), (5, 13, 9, 6, 3), (3, 6, 5, 3, 2), (1, 2, 1, 1, 0)])
def test_blktri_solve_matches_dense(dtype, shape):
    B, T, n, nx, m = shape
    qp = random_qp(B, T, n, nx, m, seed=32, std=False)
    S, _ = oracle.schur_build(qp, 1.0, 1e-3, 2.0)
    rhs = np.random.default_rng(1).standard_normal((B, T, n))
    x = hip_blktri_solve(torch.tensor(S, dtype=dtype, device=DEV), torch.tensor(rhs, dtype=dtype, device=DEV))
    xd = np.stack([np.linalg.solve(blocks_to_dense(S[b]), rhs[b].reshape(-1)).reshape(T, n) for b in range(B)])
    err = rel_err(x, xd)
    assert err < TOL[dtype], err


def test_blktri_factor_reuse_two_rhs():
    qp = random_qp(6, 15, 9, 6, 3, seed=33, std=True)
    S, _ = oracle.schur_build(qp, 0.1, 1e-6, 1000.0)
    St = torch.tensor(S, device=DEV)
    F = BlockTriFactor(St)
    rng = np.random.default_rng(2)
    for _ in range(2):
        rhs = rng.standard_normal((6, 15, 9))
        x = F.solve(torch.tensor(rhs, device=DEV))
        assert rel_err(x, oracle.blktri_solve(S, rhs)) < 1e-9


@pytest.mark.parametrize("shape", [(4, 51, 16, 12, 16), (6, 21, 6, 4, 2), (5, 9, 5, 3, 2)])
def test_schur_pcg_matches_oracle(shape):
    B, T, n, nx, m = shape
    qp = random_qp(B, T, n, nx, m, seed=34, std=True)
    S, P = oracle.schur_build(qp, 0.1, 1e-6, 1000.0)
    rng = np.random.default_rng(3)
    rhs = rng.standard_normal((B, T, n)) * 10
    x0 = rng.standard_normal((B, T, n)) * 0.1
    xo, ito = oracle.pcg(S, P, rhs, x0, eps=1e-8, max_iter=40)
    t = lambda a: torch.tensor(a, device=DEV)  # noqa: E731
    x, it = hip_pcg_solve(t(S), t(P), t(rhs), t(x0), eps=1e-8, max_iters=40)
    # stopped by tolerance: counts may differ by one between summation orders,
    # iterates agree to the stopping tolerance
    assert np.all(np.abs(it.cpu().numpy() - ito) <= 1)
    assert rel_err(x, xo) < 1e-6
    # fixed iteration count (eps = 0): parity at 1e-9
    xo, ito = oracle.pcg(S, P, rhs, x0, eps=0.0, max_iter=5)
    x, it = hip_pcg_solve(t(S), t(P), t(rhs), t(x0), eps=0.0, max_iters=5)
    np.testing.assert_array_equal(it.cpu().numpy(), ito)
    assert rel_err(x, xo) < 1e-9


@pytest.mark.parametrize("shape", [(4, 51, 16, 12, 16), (6, 21, 6, 4, 2)])
def test_schur_pcg_fp32_matches_fp64_oracle(shape):
    """tmpc_schur_pcg_f32 on fp32 copies of the system, tolerance-stopped and
    at a fixed count, against the fp64 oracle at the fp32 bar."""
    B, T, n, nx, m = shape
    qp = random_qp(B, T, n, nx, m, seed=34, std=True)
    S, P = oracle.schur_build(qp, 0.1, 1e-6, 1000.0)
    rng = np.random.default_rng(3)
    rhs = rng.standard_normal((B, T, n)) * 10
    x0 = rng.standard_normal((B, T, n)) * 0.1
    t = lambda a: torch.tensor(a, device=DEV, dtype=torch.float32)  # noqa: E731
    xo, ito = oracle.pcg(S, P, rhs, x0, eps=0.0, max_iter=5)
    x, it = hip_pcg_solve(t(S), t(P), t(rhs), t(x0), eps=0.0, max_iters=5)
    np.testing.assert_array_equal(it.cpu().numpy(), ito)
    e = rel_err(x, xo)
    print(f"schur PCG fp32 fixed count {shape}: rel err vs fp64 oracle {e:.2e}")
    assert e < TOL[torch.float32], e
    xo, ito = oracle.pcg(S, P, rhs, x0, eps=1e-8, max_iter=40)
    x, it = hip_pcg_solve(t(S), t(P), t(rhs), t(x0), eps=1e-8, max_iters=40)
    assert np.all(np.abs(it.cpu().numpy() - ito) <= 1)
    e = rel_err(x, xo)
    print(f"schur PCG fp32 tolerance-stopped {shape}: rel err vs fp64 oracle {e:.2e}")
    assert e < TOL[torch.float32], e


def test_schur_pcg_edge_cases():
    # zero rhs and zero guess: no iteration (|eta_0| <= 1e-12), x = x0
    qp = random_qp(3, 7, 6, 4, 2, seed=35, std=True)
    S, P = oracle.schur_build(qp, 0.1, 1e-6, 10.0)
    t = lambda a: torch.tensor(a, device=DEV)  # noqa: E731
    z = np.zeros((3, 7, 6))
    x, it = hip_pcg_solve(t(S), t(P), t(z), t(z), eps=1e-8, max_iters=10)
    assert torch.all(it == 0) and torch.all(x == 0)
    # max_iter = 0 still runs one iteration (cond_fun forces it < 1)
    rhs = np.random.default_rng(4).standard_normal((3, 7, 6))
    xo, ito = oracle.pcg(S, P, rhs, z, eps=1e-8, max_iter=0)
    x, it = hip_pcg_solve(t(S), t(P), t(rhs), t(z), eps=1e-8, max_iters=0)
    assert np.all(ito == 1) and torch.all(it == 1)
    assert rel_err(x, xo) < 1e-9
