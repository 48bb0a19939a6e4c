"""Pins of the CPU oracle's Schur assembly and Schur solvers (no GPU).

S      closed form S = P + sigma I + rho_f C^T C + rho G^T G on dense matrices
       (reference test tests/python/solvers/test_admm_residuals.py:679-735, with
       the G^T G term of turbompc/solvers/admm/admm.py:93).
Phiinv block-diagonal S gives Phiinv = -S^{-1} exactly; with off-diagonal
       blocks scaled by eps the error to -S^{-1} is O(eps^2) (first-order
       Neumann expansion), which a wrong index/sign/transpose breaks.
solve  numpy.linalg.solve on the dense S (test_linear_solve.py:34-45).
PCG    converges to the dense solve; exact preconditioner -> one iteration;
       the |eta_0| <= 1e-12 early exit returns the guess with 0 iterations.
"""
import numpy as np
import pytest

import oracle
from helpers import blocks_to_dense, dense_C, dense_G, dense_P, np_qp, random_qp


@pytest.mark.parametrize("std", [True, False])
def test_schur_build_matches_dense_closed_form(std):
    qp = random_qp(3, 6, 5, 3, 4, seed=1, std=std)
    rho, sigma, fac = 0.3, 1e-3, 10.0
    S, P = oracle.schur_build(qp, rho, sigma, fac)
    a = np_qp(qp)
    for b in range(3):
        C = dense_C(a["A0"][b], a["Am"][b], a["Ap"][b])
        Gd = dense_G(a["G"][b])
        Sd = dense_P(a["D"][b], a["E"][b]) + sigma * np.eye(C.shape[1]) + rho * fac * C.T @ C + rho * Gd.T @ Gd
        np.testing.assert_allclose(blocks_to_dense(S[b]), Sd, rtol=1e-12, atol=1e-12)
        # the first/last block rows carry zero padding
        assert np.all(S[b, 0, :, :5] == 0) and np.all(S[b, -1, :, 10:] == 0)


def test_phiinv_is_first_order_inverse():
    qp = random_qp(1, 5, 4, 2, 3, seed=2, std=False)
    S, P = oracle.schur_build(qp, 0.2, 1e-4, 5.0)
    Sd = blocks_to_dense(S[0])
    n, T = 4, 5
    errs = []
    for eps in (1e-2, 1e-3):
        Se = S[0].copy()
        Se[:, :, :n] *= eps
        Se[:, :, 2 * n:] *= eps
        # rebuild Phiinv for the scaled matrix with the oracle's formula through
        # a QP whose coupling vanishes: use blocks directly
        th = [Se[t, :, n:2 * n] for t in range(T)]
        thinv = [np.linalg.inv(x) for x in th]
        Pd = np.zeros((T * n, T * n))
        for t in range(T):
            Pd[t * n:(t + 1) * n, t * n:(t + 1) * n] = -thinv[t]
        # oracle Phiinv for the unscaled S has the same diagonal -theta^{-1}
        np.testing.assert_allclose(blocks_to_dense(P[0])[:n, :n], -np.linalg.inv(Sd[:n, :n]), rtol=1e-10)
        # full first-order formula on the scaled system
        Sed = blocks_to_dense(Se)
        Od = Sed - np.kron(np.eye(T), np.ones((n, n))) * Sed
        Th = np.zeros_like(Sed)
        for t in range(T):
            Th[t * n:(t + 1) * n, t * n:(t + 1) * n] = thinv[t]
        approx = -(Th - Th @ Od @ Th)
        errs.append(np.max(np.abs(approx + np.linalg.inv(Sed))))
    assert errs[1] < errs[0] * 0.05  # O(eps^2) decay

    # the oracle's off-diagonal blocks equal theta_t^-1 phi theta^-1 (sign +)
    Pd = blocks_to_dense(P[0])
    Od = Sd - np.kron(np.eye(T), np.ones((n, n))) * Sd
    Th = np.zeros_like(Sd)
    for t in range(T):
        Th[t * n:(t + 1) * n, t * n:(t + 1) * n] = np.linalg.inv(Sd[t * n:(t + 1) * n, t * n:(t + 1) * n])
    np.testing.assert_allclose(Pd, -(Th - Th @ Od @ Th), rtol=1e-9, atol=1e-12)


@pytest.mark.parametrize("dtype,tol", [(np.float64, 1e-10), (np.float32, 2e-3)])
def test_blktri_solve_matches_dense(dtype, tol):
    qp = random_qp(4, 7, 6, 4, 3, seed=3, std=False)
    S, _ = oracle.schur_build(qp, 0.5, 1e-6, 20.0)
    rhs = np.random.default_rng(0).standard_normal((4, 7, 6))
    x = oracle.blktri_solve(S.astype(dtype), rhs.astype(dtype))
    for b in range(4):
        xd = np.linalg.solve(blocks_to_dense(S[b]), rhs[b].reshape(-1)).reshape(7, 6)
        assert np.max(np.abs(x[b] - xd)) <= tol * np.max(np.abs(xd))


def test_pcg_converges_to_dense_solution():
    qp = random_qp(3, 8, 5, 3, 2, seed=4, std=False)
    S, P = oracle.schur_build(qp, 0.1, 1e-6, 10.0)
    rng = np.random.default_rng(1)
    # scaled so the absolute stopping term 1e-12 on eta (pcg_primal.py:113)
    # sits far below the relative one
    rhs = rng.standard_normal((3, 8, 5)) * 1e4
    x, it = oracle.pcg(S, P, rhs, np.zeros_like(rhs), eps=1e-24, max_iter=500)
    for b in range(3):
        xd = np.linalg.solve(blocks_to_dense(S[b]), rhs[b].reshape(-1)).reshape(8, 5)
        np.testing.assert_allclose(x[b], xd, rtol=1e-8, atol=1e-10)
        assert 1 <= it[b] <= 500


def test_pcg_exact_preconditioner_one_iteration_and_early_exit():
    rng = np.random.default_rng(5)
    T, n = 4, 3
    S = np.zeros((1, T, n, 3 * n))
    P = np.zeros_like(S)
    for t in range(T):
        L = rng.standard_normal((n, n))
        th = L @ L.T + n * np.eye(n)
        S[0, t, :, n:2 * n] = th
        P[0, t, :, n:2 * n] = -np.linalg.inv(th)
    rhs = rng.standard_normal((1, T, n))
    x, it = oracle.pcg(S, P, rhs, np.zeros_like(rhs), eps=1e-10, max_iter=50)
    assert it[0] == 1
    for t in range(T):
        np.testing.assert_allclose(x[0, t], np.linalg.solve(S[0, t, :, n:2 * n], rhs[0, t]), rtol=1e-10)
    # zero residual: no iteration, guess returned
    x0 = x.copy()
    x2, it2 = oracle.pcg(S, P, np.zeros_like(rhs), np.zeros_like(rhs), eps=1e-10, max_iter=50)
    assert it2[0] == 0 and np.all(x2 == 0)
    del x0


def test_pcg_max_iter_bounds_iterations():
    qp = random_qp(2, 10, 6, 4, 2, seed=6, std=False)
    S, P = oracle.schur_build(qp, 0.1, 1e-6, 1000.0)
    rhs = np.random.default_rng(2).standard_normal((2, 10, 6))
    _, it = oracle.pcg(S, P, rhs, np.zeros_like(rhs), eps=1e-30, max_iter=3)
    assert np.all(it == 3)
