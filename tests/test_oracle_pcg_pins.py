"""Pins of the oracle's PCG recurrences (pcg_primal.py:70-175) that do not
restate them.

Finite termination: in exact arithmetic, preconditioned CG on S x = b stops
after as many iterations as M^{-1} S has distinct eigenvalues (for a right-hand
side with a component in each eigenspace).  S = L (s0 I + U U^T) L^T with L
block diagonal and the r columns of U each supported on two adjacent stages is
block tridiagonal; with M^{-1} = (L L^T)^{-1} (block diagonal, the oracle's
Phiinv = -M^{-1}), M^{-1} S is similar to s0 I + U U^T, which has r + 1
distinct eigenvalues.  A wrong beta or eta update loses conjugacy and with it
this count.

Galerkin property: the j-th iterate from x0 is the unique x in
x0 + K_j(M^{-1} S, M^{-1} r0) whose residual b - S x is orthogonal to that
Krylov space.  It is computed here from an explicit Krylov basis and a small
dense solve, independently of the recurrences, and the oracle's fixed-count
iterates (max_iter = j) must equal it.
"""
import numpy as np
import pytest

import oracle
from helpers import blocks_to_dense, random_qp


def _dense_blockdiag(blocks):
    T, n, _ = blocks.shape
    out = np.zeros((T * n, T * n))
    for t in range(T):
        out[t * n:(t + 1) * n, t * n:(t + 1) * n] = blocks[t]
    return out


def _to_blocks(A, T, n):
    """Dense block-tridiagonal (T n, T n) -> (T, n, 3n) rows [prev | diag | next]."""
    S = np.zeros((T, n, 3 * n))
    for t in range(T):
        S[t, :, n:2 * n] = A[t * n:(t + 1) * n, t * n:(t + 1) * n]
        if t > 0:
            S[t, :, :n] = A[t * n:(t + 1) * n, (t - 1) * n:t * n]
        if t < T - 1:
            S[t, :, 2 * n:] = A[t * n:(t + 1) * n, (t + 1) * n:(t + 2) * n]
    return S


def _few_eigenvalue_system(rng, T, n, r, s0=1.0):
    L = rng.standard_normal((T, n, n)) * 0.3 + np.eye(n) * rng.uniform(1.0, 2.0, size=(T, 1, 1))
    U = np.zeros((T * n, r))
    for j in range(r):
        t = j % (T - 1)  # columns on the stage pairs (t, t+1)
        U[t * n:(t + 2) * n, j] = rng.standard_normal(2 * n)
    Ld = _dense_blockdiag(L)
    A = Ld @ (s0 * np.eye(T * n) + U @ U.T) @ Ld.T
    Minv = np.stack([np.linalg.inv(L[t] @ L[t].T) for t in range(T)])
    Phi = np.zeros((T, n, 3 * n))
    Phi[:, :, n:2 * n] = -Minv
    return A, Phi


@pytest.mark.parametrize("r", [1, 3, 6])
def test_pcg_stops_after_as_many_iterations_as_distinct_eigenvalues(r):
    rng = np.random.default_rng(10 + r)
    T, n, B = 5, 4, 3
    S = np.zeros((B, T, n, 3 * n))
    P = np.zeros_like(S)
    dense = []
    for b in range(B):
        A, Phi = _few_eigenvalue_system(rng, T, n, r)
        S[b], P[b] = _to_blocks(A, T, n), Phi
        dense.append(A)
        # the construction: M^{-1} S has r + 1 distinct eigenvalues
        Minv = _dense_blockdiag(-Phi[:, :, n:2 * n])
        lam = np.sort(np.linalg.eigvals(Minv @ A).real)
        assert len(np.unique(np.round(lam, 8))) == r + 1
    rhs = rng.standard_normal((B, T, n))
    x, it = oracle.pcg(S, P, rhs, np.zeros_like(rhs), eps=1e-20, max_iter=100)
    assert np.all(it == r + 1), it
    for b in range(B):
        xd = np.linalg.solve(dense[b], rhs[b].reshape(-1)).reshape(T, n)
        np.testing.assert_allclose(x[b], xd, rtol=1e-9, atol=1e-11)
    # one iteration fewer leaves a residual far from zero
    x2, it2 = oracle.pcg(S, P, rhs, np.zeros_like(rhs), eps=1e-20, max_iter=r)
    assert np.all(it2 == r)
    for b in range(B):
        res = rhs[b].reshape(-1) - dense[b] @ x2[b].reshape(-1)
        assert np.max(np.abs(res)) > 1e-6 * np.max(np.abs(rhs[b]))


def _galerkin_iterate(A, Minv, b, x0, j):
    r0 = b - A @ x0
    K = Minv @ A
    v = Minv @ r0
    basis = []
    for _ in range(j):
        basis.append(v)
        v = K @ v
    Q, _ = np.linalg.qr(np.stack(basis, axis=1))
    y = np.linalg.solve(Q.T @ A @ Q, Q.T @ r0)
    return x0 + Q @ y


@pytest.mark.parametrize("dtype,tol", [(np.float64, 1e-9)])
def test_pcg_fixed_count_iterates_are_galerkin_projections(dtype, tol):
    """Warm-started PCG with the oracle's own block preconditioner of a random
    Schur system: every fixed-count iterate is the Galerkin solution on its
    Krylov space."""
    qp = random_qp(2, 6, 4, 2, 3, seed=21, std=False)
    S, P = oracle.schur_build(qp, 0.3, 1e-3, 5.0)
    rng = np.random.default_rng(3)
    B, T, n = 2, 6, 4
    rhs = rng.standard_normal((B, T, n))
    x0 = rng.standard_normal((B, T, n)) * 0.1
    for b in range(B):
        A = blocks_to_dense(S[b])
        Minv = -blocks_to_dense(P[b])
        # the block preconditioner is SPD here (weak coupling)
        assert np.min(np.linalg.eigvalsh(0.5 * (Minv + Minv.T))) > 0
    for j in range(1, 6):
        x, it = oracle.pcg(S.astype(dtype), P.astype(dtype), rhs.astype(dtype), x0.astype(dtype), eps=1e-30,
                           max_iter=j)
        assert np.all(it == j)
        for b in range(B):
            A = blocks_to_dense(S[b])
            Minv = -blocks_to_dense(P[b])
            xg = _galerkin_iterate(A, Minv, rhs[b].reshape(-1), x0[b].reshape(-1), j).reshape(T, n)
            assert np.max(np.abs(x[b] - xg)) <= tol * np.max(np.abs(xg)), (j, b)
