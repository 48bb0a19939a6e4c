"""TEST INFRASTRUCTURE ONLY — CPU restatement of the SQP loop for the quadrotor
and obstacle-avoidance workloads.

Restates TurboMPCSolver._solve_impl (turbompc/solvers/turbompc_solver.py:1519-1760)
with the first_order criterion at a fixed iteration count (tol_convergence = 0):
  linearize (RK4 Jacobians by complex step, liboracle; obstacle rows in numpy)
  -> ADMM (liboracle)
  -> relinearize at the new iterate, carrying the ADMM state (including rho)
Used by bench.py's cpu_baseline leg and by the SQP parity tests.

Pins: the quadrotor Jacobians are checked against central differences and
torch.func.jacfwd (tests/test_oracle_adjoint_quadrotor.py); the obstacle rows
against central differences of g, known answers on the sphere and the exactness
of the linearization at its own point, and their Hessian against differences
of the gradient and its null direction (tests/test_oracle_obstacle.py).
"""
from __future__ import annotations

from collections import namedtuple
from types import SimpleNamespace

import numpy as np

from . import oracle as ora

QPNS = namedtuple("QPNS", ["cost", "eq", "ineq"])


def _ns(**kw):
    return SimpleNamespace(**kw)


def linearize_quadrotor(states, controls, dt, params):
    """A_minus (B,N,13,17), c (B,N,13) at (states, controls) (B,T,13), (B,T,4)."""
    B, T, _ = states.shape
    N = T - 1
    xu = np.concatenate([states[:, :-1], controls[:, :-1]], axis=-1).reshape(-1, 17)
    f, J = ora.quadrotor_rk4_jac(xu, dt, params)
    c = -f + np.einsum("kij,kj->ki", J, xu)
    return J.reshape(B, N, 13, 17), c.reshape(B, N, 13)


OBSTACLE_MARGIN = 0.001
OBSTACLE_LOWER = -1.0e9


def linearize_obstacles(states, centers, radii, dim):
    """Obstacle rows of get_inequalities_linearized_matrices
    (optimal_control_problem.py:580-626) for g_k = 1 - |p - c_k| / (r_k + 0.001)
    (obstacle_avoidance.py:28-41), l = -1e9, u = 0: returns the gradient rows
    Gx (B,T,K,dim) over the position block and the linearized bounds
    l, u (B,T,K) = bound - (g(xbar) - Gx xbar)."""
    p = states[..., None, :dim]  # (B,T,1,dim)
    d = p - centers[:, None]  # (B,T,K,dim)
    nrm = np.sqrt(np.sum(d * d, axis=-1))
    den = radii[:, None] + OBSTACLE_MARGIN
    g = 1.0 - nrm / den
    grad = -(d / nrm[..., None]) / den[..., None]
    off = g - np.sum(grad * p, axis=-1)
    return grad, OBSTACLE_LOWER - off, 0.0 - off


def obstacle_hessian(states, centers, radii, dim, mus, n):
    """(B,T,n,n) sum_k mu_k d^2 g_k/dz^2 (get_inequality_lagrangian_hessian,
    optimal_control_problem.py:1443-1480): -(I/|d| - d d^T/|d|^3)/(r + 0.001)
    on the position block."""
    p = states[..., None, :dim]
    d = p - centers[:, None]
    nrm = np.sqrt(np.sum(d * d, axis=-1))
    den = radii[:, None] + OBSTACLE_MARGIN
    eye = np.eye(dim)
    hk = -(eye / nrm[..., None, None] - d[..., :, None] * d[..., None, :] / nrm[..., None, None] ** 3) / den[..., None, None]
    B, T = states.shape[:2]
    H = np.zeros((B, T, n, n))
    H[..., :dim, :dim] = np.einsum("btk,btkij->btij", mus, hk)
    return H


def sqp_fixed(qp_at, x_guess, u_guess, *, n, m, n0, cfg: "ora.OracleCfg", rho0, n_sqp, dtype=np.float64,
              nthreads=None):
    """Fixed-count SQP: qp_at(states, controls) -> QP; the ADMM state (including
    rho and the slack) carries across iterations; x starts at 0
    (turbompc_solver.py:1545-1551).  Returns (states, controls, admm_state)."""
    states, controls = x_guess.astype(np.float64), u_guess.astype(np.float64)
    B, T, nx = states.shape
    qp = qp_at(states, controls)
    z0 = np.clip(np.zeros((B, T, m)), qp.ineq.l, qp.ineq.u)
    st = ora.OracleState(np.zeros((B, T, n)), np.zeros((B, T, m)), np.zeros((B, n0)),
                         np.zeros((B, T - 1, nx)), z0, np.zeros((B, T, m)), np.full((B,), float(rho0)))
    for it in range(n_sqp):
        st, _, _ = ora.admm_solve(qp, st, cfg, schur="direct", dtype=dtype, nthreads=nthreads)
        st = ora.OracleState(*[np.asarray(a, dtype=np.float64) for a in st])
        states, controls = st.x_blocks[..., :nx], st.x_blocks[..., nx:]
        if it + 1 < n_sqp:
            qp = qp_at(states, controls)
    return states, controls, st


def obstacle_sqp(static, x_guess, u_guess, *, A_minus, c, centers, radii, dim, cfg: "ora.OracleCfg", rho0, n_sqp,
                 slack_weight=0.0, use_slack=False, dtype=np.float64, nthreads=None):
    """static: numpy QP blocks that do not change (D, E, q, A0, c0, A_plus) and
    the box rows (G, l, u) (B,T,mb,n); the obstacle rows follow the box rows."""
    Gb, lb, ub = static["G"], static["l"], static["u"]
    B, T, mb, n = Gb.shape
    K = centers.shape[1]

    def qp_at(s, u):
        grad, lo, up = linearize_obstacles(s, centers, radii, dim)
        Go = np.zeros((B, T, K, n))
        Go[..., :dim] = grad
        return QPNS(
            _ns(D=static["D"], E=static["E"], q=static["q"]),
            _ns(A0=static["A0"], A_minus=A_minus, A_plus=static["A_plus"], c0=static["c0"], c=c),
            _ns(G=np.concatenate([Gb, Go], axis=2), l=np.concatenate([lb, lo], axis=2),
                u=np.concatenate([ub, up], axis=2), slack_penalization_weight=slack_weight,
                use_slack_variables=use_slack),
        )

    return sqp_fixed(qp_at, x_guess, u_guess, n=n, m=mb + K, n0=static["A0"].shape[-2], cfg=cfg, rho0=rho0,
                     n_sqp=n_sqp, dtype=dtype, nthreads=nthreads)


def quadrotor_sqp(static, x_guess, u_guess, *, dt, params, cfg: "ora.OracleCfg", rho0, n_sqp, dtype=np.float64,
                  nthreads=None):
    """static: dict of numpy QP blocks that do not change (D, E, q, A0, c0, A_plus, G, l, u).
    Returns (states, controls, admm_state)."""
    n = static["D"].shape[-1]
    m = static["G"].shape[-2]

    def qp_at(s, u):
        Am, c = linearize_quadrotor(s, u, dt, params)
        return QPNS(
            _ns(D=static["D"], E=static["E"], q=static["q"]),
            _ns(A0=static["A0"], A_minus=Am, A_plus=static["A_plus"], c0=static["c0"], c=c),
            _ns(G=static["G"], l=static["l"], u=static["u"], slack_penalization_weight=0.0,
                use_slack_variables=False),
        )

    return sqp_fixed(qp_at, x_guess, u_guess, n=n, m=m, n0=static["A0"].shape[-2], cfg=cfg, rho0=rho0,
                     n_sqp=n_sqp, dtype=dtype, nthreads=nthreads)
