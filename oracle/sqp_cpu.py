"""TEST INFRASTRUCTURE ONLY — CPU restatement of the SQP loop for the quadrotor workload.

Restates TurboMPCSolver._solve_impl (turbompc/solvers/turbompc_solver.py:1519-1760)
with the first_order criterion at a fixed iteration count (tol_convergence = 0):
  linearize (RK4 Jacobians by complex step, liboracle)  ->  ADMM (liboracle)
  -> relinearize at the new iterate, carrying the ADMM state (including rho)
Used by bench.py's cpu_baseline leg and by the SQP parity tests.
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


def quadrotor_sqp(static, x_guess, u_guess, *, dt, params, cfg: "ora.OracleCfg", rho0, n_sqp, dtype=np.float64,
                  nthreads=None):
    """static: dict of numpy QP blocks that do not change (D, E, q, A0, c0, A_plus, G, l, u).
    Returns (states, controls, admm_state)."""
    states, controls = x_guess.astype(np.float64), u_guess.astype(np.float64)
    B, T, nx = states.shape
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

    qp = qp_at(states, controls)
    z0 = np.clip(np.zeros((B, T, m)), static["l"], static["u"])
    st = ora.OracleState(np.zeros((B, T, n)), np.zeros((B, T, m)), np.zeros((B, static["A0"].shape[-2])),
                         np.zeros((B, T - 1, nx)), z0, np.zeros((B, T, m)), np.full((B,), float(rho0)))
    for it in range(n_sqp):
        st, _, _ = ora.admm_solve(qp, st, cfg, schur="direct", dtype=dtype, nthreads=nthreads)
        st = ora.OracleState(*[np.asarray(a, dtype=np.float64) for a in st])
        states, controls = st.x_blocks[..., :nx], st.x_blocks[..., nx:]
        if it + 1 < n_sqp:
            qp = qp_at(states, controls)
    return states, controls, st
