"""Writes the golden fixtures of this directory from the CPU restatement (oracle/).

The reference holds no golden vectors for this path and cannot run here (its
CPU path needs JAX), so the fixtures freeze the oracle's outputs on small
seeded cases: the GPU parity tests compare against them without running the
oracle, and tests/test_golden.py re-derives them on the CPU, so a change of the
oracle shows up as a fixture mismatch.  Each file holds its inputs (or the
generator's seed and the generated inputs, which the tests check first) and
the expected outputs, in float64.

    python tests/golden/make_fixtures.py      # from the repository root
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))

import oracle  # noqa: E402
from oracle.sqp_cpu import obstacle_sqp, quadrotor_sqp  # noqa: E402
from turbompc_amd.problems import configs  # noqa: E402
from turbompc_amd.problems.ocp import LinearOCP  # noqa: E402
from turbompc_amd.problems.quadrotor import make_quadrotor_config  # noqa: E402

ADMM_CFG = dict(check_every=25, adapt_rho_every=0, sigma=1e-6, eps_abs=1e-9, eps_rel=1e-9, rho_f_factor=1000.0,
                alpha=1.0)


def _np(t):
    return np.asarray(t.detach().cpu(), dtype=np.float64)


def qp_arrays(qp):
    return dict(D=_np(qp.cost.D), E=_np(qp.cost.E), q=_np(qp.cost.q), A0=_np(qp.eq.A0), A_minus=_np(qp.eq.A_minus),
                A_plus=_np(qp.eq.A_plus), c0=_np(qp.eq.c0), c=_np(qp.eq.c), G=_np(qp.ineq.G), l=_np(qp.ineq.l),
                u=_np(qp.ineq.u))


def qp_ns(a, slack_weight=0.0, use_slack=False):
    """The duck-typed QP the oracle takes, from the arrays of a fixture."""
    from types import SimpleNamespace as NS
    return NS(cost=NS(D=a["D"], E=a["E"], q=a["q"]),
              eq=NS(A0=a["A0"], A_minus=a["A_minus"], A_plus=a["A_plus"], c0=a["c0"], c=a["c"]),
              ineq=NS(G=a["G"], l=a["l"], u=a["u"], slack_penalization_weight=slack_weight,
                      use_slack_variables=use_slack))


def admm_initial_state(a, rho0):
    B, T, n = a["q"].shape
    m, nx, n0 = a["l"].shape[-1], a["A_minus"].shape[-2], a["A0"].shape[-2]
    z0 = np.clip(np.zeros((B, T, m)), a["l"], a["u"])
    return oracle.OracleState(np.zeros((B, T, n)), np.zeros((B, T, m)), np.zeros((B, n0)),
                              np.zeros((B, T - 1, nx)), z0, np.zeros((B, T, m)), np.full((B,), float(rho0)))


def admm_config1():
    """config 1 (B = 4): 50 ADMM iterations from x = 0, rho = 0.1."""
    prob = configs.config1(B=4, seed=0)
    a = qp_arrays(prob.build_qp(*prob.initial_guess()))
    cfg = oracle.OracleCfg(max_iter=50, **ADMM_CFG)
    st, iters, _ = oracle.admm_solve(qp_ns(a), admm_initial_state(a, 0.1), cfg, schur="direct")
    out = {f"out_{k}": np.asarray(v, dtype=np.float64) for k, v in st._asdict().items()}
    return dict(a, rho0=np.array(0.1), max_iter=np.array(50), iters=np.asarray(iters), **out)


def _quadrotor_static(prob):
    D, E, q = (_np(t) for t in prob.cost_blocks())
    A0, c0 = (_np(t) for t in prob.initial_equality())
    G, l, u = (_np(t) for t in prob.inequality_blocks())
    return dict(D=D, E=E, q=q, A0=A0, c0=c0, A_plus=_np(prob.a_plus()), G=G, l=l, u=u)


def sqp_config3():
    """config 3 shapes (quadrotor, B = 4, seed 0): 5 SQP x 20 ADMM."""
    prob = make_quadrotor_config(B=4, seed=0, dtype=torch.float64, device="cpu")
    static = _quadrotor_static(prob)
    xg, ug = (_np(t) for t in prob.initial_guess())
    cfg = oracle.OracleCfg(max_iter=20, **ADMM_CFG)
    xs, us, st = quadrotor_sqp(static, xg, ug, dt=prob.dt, params=prob.params, cfg=cfg, rho0=0.1, n_sqp=5)
    return dict(B=np.array(4), seed=np.array(0), x0=_np(prob.x0), x_ref=_np(prob.x_ref), states_guess=xg,
                controls_guess=ug, states=xs, controls=us, y_f_dyn=st.y_f_dyn, y_g=st.y_g)


def linesearch_config4():
    """config 4 shapes (obstacles, B = 3, seed 0, soft rows with gamma = 50):
    8 SQP x 30 ADMM with the merit line search."""
    gamma = 50.0
    prob = configs.config4(B=3, seed=0, use_slack_variables=True, slack_penalization_weight=gamma)
    D, E, q = (_np(t) for t in prob.cost_blocks())
    A0, c0 = (_np(t) for t in prob.initial_equality())
    G, l, u = (_np(t) for t in LinearOCP.inequality_blocks(prob))
    static = dict(D=D, E=E, q=q, A0=A0, c0=c0, A_plus=_np(prob.a_plus()), G=G, l=l, u=u)
    xg, ug = (_np(t) for t in prob.initial_guess())
    Am, c = (_np(t) for t in prob.dynamics_blocks(*prob.initial_guess()))
    cfg = oracle.OracleCfg(max_iter=30, check_every=50, adapt_rho_every=0, sigma=1e-6, eps_abs=1e-9, eps_rel=1e-9,
                           rho_f_factor=1000.0, alpha=1.0)
    xs, us, st, sl, alphas = obstacle_sqp(static, xg, ug, A_minus=Am, c=c, centers=_np(prob.centers),
                                          radii=_np(prob.radii), dim=3, cfg=cfg, rho0=0.1, n_sqp=8,
                                          slack_weight=gamma, use_slack=True, linesearch={})
    return dict(B=np.array(3), seed=np.array(0), gamma=np.array(gamma), x0=_np(prob.x0), centers=_np(prob.centers),
                radii=_np(prob.radii), states=xs, controls=us, slacks=sl, xi_g=st.xi_g, alphas=alphas)


def adjoint_config5():
    """config 5 (B = 2): the adjoint KKT of the QP at the initial guess with a
    random active-sign pattern and right-hand side."""
    prob = configs.config5(B=2, seed=0)
    a = qp_arrays(prob.build_qp(*prob.initial_guess()))
    rng = np.random.default_rng(5)
    sign = rng.choice([-1.0, 0.0, 1.0], size=a["l"].shape, p=[0.2, 0.6, 0.2])
    a["G"] = a["G"] * sign[..., None]
    a["q"] = rng.standard_normal(a["q"].shape)
    dz, mult = oracle.adjoint_kkt(qp_ns(a))
    return dict(a, dz=np.asarray(dz, dtype=np.float64), mult=np.asarray(mult, dtype=np.float64))


def quadrotor_step():
    """The RK4 step of the quadrotor at random states and controls (B = 3, N = 6)."""
    prob = make_quadrotor_config(B=3, seed=2, dtype=torch.float64, device="cpu")
    rng = np.random.default_rng(3)
    s = rng.standard_normal((3, 7, 13))
    s[..., 3:7] /= np.linalg.norm(s[..., 3:7], axis=-1, keepdims=True)
    u = rng.uniform(0.0, 4.0, (3, 7, 4))
    xu = np.concatenate([s[:, :-1], u[:, :-1]], axis=-1).reshape(-1, 17)
    f, J = oracle.quadrotor_rk4_jac(xu, float(prob.dt), prob.params)
    return dict(states=s, controls=u, dt=np.array(float(prob.dt)), params=np.asarray(prob.params, dtype=np.float64),
                next=f.reshape(3, 6, 13), jac=J.reshape(3, 6, 13, 17))


FIXTURES = {
    "admm_config1": admm_config1,
    "sqp_config3": sqp_config3,
    "linesearch_config4": linesearch_config4,
    "adjoint_config5": adjoint_config5,
    "quadrotor_step": quadrotor_step,
}


def main():
    for name, fn in FIXTURES.items():
        np.savez_compressed(HERE / f"{name}.npz", **fn())
        print(f"wrote {name}.npz ({(HERE / f'{name}.npz').stat().st_size} bytes)")


if __name__ == "__main__":
    main()
