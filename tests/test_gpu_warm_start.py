"""Warm-started MPC solves against the CPU SQP: a second solve from the first
solve's solution shifted by one stage, with the first solve's ADMM state
(rho included) passed through and the next initial state x_1, as in the
reference's closed-loop usage (docs/API.md:146-163;
turbompc/solvers/turbompc_solver.py:1032-1037, :1545-1551: no fresh ADMM
state when one is given).  The CPU SQP takes the same starting state
(oracle/sqp_cpu.py sqp_fixed, pinned by test_oracle_sqp's chain test).
fp64 at the 1e-9 parity bar, on the device SQP loop, the host-masked loop and
the line-search loop."""
import copy

import numpy as np
import pytest
import torch

import oracle
from helpers import TOL, rel_err
from oracle.sqp_cpu import obstacle_sqp, quadrotor_sqp
from turbompc_amd.problems import configs
from turbompc_amd.problems.ocp import QuadraticTrackingOCP
from turbompc_amd.problems.quadrotor import make_quadrotor_config
from turbompc_amd.solvers.turbompc_solver import DEFAULT_SOLVER_PARAMS, TurboMPCSolver

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _params(n_sqp, admm_iters, linesearch=False):
    p = copy.deepcopy(DEFAULT_SOLVER_PARAMS)
    p["num_sqp_iteration_max"] = n_sqp
    p["tol_convergence"] = 0.0
    p["admm"]["max_iter"] = admm_iters
    p["admm"]["adapt_rho_every"] = 0
    p["admm"]["relaxation_parameter"] = 1.0
    p["linesearch"] = linesearch
    return p


def _shift(a):
    """The receding-horizon shift: stages 1..N, then stage N again."""
    return np.concatenate([a[:, 1:], a[:, -1:]], axis=1)


def _shift_t(t):
    return torch.cat([t[:, 1:], t[:, -1:]], dim=1)


def _static(prob):
    """The QP blocks that do not depend on the iterate, with the box rows
    (the obstacle rows of config 4 are linearized by the CPU SQP itself)."""
    D, E, q = (t.numpy() for t in prob.cost_blocks())
    A0, c0 = (t.numpy() for t in prob.initial_equality())
    G, l, u = (t.numpy() for t in QuadraticTrackingOCP.inequality_blocks(prob))
    return dict(D=D, E=E, q=q, A0=A0, c0=c0, A_plus=prob.a_plus().numpy(), G=G, l=l, u=u)


@pytest.mark.parametrize("loop", ["device", "masked", "linesearch"])
def test_quadrotor_warm_started_second_solve_matches_cpu(loop):
    B, n_sqp, K = 8, 3, 10
    ls = loop == "linesearch"
    cfg = oracle.OracleCfg(max_iter=K, check_every=25, adapt_rho_every=0, sigma=1e-6, eps_abs=1e-9, eps_rel=1e-9,
                           rho_f_factor=1000.0, alpha=1.0)
    cpu = make_quadrotor_config(B=B, seed=7, dtype=torch.float64, device="cpu")
    static = _static(cpu)
    xg, ug = (t.numpy() for t in cpu.initial_guess())
    kw = dict(dt=cpu.dt, params=cpu.params, cfg=cfg, rho0=0.1, n_sqp=n_sqp, linesearch={} if ls else None)
    xs1, us1, st1, *_ = quadrotor_sqp(static, xg, ug, **kw)
    x1 = xs1[:, 1].copy()  # the next initial state
    xs2, us2, st2, *_ = quadrotor_sqp(dict(static, c0=x1), _shift(xs1), _shift(us1), state0=st1, **kw)

    solver = TurboMPCSolver(make_quadrotor_config(B=B, seed=7, dtype=torch.float64, device=DEV),
                            _params(n_sqp, K, linesearch=ls))
    if loop == "masked":
        solver._sqp_loop = "masked"
    first = solver.solve(solver.initial_guess())
    assert rel_err(first.states, xs1) < TOL[torch.float64]
    guess = first._replace(states=_shift_t(first.states), controls=_shift_t(first.controls),
                           slack=_shift_t(first.slack))
    keep = [t.clone() for t in first.admm_state]
    second = solver.solve(guess, {"initial_state": first.states[:, 1]})
    torch.cuda.synchronize()
    errs = {"states": rel_err(second.states, xs2), "controls": rel_err(second.controls, us2),
            "y_f_dyn": rel_err(second.admm_state.y_f_dyn, st2.y_f_dyn), "y_g": rel_err(second.admm_state.y_g, st2.y_g)}
    print(f"warm-started quadrotor SQP ({loop}): " + ", ".join(f"{k} {v:.2e}" for k, v in errs.items()))
    assert errs["states"] < TOL[torch.float64] and errs["controls"] < TOL[torch.float64]
    assert errs["y_f_dyn"] < 1e-8 and errs["y_g"] < 1e-8
    # the caller's state is read, not updated
    for a, b in zip(first.admm_state, keep):
        assert torch.equal(a, b)
    # and the warm start matters: a cold second solve lands elsewhere
    cold = solver.solve(solver.initial_guess()._replace(states=guess.states, controls=guess.controls),
                        {"initial_state": first.states[:, 1]})
    assert rel_err(cold.states, xs2) > 1e-6


def test_config4_warm_started_second_solve_with_linesearch_matches_cpu():
    B, n_sqp, K = 6, 4, 30
    prob = configs.config4(B=B, seed=3)
    static = _static(prob)
    xg, ug = (t.numpy() for t in prob.initial_guess())
    Am, c = (t.numpy() for t in prob.dynamics_blocks(*prob.initial_guess()))
    cfg = oracle.OracleCfg(max_iter=K, check_every=50, adapt_rho_every=0, sigma=1e-6, eps_abs=1e-9, eps_rel=1e-9,
                           rho_f_factor=1000.0, alpha=1.0)
    kw = dict(A_minus=Am, c=c, centers=prob.centers.numpy(), radii=prob.radii.numpy(), dim=3, cfg=cfg, rho0=0.1,
              n_sqp=n_sqp, linesearch={})
    xs1, us1, st1, _, _ = obstacle_sqp(static, xg, ug, **kw)
    x1 = xs1[:, 1].copy()
    xs2, us2, st2, _, al2 = obstacle_sqp(dict(static, c0=x1), _shift(xs1), _shift(us1), state0=st1, **kw)

    solver = TurboMPCSolver(prob.to(DEV), _params(n_sqp, K, linesearch=True))
    first = solver.solve(solver.initial_guess())
    guess = first._replace(states=_shift_t(first.states), controls=_shift_t(first.controls),
                           slack=_shift_t(first.slack))
    second = solver.solve(guess, {"initial_state": first.states[:, 1]})
    torch.cuda.synchronize()
    np.testing.assert_array_equal(second.linesearch_alphas.cpu().numpy(), al2)
    e_s, e_u = rel_err(second.states, xs2), rel_err(second.controls, us2)
    print(f"warm-started config 4 SQP with line search: states {e_s:.2e}, controls {e_u:.2e}, steps {al2.tolist()}")
    assert e_s < TOL[torch.float64] and e_u < TOL[torch.float64]
    assert rel_err(second.admm_state.y_g, st2.y_g) < 1e-8
