"""The HIP path against the committed golden fixtures (tests/golden/*.npz,
outputs of the CPU restatement, re-derived on the CPU by tests/test_golden.py):
a fixed-count ADMM solve (config 1), the quadrotor SQP (config 3 shapes, 5 x 20),
the SQP with the merit line search on soft obstacle rows (config 4 shapes,
8 x 30), the adjoint KKT (config 5), and the quadrotor RK4 step and Jacobian."""
import copy
from pathlib import Path

import numpy as np
import pytest
import torch

from helpers import TOL, rel_err
from turbompc_amd.problems import configs
from turbompc_amd.problems.quadrotor import make_quadrotor_config
from turbompc_amd.solvers.admm.admm import ADMMSolver, ADMMState
from turbompc_amd.solvers.backward.backward_kkt_hip import solve_backward_kkt_hip
from turbompc_amd.solvers.linear_systems_solvers.backends import AdmmBackend
from turbompc_amd.solvers.qp_data import QPCostBlocks, QPData, QPEqualityBlocks, QPInequalityBlocks
from turbompc_amd.solvers.qp_utils import ZShape
from turbompc_amd.solvers.turbompc_solver import DEFAULT_SOLVER_PARAMS, TurboMPCSolver

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLDEN = Path(__file__).resolve().parent / "golden"


def _load(name):
    return np.load(GOLDEN / f"{name}.npz")


def _qp(z):
    t = lambda k: torch.tensor(z[k], dtype=torch.float64, device=DEV)  # noqa: E731
    return QPData(cost=QPCostBlocks(t("D"), t("E"), t("q")),
                  eq=QPEqualityBlocks(t("A0"), t("A_minus"), t("A_plus"), t("c0"), t("c")),
                  ineq=QPInequalityBlocks(t("G"), t("l"), t("u"), torch.tensor(0.0, dtype=torch.float64), False))


def _params(n_sqp, admm_iters, linesearch=False):
    p = copy.deepcopy(DEFAULT_SOLVER_PARAMS)
    p["num_sqp_iteration_max"] = n_sqp
    p["tol_convergence"] = 0.0
    p["admm"]["max_iter"] = admm_iters
    p["admm"]["adapt_rho_every"] = 0
    p["admm"]["relaxation_parameter"] = 1.0
    p["linesearch"] = linesearch
    return p


def test_admm_config1_matches_golden():
    z = _load("admm_config1")
    qp = _qp(z)
    B, T, n, nx, n0, m = qp.dims
    solver = ADMMSolver(ZShape(T - 1, nx, n - nx), {"max_iter": 200, "tol_epsilon": 1e-8}, sigma=1e-6,
                        max_iter=int(z["max_iter"]), eps_abs=1e-9, eps_rel=1e-9, check_termination_every=25,
                        adapt_rho_every=0, rho_f_factor=1000.0, admm_backend=AdmmBackend.HIP_DIRECT)
    st0 = solver.initial_state(qp, rho_bar=float(z["rho0"]))
    (_, _), stats, out = solver.solve(qp, st0, alpha=1.0)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(stats.num_iter.cpu().numpy(), z["iters"])
    for k in ADMMState._fields:
        if z[f"out_{k}"].size:
            assert rel_err(getattr(out, k), z[f"out_{k}"]) < TOL[torch.float64], k


def test_sqp_config3_matches_golden():
    z = _load("sqp_config3")
    prob = make_quadrotor_config(B=int(z["B"]), seed=int(z["seed"]), dtype=torch.float64, device=DEV)
    # the generator still makes the problems the fixture was made from
    np.testing.assert_array_equal(prob.x0.cpu().numpy(), z["x0"])
    np.testing.assert_array_equal(prob.x_ref.cpu().numpy(), z["x_ref"])
    solver = TurboMPCSolver(prob, _params(5, 20))
    sol = solver.solve(solver.initial_guess())
    torch.cuda.synchronize()
    assert rel_err(sol.states, z["states"]) < TOL[torch.float64]
    assert rel_err(sol.controls, z["controls"]) < TOL[torch.float64]
    assert rel_err(sol.admm_state.y_f_dyn, z["y_f_dyn"]) < 1e-8


def test_linesearch_config4_matches_golden():
    z = _load("linesearch_config4")
    prob = configs.config4(B=int(z["B"]), seed=int(z["seed"]), use_slack_variables=True,
                           slack_penalization_weight=float(z["gamma"]))
    np.testing.assert_array_equal(prob.x0.numpy(), z["x0"])
    np.testing.assert_array_equal(prob.centers.numpy(), z["centers"])
    solver = TurboMPCSolver(prob.to(DEV), _params(8, 30, linesearch=True))
    sol = solver.solve(solver.initial_guess())
    torch.cuda.synchronize()
    np.testing.assert_array_equal(sol.linesearch_alphas.cpu().numpy(), z["alphas"])
    assert rel_err(sol.states, z["states"]) < TOL[torch.float64]
    assert rel_err(sol.controls, z["controls"]) < TOL[torch.float64]
    assert rel_err(sol.slack, z["xi_g"]) < 1e-8


def test_adjoint_config5_matches_golden():
    z = _load("adjoint_config5")
    dz, mult = solve_backward_kkt_hip(_qp(z))
    torch.cuda.synchronize()
    assert rel_err(dz, z["dz"]) < TOL[torch.float64]
    assert rel_err(mult, z["mult"]) < TOL[torch.float64]


def test_quadrotor_step_and_jacobian_match_golden():
    z = _load("quadrotor_step")
    B, T = z["states"].shape[:2]
    prob = make_quadrotor_config(B=B, seed=2, N=T - 1, dtype=torch.float64, device=DEV)
    assert float(prob.dt) == float(z["dt"])
    np.testing.assert_array_equal(np.asarray(prob.params), z["params"])
    s = torch.tensor(z["states"], device=DEV)
    u = torch.tensor(z["controls"], device=DEV)
    nxt = prob.next_states(s, u)
    Am, c = prob.dynamics_blocks(s, u)
    torch.cuda.synchronize()
    assert rel_err(nxt, z["next"]) < 1e-13
    assert rel_err(Am, z["jac"]) < 1e-10
    # c = J z - f at the linearization point
    zz = np.concatenate([z["states"][:, :-1], z["controls"][:, :-1]], axis=-1)
    assert rel_err(c, np.einsum("btij,btj->bti", z["jac"], zz) - z["next"]) < 1e-10
