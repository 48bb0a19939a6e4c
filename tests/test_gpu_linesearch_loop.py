"""The merit line-search SQP loop on the device SQP step (_solve_impl_device_ls)
against the host-masked loop (_solve_impl_masked) on the same inputs: the
iterates, the ADMM state, the steps chosen and every per-iteration record,
bit for bit, with fixed iteration counts and with per-problem termination
(tol_convergence > 0, problems stopping at different iterations)."""
import copy

import pytest
import torch

from turbompc_amd.problems import configs
from turbompc_amd.problems.quadrotor import make_quadrotor_config
from turbompc_amd.solvers.turbompc_solver import DEFAULT_SOLVER_PARAMS, TurboMPCSolver

pytestmark = pytest.mark.gpu


def _params(n_sqp, admm_iters, tol):
    p = copy.deepcopy(DEFAULT_SOLVER_PARAMS)
    p["num_sqp_iteration_max"] = n_sqp
    p["tol_convergence"] = tol
    p["admm"]["max_iter"] = admm_iters
    p["admm"]["adapt_rho_every"] = 0
    p["admm"]["relaxation_parameter"] = 1.0
    p["linesearch"] = True
    return p


def _tol_splitting(prob, params, k):
    """A tolerance that stops about half the problems after SQP iteration k:
    the median of the convergence errors recorded there at tol 0."""
    p0 = copy.deepcopy(params)
    p0["tol_convergence"] = 0.0
    solver = TurboMPCSolver(prob, p0)
    errs = solver.solve(solver.initial_guess()).solver_stats.convergence_errors[:, k]
    return float(errs.median())


def _both(prob, params):
    out = []
    for loop in ("device", "masked"):
        solver = TurboMPCSolver(prob, params)
        solver._sqp_loop = loop
        out.append(solver.solve(solver.initial_guess()))
    torch.cuda.synchronize()
    return out


def _assert_same(a, b):
    for k in ("states", "controls", "slack", "num_iter", "convergence_error", "admm_iters", "linesearch_alphas",
              "nonfinite"):
        assert torch.equal(getattr(a, k), getattr(b, k)), k
    for k in a.admm_state._fields:
        assert torch.equal(getattr(a.admm_state, k), getattr(b.admm_state, k)), k
    for k in a.solver_stats._fields:
        assert torch.equal(getattr(a.solver_stats, k), getattr(b.solver_stats, k)), k
    for k in a.kkt_state._fields:
        x, y = getattr(a.kkt_state, k), getattr(b.kkt_state, k)
        assert (x is None and y is None) or torch.equal(x, y), k


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("stop", [False, True])
def test_quadrotor_linesearch_device_loop_equals_masked(dtype, stop):
    prob = make_quadrotor_config(B=24, seed=4, dtype=dtype, device="cuda")
    params = _params(8, 20, 0.0)
    if stop:
        params["tol_convergence"] = _tol_splitting(prob, params, 3)
    dev, msk = _both(prob, params)
    print(f"  tol {params['tol_convergence']:.3g}, SQP iterations per problem {dev.num_iter.tolist()}", flush=True)
    _assert_same(dev, msk)
    if stop:  # problems stop at different iterations
        assert len(set(dev.num_iter.tolist())) >= 2


@pytest.mark.parametrize("use_slack", [False, True])
@pytest.mark.parametrize("stop", [False, True])
def test_config4_linesearch_device_loop_equals_masked(use_slack, stop):
    prob = configs.config4(B=12, seed=1, use_slack_variables=use_slack, slack_penalization_weight=50.0).to("cuda")
    params = _params(8, 30, 0.0)
    if stop:
        params["tol_convergence"] = _tol_splitting(prob, params, 3)
    dev, msk = _both(prob, params)
    print(f"  tol {params['tol_convergence']:.3g}, SQP iterations per problem {dev.num_iter.tolist()}", flush=True)
    _assert_same(dev, msk)
    if stop:
        assert len(set(dev.num_iter.tolist())) >= 2
