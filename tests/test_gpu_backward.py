"""Backward pass of the differentiable solve (a14 adjoint KKT end to end, a15
gradient assembly): gradients of L = <cs, states> + <cu, controls> with
respect to the initial state and the tracking weights, against central
differences of the forward solve; and the quadrotor's dynamics Lagrangian
Hessian against differences of its linearization."""
import copy

import numpy as np
import pytest
import torch

from helpers import rel_err
from turbompc_amd.problems import configs
from turbompc_amd.problems.quadrotor import make_quadrotor_config
from turbompc_amd.solvers.turbompc_solver import DEFAULT_SOLVER_PARAMS, TurboMPCSolver

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _tight_params(n_sqp, admm_iters, tol=0.0, eps=1e-13):
    p = copy.deepcopy(DEFAULT_SOLVER_PARAMS)
    p["num_sqp_iteration_max"] = n_sqp
    p["tol_convergence"] = tol
    p["admm"]["max_iter"] = admm_iters
    p["admm"]["eps_abs"] = eps
    p["admm"]["eps_rel"] = eps
    return p


def test_quadrotor_lagrangian_hessian_matches_jacobian_differences():
    B = 3
    prob = make_quadrotor_config(B=B, seed=4, dtype=torch.float64, device=DEV)
    g = torch.Generator().manual_seed(9)
    xs, us = prob.initial_guess()
    xs = xs + 0.2 * torch.randn(xs.shape, generator=g, dtype=torch.float64).to(DEV)
    us = us + 1.0 + 0.3 * torch.randn(us.shape, generator=g, dtype=torch.float64).to(DEV)
    N = prob.horizon
    lam = torch.randn((B, N, 13), generator=g, dtype=torch.float64).to(DEV)
    H = prob.dynamics_lagrangian_hessian(xs, us, lam)
    assert H.shape == (B, N + 1, 17, 17)
    assert torch.equal(H[:, N], torch.zeros_like(H[:, N]))
    assert rel_err(H, H.transpose(-1, -2)) == 0.0
    h = 1e-5
    cols = []
    for j in range(17):
        dx, du = torch.zeros_like(xs), torch.zeros_like(us)
        if j < 13:
            dx[..., j] = h
        else:
            du[..., j - 13] = h
        Ap, _ = prob.dynamics_blocks(xs + dx, us + du)
        Am, _ = prob.dynamics_blocks(xs - dx, us - du)
        cols.append(torch.einsum("bti,btik->btk", lam, (Ap - Am) / (2 * h)))
    Hfd = torch.stack(cols, dim=-1)  # column j of d/dz (lambda . J)
    assert rel_err(H[:, :N], Hfd) < 1e-6


def _check_gradients(solver, prob, n_checks, h, rtol, seed, floor=1e-2, warm=False):
    """warm: the finite-difference solves start from the solution (states,
    controls and ADMM state), which a converged SQP reaches again in a few
    iterations."""
    guess = solver.initial_guess()
    g = torch.Generator().manual_seed(seed)
    B, T, nx = guess.states.shape
    cs = torch.randn(guess.states.shape, generator=g, dtype=torch.float64).to(DEV)
    cu = torch.randn(guess.controls.shape, generator=g, dtype=torch.float64).to(DEV)
    fsolve = solver.get_differentiable_solve_function()
    x0 = prob.x0.clone().requires_grad_(True)
    w = {k: v.clone().requires_grad_(True) for k, v in prob.weights_dict().items()}
    sol = fsolve(guess, {"initial_state": x0}, w)
    L = (cs * sol.states).sum() + (cu * sol.controls).sum()
    L.backward()
    if warm:
        guess = sol._replace(states=sol.states.detach(), controls=sol.controls.detach())

    def loss(x0v, wv):
        s = solver.solve(guess, {"initial_state": x0v}, wv)
        return float((cs * s.states).sum() + (cu * s.controls).sum())

    base_w = {k: v.detach().clone() for k, v in w.items()}
    rng = np.random.default_rng(seed)
    checks = [("x0", int(rng.integers(B)), int(rng.integers(nx))) for _ in range(n_checks)]
    for k, v in base_w.items():
        checks += [(k, int(rng.integers(B)), int(rng.integers(v.shape[1]))) for _ in range(n_checks)]
    for name, b, i in checks:
        if name == "x0":
            xp, xm = x0.detach().clone(), x0.detach().clone()
            xp[b, i] += h
            xm[b, i] -= h
            fd = (loss(xp, base_w) - loss(xm, base_w)) / (2 * h)
            got = float(x0.grad[b, i])
        else:
            wp = {k: v.clone() for k, v in base_w.items()}
            wm = {k: v.clone() for k, v in base_w.items()}
            wp[name][b, i] += h
            wm[name][b, i] -= h
            fd = (loss(x0.detach(), wp) - loss(x0.detach(), wm)) / (2 * h)
            got = float(w[name].grad[b, i])
        print(f"  {name}[{b},{i}]: adjoint {got:.9g}  central difference {fd:.9g}", flush=True)
        assert abs(got - fd) <= rtol * max(abs(fd), floor), (name, b, i, got, fd)


def test_linear_ocp_gradients_match_finite_differences():
    # config 1 (double integrator, control bounds): one QP, solved to ~1e-12
    prob = configs.config1(B=3, seed=2).to(DEV, torch.float64)
    solver = TurboMPCSolver(prob, _tight_params(1, 4000))
    _check_gradients(solver, prob, n_checks=3, h=1e-4, rtol=1e-4, seed=1)


def test_quadrotor_gradients_match_finite_differences():
    # nonlinear dynamics: the adjoint QP carries the exact Lagrangian Hessian;
    # full SQP steps from the straight-line guess need ~60 iterations to reach
    # a first-order error of ~1e-9, where implicit and finite-difference
    # derivatives agree (without the Hessian term they differ by ~20%)
    prob = make_quadrotor_config(B=2, seed=3, dtype=torch.float64, device=DEV)
    solver = TurboMPCSolver(prob, _tight_params(60, 1000))
    sol = solver.solve(solver.initial_guess())
    assert float(sol.convergence_error.max()) < 1e-7
    # gradients here span 5e-3 .. 2e2: the floor keeps the tiny ones to an
    # absolute 1e-4.  The difference solves start from the solution, so that
    # the + and - solves follow nearly the same iterations and their ~1e-9
    # convergence errors cancel in the difference: from the initial guess the
    # central differences of the weight gradients moved by 1.5e-4 between two
    # builds whose factorizations differ only in summation order.  The step
    # h = 1e-4 keeps that solve noise (about 1e-9 / h) a decade below the bar,
    # and the O(h^2) truncation error of the central difference far below it
    # (at h = 1e-5 a build that changed the summation order of the streaming
    # kernel's products moved one difference quotient by 1.05e-4)
    _check_gradients(solver, prob, n_checks=1, h=1e-4, rtol=1e-4, seed=2, floor=1.0, warm=True)


def test_obstacle_lagrangian_hessian_matches_gradient_differences():
    B = 3
    prob = configs.config4(B=B, seed=6).to(DEV, torch.float64)
    xs, us = prob.initial_guess()
    g = torch.Generator().manual_seed(4)
    xs = xs + 0.3 * torch.randn(xs.shape, generator=g, dtype=torch.float64).to(DEV)
    m, mb = prob.num_inequality_constraints, prob.num_box_constraints
    mus = torch.randn((B, prob.horizon + 1, m), generator=g, dtype=torch.float64).to(DEV)
    H = prob.inequality_lagrangian_hessian(xs, us, mus)
    h = 1e-6
    cols = []
    for j in range(9):
        dx = torch.zeros_like(xs)
        if j < 6:
            dx[..., j] = h
        Gp, _, _ = prob.inequality_blocks_at(xs + dx, us)
        Gm, _, _ = prob.inequality_blocks_at(xs - dx, us)
        cols.append(torch.einsum("bti,btik->btk", mus[..., mb:], (Gp - Gm)[:, :, mb:] / (2 * h)))
    Hfd = torch.stack(cols, dim=-1)
    assert rel_err(H, Hfd) < 1e-7


def test_obstacle_gradients_match_finite_differences():
    # nonlinear inequality rows: the adjoint QP carries their Lagrangian Hessian
    prob = configs.config4(B=2, seed=7).to(DEV, torch.float64)
    # solves stopped at a first-order error of 1e-11, differences over h = 1e-4:
    # the difference quotient's error (about tol / h) stays well below the bar
    solver = TurboMPCSolver(prob, _tight_params(40, 4000, tol=1e-11, eps=1e-12))
    sol = solver.solve(solver.initial_guess())
    print(f"  SQP iterations {sol.num_iter.tolist()}, first-order error {sol.convergence_error.tolist()}", flush=True)
    assert float(sol.convergence_error.max()) < 1e-8
    # every problem has an active obstacle row, so the Hessian term is in play
    mb = prob.num_box_constraints
    assert bool((sol.admm_state.y_g[..., mb:].abs().flatten(1).amax(dim=1) > 1.0).all())
    _check_gradients(solver, prob, n_checks=2, h=1e-4, rtol=1e-4, seed=3, floor=1.0, warm=True)


def test_slack_weight_gradient_matches_finite_differences():
    # soft obstacle rows: dL/dgamma from the active slacks
    # (_recover_slack_active_ineq_gradient, turbompc_solver.py:620-643)
    gamma = 20.0
    prob = configs.config4(B=2, seed=7, use_slack_variables=True,
                           slack_penalization_weight=gamma).to(DEV, torch.float64)
    solver = TurboMPCSolver(prob, _tight_params(40, 4000, tol=1e-10, eps=1e-12))
    gam = torch.tensor(gamma, dtype=torch.float64, requires_grad=True)
    x0 = prob.x0.clone().requires_grad_(True)
    out = solver.get_differentiable_solve_function()(solver.initial_guess(), {"initial_state": x0},
                                                     {"slack_penalization_weight": gam})
    print(f"  SQP iterations {out.num_iter.tolist()}, first-order error {out.convergence_error.tolist()}", flush=True)
    assert float(out.convergence_error.max()) < 1e-8
    assert float(out.slack.abs().max()) > 1e-4
    mb = prob.num_box_constraints
    assert float(out.slack[..., mb:].abs().max()) > 1e-4  # a softened obstacle row
    g = torch.Generator().manual_seed(5)
    cs = torch.randn(out.states.shape, generator=g, dtype=torch.float64).to(DEV)
    cu = torch.randn(out.controls.shape, generator=g, dtype=torch.float64).to(DEV)
    ((cs * out.states).sum() + (cu * out.controls).sum()).backward()
    guess = out._replace(states=out.states.detach(), controls=out.controls.detach())  # warm start

    def loss(gv, x0v):
        s = solver.solve(guess, {"initial_state": x0v}, {"slack_penalization_weight": gv})
        return float((cs * s.states).sum() + (cu * s.controls).sum())

    h = 1e-4
    fd = (loss(gamma + h, prob.x0) - loss(gamma - h, prob.x0)) / (2 * h)
    print(f"  gamma: adjoint {float(gam.grad):.9g}  central difference {fd:.9g}", flush=True)
    assert abs(float(gam.grad) - fd) <= 1e-4 * max(abs(fd), 1e-2), (float(gam.grad), fd)
    for b, i in ((0, 1), (1, 4)):
        xp, xm = prob.x0.clone(), prob.x0.clone()
        xp[b, i] += 1e-5
        xm[b, i] -= 1e-5
        fd = (loss(gamma, xp) - loss(gamma, xm)) / 2e-5
        print(f"  x0[{b},{i}]: adjoint {float(x0.grad[b, i]):.9g}  central difference {fd:.9g}", flush=True)
        assert abs(float(x0.grad[b, i]) - fd) <= 1e-4 * max(abs(fd), 1.0), (b, i, float(x0.grad[b, i]), fd)
