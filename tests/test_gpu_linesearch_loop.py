"""The SQP loop on the device SQP step with the activity given by the host
(_solve_impl_device_ls: the merit line search, the `step` criterion) against
the host-masked loop (_solve_impl_masked) on the same inputs: the iterates,
the ADMM state, the steps chosen and every per-iteration record, bit for bit,
with fixed iteration counts and with per-problem termination (tol_convergence
> 0, problems stopping at different iterations)."""
import copy

import pytest
import torch
from helpers import rel_err

from turbompc_amd.problems import configs
from turbompc_amd.problems.quadrotor import make_quadrotor_config
from turbompc_amd.solvers.turbompc_solver import DEFAULT_SOLVER_PARAMS, TurboMPCSolver

pytestmark = pytest.mark.gpu


def _params(n_sqp, admm_iters, tol, linesearch=True, criterion="first_order"):
    p = copy.deepcopy(DEFAULT_SOLVER_PARAMS)
    p["convergence_criterion"] = criterion
    p["num_sqp_iteration_max"] = n_sqp
    p["tol_convergence"] = tol
    p["admm"]["max_iter"] = admm_iters
    p["admm"]["adapt_rho_every"] = 0
    p["admm"]["relaxation_parameter"] = 1.0
    p["linesearch"] = linesearch
    return p


def _tol_splitting(prob, params):
    """A tolerance under which the problems stop at different SQP iterations:
    from the convergence errors recorded at tol 0 (problem b stops after the
    first iteration whose error is <= tol), the quantile of those errors that
    gives the most distinct stopping iterations."""
    p0 = copy.deepcopy(params)
    p0["tol_convergence"] = 0.0
    solver = TurboMPCSolver(prob, p0)
    errs = solver.solve(solver.initial_guess()).solver_stats.convergence_errors[:, :-1].double().cpu()
    best, best_n = None, 0
    for q in torch.linspace(0.05, 0.95, 19, dtype=torch.float64):
        tol = float(torch.quantile(errs.flatten(), q))
        below = errs <= tol
        first = torch.where(below.any(dim=1), below.to(torch.int8).argmax(dim=1), torch.full_like(below[:, 0], -1,
                            dtype=torch.long))
        n = len(set(first.tolist()))
        if n > best_n:
            best, best_n = tol, n
    return best


def _both(prob, params):
    out = []
    for loop in ("device", "masked"):
        solver = TurboMPCSolver(prob, params)
        solver._sqp_loop = loop
        out.append(solver.solve(solver.initial_guess()))
    torch.cuda.synchronize()
    return out


def _equal(x, y):
    """Bitwise equality, NaN where the other has NaN counting as equal."""
    if x is None or y is None:
        return x is None and y is None
    if not x.is_floating_point():
        return torch.equal(x, y)
    nx, ny = torch.isnan(x), torch.isnan(y)
    return torch.equal(nx, ny) and torch.equal(x[~nx], y[~ny])


def _assert_same(a, b):
    for k in ("states", "controls", "slack", "num_iter", "convergence_error", "admm_iters", "linesearch_alphas",
              "nonfinite"):
        assert _equal(getattr(a, k), getattr(b, k)), k
    for k in a.admm_state._fields:
        assert _equal(getattr(a.admm_state, k), getattr(b.admm_state, k)), k
    for k in a.solver_stats._fields:
        assert _equal(getattr(a.solver_stats, k), getattr(b.solver_stats, k)), k
    for k in a.kkt_state._fields:
        assert _equal(getattr(a.kkt_state, k), getattr(b.kkt_state, k)), k


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("stop", [False, True])
@pytest.mark.parametrize("mode", ["linesearch", "step", "step+linesearch"])
def test_quadrotor_device_loop_equals_masked(dtype, stop, mode):
    prob = make_quadrotor_config(B=24, seed=4, dtype=dtype, device="cuda")
    params = _params(8, 20, 0.0, linesearch="linesearch" in mode,
                     criterion="step" if mode.startswith("step") else "first_order")
    if stop:
        params["tol_convergence"] = _tol_splitting(prob, params)
    dev, msk = _both(prob, params)
    print(f"  tol {params['tol_convergence']:.3g}, SQP iterations per problem {dev.num_iter.tolist()}", flush=True)
    _assert_same(dev, msk)
    if stop:  # problems stop at different iterations
        assert len(set(dev.num_iter.tolist())) >= 2


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_first_order_device_loop_stops_on_the_recorded_errors(dtype):
    """The first-order device loop (the fused check of each SQP step, no line
    search) with problems stopping at different iterations: a stopped
    problem's convergence error is the check that stopped it, value for
    value (the loop re-evaluates that check at every later step on the same
    iterate, state and QP, and takes it without a masked merge).  Against
    the host-masked loop: the same iterates, stopping steps and ADMM counts
    bit for bit; the errors agree to rounding (the masked loop evaluates
    them with the separate check kernel, the device loop in the fused sweep)."""
    prob = make_quadrotor_config(B=24, seed=4, dtype=dtype, device="cuda")
    params = _params(8, 20, 0.0, linesearch=False, criterion="first_order")
    params["tol_convergence"] = _tol_splitting(prob, params)
    dev, msk = _both(prob, params)
    it = dev.num_iter.cpu()
    print(f"  tol {params['tol_convergence']:.3g}, SQP iterations per problem {it.tolist()}", flush=True)
    assert len(set(it.tolist())) >= 2
    hist = dev.solver_stats.convergence_errors.cpu()
    conv = dev.convergence_error.cpu()
    for b in range(it.shape[0]):
        assert hist[b, it[b] - 1] == conv[b], (b, int(it[b]), hist[b].tolist(), float(conv[b]))
    for k in ("states", "controls", "slack", "num_iter", "admm_iters", "nonfinite"):
        assert _equal(getattr(dev, k), getattr(msk, k)), k
    tol = 1e-12 if dtype == torch.float64 else 1e-5
    assert rel_err(dev.convergence_error, msk.convergence_error) < tol
    assert rel_err(dev.solver_stats.convergence_errors, msk.solver_stats.convergence_errors) < tol


@pytest.mark.parametrize("use_slack", [False, True])
@pytest.mark.parametrize("stop", [False, True])
@pytest.mark.parametrize("mode", ["linesearch", "step"])
def test_config4_device_loop_equals_masked(use_slack, stop, mode):
    prob = configs.config4(B=12, seed=1, use_slack_variables=use_slack, slack_penalization_weight=50.0).to("cuda")
    params = _params(8, 30, 0.0, linesearch=mode == "linesearch",
                     criterion="step" if mode == "step" else "first_order")
    if stop:
        params["tol_convergence"] = _tol_splitting(prob, params)
    dev, msk = _both(prob, params)
    print(f"  tol {params['tol_convergence']:.3g}, SQP iterations per problem {dev.num_iter.tolist()}", flush=True)
    _assert_same(dev, msk)
    if stop:
        assert len(set(dev.num_iter.tolist())) >= 2


@pytest.mark.parametrize("mode", ["linesearch", "step"])
def test_warm_started_device_loop_equals_masked(mode):
    """A second solve from the first one's solution (its ADMM state carried):
    the caller's state is read, not updated, by the device loop."""
    prob = make_quadrotor_config(B=16, seed=6, dtype=torch.float64, device="cuda")
    params = _params(4, 20, 0.0, linesearch=mode == "linesearch",
                     criterion="step" if mode == "step" else "first_order")
    first = TurboMPCSolver(prob, params).solve(TurboMPCSolver(prob, params).initial_guess())
    keep = [t.clone() for t in first.admm_state]
    out = []
    for loop in ("device", "masked"):
        solver = TurboMPCSolver(prob, params)
        solver._sqp_loop = loop
        out.append(solver.solve(first))
    torch.cuda.synchronize()
    _assert_same(*out)
    for a, b in zip(first.admm_state, keep):
        assert torch.equal(a, b)


@pytest.mark.parametrize("mode", ["linesearch", "step"])
def test_device_loop_equals_masked_with_a_nonfinite_problem(mode):
    """One problem's control weight is infinite, so its QP solution (and its
    ADMM state) is non-finite: the device loop takes the activity as given
    (no fused check decides it), so it runs that problem exactly when the
    masked loop does, and every other problem is untouched."""
    prob = configs.config4(B=8, seed=2).to("cuda")
    wu = prob.wu.clone()
    wu[3, 1] = float("inf")
    prob = prob.with_weights({"weights_penalization_control_squared": wu})
    params = _params(5, 30, 0.0, linesearch=mode == "linesearch",
                     criterion="step" if mode == "step" else "first_order")
    dev, msk = _both(prob, params)
    print(f"  SQP iterations per problem {dev.num_iter.tolist()}, non-finite {dev.nonfinite.tolist()}", flush=True)
    assert dev.nonfinite.tolist() == [b == 3 for b in range(8)]
    _assert_same(dev, msk)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("stop", [False, True])
def test_quadrotor_step_linearization_equals_build_qp(dtype, stop):
    """The quadrotor's SQP steps build their own dynamics rows
    (tmpc_sqp_admm_step_quadrotor_*: the linearization at the step's input
    iterate, written into the QP buffers and straight into the stage
    records): the solve is bit for bit the one whose loop builds each QP
    with build_qp and lets the step copy the rows into the records."""
    prob = make_quadrotor_config(B=24, seed=7, dtype=dtype, device="cuda")
    params = _params(6, 20, 0.0, linesearch=False, criterion="first_order")
    if stop:
        params["tol_convergence"] = _tol_splitting(prob, params)
    out = []
    for fused in (True, False):
        p = copy.copy(prob)
        if not fused:
            p.step_linearization = lambda: None  # noqa: E731  the build_qp path
        assert (p.step_linearization() is not None) == fused
        solver = TurboMPCSolver(p, params)
        out.append(solver.solve(solver.initial_guess()))
    torch.cuda.synchronize()
    _assert_same(*out)
    if stop:
        assert len(set(out[0].num_iter.tolist())) >= 2


def _planar_obstacles(B, seed):
    """A planar double integrator (nx = 4, nu = 2) among three discs: n = 6
    with 4 + 2 + 3 stacked rows, so the streaming records are 9 wide (padded)."""
    from turbompc_amd.problems.obstacle import ObstacleOCP

    g = torch.Generator().manual_seed(seed)
    u = lambda lo, hi, *s: lo + (hi - lo) * torch.rand(s, generator=g, dtype=torch.float64)  # noqa: E731
    dt, N, nx, nu, K = 0.1, 20, 4, 2, 3
    A = torch.tensor([[1.0, 0, dt, 0], [0, 1.0, 0, dt], [0, 0, 1.0, 0], [0, 0, 0, 1.0]], dtype=torch.float64)
    Bm = torch.tensor([[0.5 * dt * dt, 0], [0, 0.5 * dt * dt], [dt, 0], [0, dt]], dtype=torch.float64)
    x0 = torch.cat([torch.stack([torch.full((B,), -3.0, dtype=torch.float64), u(-1, 1, B)], 1),
                    torch.zeros(B, 2, dtype=torch.float64)], 1)
    xg = torch.cat([torch.stack([torch.full((B,), 3.0, dtype=torch.float64), u(-1, 1, B)], 1),
                    torch.zeros(B, 2, dtype=torch.float64)], 1)
    return ObstacleOCP(
        A=A, Bm=Bm, horizon=N, num_states=nx, num_controls=nu, initial_state=x0,
        weights_state=torch.tensor([1.0, 1.0, 0.1, 0.1], dtype=torch.float64).expand(B, nx),
        weights_control=torch.full((B, nu), 0.01, dtype=torch.float64),
        weights_final=torch.tensor([10.0, 10.0, 1.0, 1.0], dtype=torch.float64).expand(B, nx),
        reference_state=xg[:, None].expand(B, N + 1, nx),
        control_bounds=(torch.full((nu,), -2.0, dtype=torch.float64), torch.full((nu,), 2.0, dtype=torch.float64)),
        initial_guess_final_state=xg, obstacles_centers=u(-1.5, 1.5, B, K, 2), obstacles_radii=u(0.2, 0.5, B, K),
        obstacles_dimension=2)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_obstacle_step_on_padded_records_equals_build_qp(dtype):
    """The obstacle SQP step where the stage records are wider than the QP
    (n = 6 padded to 9): the step writes the obstacle rows into the QP only
    and the library copies G, l, u into the records; the solve equals the
    build_qp loop's bit for bit."""
    prob = _planar_obstacles(16, 3).to("cuda", dtype)
    params = _params(5, 15, 0.0, linesearch=False, criterion="first_order")
    out = []
    for fused in (True, False):
        p = copy.copy(prob)
        if not fused:
            p.step_linearization = lambda: None  # noqa: E731  the build_qp path
        solver = TurboMPCSolver(p, params)
        out.append(solver.solve(solver.initial_guess()))
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out[0].states).all())
    _assert_same(*out)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("stop", [False, True])
@pytest.mark.parametrize("slack", [False, True])
def test_obstacle_step_linearization_equals_build_qp(dtype, stop, slack):
    """Config 4's SQP steps build their own obstacle rows
    (tmpc_sqp_admm_step_obstacle_*: the linearization at the step's input
    iterate, written into the QP's G, l, u and straight into the stage
    records, the box rows and the dynamics records kept): the solve is bit
    for bit the one whose loop builds each QP with build_qp and lets the step
    copy G, l, u into the records (TMPC_FLAG_WARM_INEQ)."""
    prob = configs.config4(B=24, seed=8, use_slack_variables=slack, slack_penalization_weight=50.0).to(
        "cuda", dtype)
    params = _params(6, 15, 0.0, linesearch=False, criterion="first_order")
    if stop:
        params["tol_convergence"] = _tol_splitting(prob, params)
    out = []
    for fused in (True, False):
        p = copy.copy(prob)
        if not fused:
            p.step_linearization = lambda: None  # noqa: E731  the build_qp path
        assert (p.step_linearization() is not None) == fused
        solver = TurboMPCSolver(p, params)
        out.append(solver.solve(solver.initial_guess()))
    torch.cuda.synchronize()
    _assert_same(*out)
    if stop:
        assert len(set(out[0].num_iter.tolist())) >= 2
