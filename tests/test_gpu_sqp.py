"""GPU SQP (TurboMPCSolver, admm_hip_direct) against the CPU SQP restatement
(oracle/sqp_cpu.py) on the quadrotor workload of the benchmark (config 3
shapes, small batch): 5 SQP iterations x 20 ADMM iterations, fixed counts.
"""
import copy

import numpy as np
import pytest
import torch

import oracle
from helpers import TOL, rel_err
from oracle.sqp_cpu import quadrotor_sqp
from turbompc_amd.problems.quadrotor import make_quadrotor_config
from turbompc_amd.solvers.turbompc_solver import DEFAULT_SOLVER_PARAMS, TurboMPCSolver

pytestmark = pytest.mark.gpu


def _params(n_sqp, admm_iters):
    p = copy.deepcopy(DEFAULT_SOLVER_PARAMS)
    p["num_sqp_iteration_max"] = n_sqp
    p["tol_convergence"] = 0.0
    p["admm"]["max_iter"] = admm_iters
    p["admm"]["adapt_rho_every"] = 0
    p["admm"]["relaxation_parameter"] = 1.0
    return p


def _cpu_sqp(B, seed, n_sqp, admm_iters, dtype):
    prob = make_quadrotor_config(B=B, seed=seed, dtype=torch.float64, device="cpu")
    D, E, q = (t.numpy() for t in prob.cost_blocks())
    A0, c0 = (t.numpy() for t in prob.initial_equality())
    G, l, u = (t.numpy() for t in prob.inequality_blocks())
    static = dict(D=D, E=E, q=q, A0=A0, c0=c0, A_plus=prob.a_plus().numpy(), G=G, l=l, u=u)
    xg, ug = (t.numpy() for t in prob.initial_guess())
    cfg = oracle.OracleCfg(max_iter=admm_iters, check_every=25, adapt_rho_every=0, sigma=1e-6, eps_abs=1e-9,
                           eps_rel=1e-9, rho_f_factor=1000.0, alpha=1.0)
    return quadrotor_sqp(static, xg, ug, dt=prob.dt, params=prob.params, cfg=cfg, rho0=0.1, n_sqp=n_sqp, dtype=dtype)


@pytest.mark.parametrize("n_sqp", [1, 5])
def test_quadrotor_sqp_fp64_matches_cpu(n_sqp):
    B = 8
    xs, us, st = _cpu_sqp(B, 0, n_sqp, 20, np.float64)
    prob = make_quadrotor_config(B=B, seed=0, dtype=torch.float64, device="cuda")
    solver = TurboMPCSolver(prob, _params(n_sqp, 20))
    sol = solver.solve(solver.initial_guess())
    torch.cuda.synchronize()
    assert rel_err(sol.states, xs) < TOL[torch.float64]
    assert rel_err(sol.controls, us) < TOL[torch.float64]
    assert rel_err(sol.admm_state.y_f_dyn, st.y_f_dyn) < 1e-8
    assert torch.all(sol.num_iter == n_sqp)
    assert torch.all(sol.admm_iters[:, :n_sqp] == 20)


def test_quadrotor_sqp_fp32_matches_cpu():
    B = 16
    xs, us, _ = _cpu_sqp(B, 1, 5, 20, np.float64)
    prob = make_quadrotor_config(B=B, seed=1, dtype=torch.float32, device="cuda")
    solver = TurboMPCSolver(prob, _params(5, 20))
    sol = solver.solve(solver.initial_guess())
    torch.cuda.synchronize()
    for name, got, ref in (("states", sol.states, xs), ("controls", sol.controls, us)):
        e = rel_err(got, ref)
        print(f"quadrotor SQP fp32 {name}: rel err vs fp64 CPU SQP {e:.2e}")
        assert e < TOL[torch.float32], (name, e)


def test_sqp_stops_per_problem_on_tolerance():
    # with a finite tolerance each problem stops on its own first-order error
    B = 6
    prob = make_quadrotor_config(B=B, seed=2, dtype=torch.float64, device="cuda")
    p = _params(8, 20)
    p["tol_convergence"] = 5e-2
    solver = TurboMPCSolver(prob, p)
    sol = solver.solve(solver.initial_guess())
    it = sol.num_iter.cpu().numpy()
    conv = sol.convergence_error.cpu().numpy()
    assert np.all(it >= 1) and np.all(it <= 8)
    # stopped problems satisfy the tolerance; problems at the cap may not
    assert np.all((conv <= 5e-2) | (it == 8))
    hist = sol.solver_stats.convergence_errors.cpu().numpy()
    for b in range(B):
        assert hist[b, it[b] - 1] == pytest.approx(conv[b])


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_first_order_check_kernel_matches_torch(dtype):
    B = 12
    prob = make_quadrotor_config(B=B, seed=3, dtype=dtype, device="cuda")
    solver = TurboMPCSolver(prob, _params(2, 10))
    sol = solver.solve(solver.initial_guess())
    qp = prob.build_qp(sol.states, sol.controls)
    args = (qp, sol.states, sol.controls, sol.slack, sol.admm_state)
    ck, ek, ik, gk = solver._first_order_check(*args)
    ct, et, it_, gt = solver._first_order_check_torch(*args)
    tol = 1e-12 if dtype == torch.float64 else 1e-5
    for a, b in ((ck, ct), (ek, et), (ik, it_), (gk, gt)):
        assert rel_err(a, b) < tol


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_first_order_check_kernel_matches_torch_with_slack(dtype):
    """Soft obstacle rows: the slack-stationarity term |gamma xi + y_g| of the
    reference (turbompc_solver.py:1207-1212) in both checks.  The slack is
    shifted off the ADMM fixed point so that this term sets the error."""
    from turbompc_amd.problems import configs

    prob = configs.config4(B=6, seed=4, use_slack_variables=True, slack_penalization_weight=30.0).to("cuda", dtype)
    solver = TurboMPCSolver(prob, _params(2, 10))
    sol = solver.solve(solver.initial_guess())
    qp = prob.build_qp(sol.states, sol.controls)
    slack = sol.slack + 0.05
    args = (qp, sol.states, sol.controls, slack, sol.admm_state)
    ck, ek, ik, gk = solver._first_order_check(*args)
    ct, et, it_, gt = solver._first_order_check_torch(*args)
    tol = 1e-12 if dtype == torch.float64 else 1e-5
    for a, b in ((ck, ct), (ek, et), (ik, it_), (gk, gt)):
        assert rel_err(a, b) < tol
    # the slack term dominates the error here (30 * 0.05 = 1.5 on every row)
    assert bool(torch.all(ct >= 1.0))


@pytest.mark.parametrize("std", [False, True])
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("use_slack", [False, True])
@pytest.mark.parametrize("diag", [False, True])
def test_first_order_check_kernel_matches_dense_assembly(std, dtype, use_slack, diag):
    """The check on random QPs (general E / A_plus, or the explicit-integrator
    structure read with std_dynamics=True) against dense P, C, G products."""
    from helpers import dense_C, dense_G, dense_P, np_qp, random_qp
    from turbompc_amd.solvers.sqp_hip import first_order_check

    B, T, n, nx, m = 5, 7, 9, 6, 11
    qp = random_qp(B, T, n, nx, m, seed=11 + std, std=std, diag=diag)
    rng = np.random.default_rng(4)
    x, yg = rng.standard_normal((B, T, n)), rng.standard_normal((B, T, m))
    y0, yf = rng.standard_normal((B, nx)), rng.standard_normal((B, T - 1, nx))
    sl = rng.standard_normal((B, T, m)) * 0.3 if use_slack else None
    w = 2.5
    dev = lambda a: torch.tensor(a, dtype=dtype, device="cuda")  # noqa: E731
    conv, eq, iq, g = first_order_check(qp.to("cuda", dtype), dev(x), dev(y0), dev(yf), dev(yg),
                                        dev(sl) if use_slack else None, w, std_dynamics=std, diag_cost=diag)
    a = np_qp(qp)
    for b in range(B):
        P, C, Gd = dense_P(a["D"][b], a["E"][b]), dense_C(a["A0"][b], a["Am"][b], a["Ap"][b]), dense_G(a["G"][b])
        xv = x[b].ravel()
        y = np.concatenate([y0[b], yf[b].ravel()])
        stat = np.abs(P @ xv + a["q"][b].ravel() + C.T @ y + Gd.T @ yg[b].ravel()).max()
        e = np.abs(C @ xv - np.concatenate([a["c0"][b], a["c"][b].ravel()])).max()
        gv = Gd @ xv + (sl[b].ravel() if use_slack else 0.0)
        i = max(np.maximum(a["l"][b].ravel() - gv, 0).max(), np.maximum(gv - a["u"][b].ravel(), 0).max())
        s = np.abs(w * sl[b].ravel() + yg[b].ravel()).max() if use_slack else 0.0
        tol = 1e-12 if dtype == torch.float64 else 1e-5
        scale = max(stat, e, i, 1.0)
        assert abs(float(conv[b]) - max(stat, e, i, s)) <= tol * scale
        assert abs(float(eq[b]) - e) <= tol * scale
        assert abs(float(iq[b]) - i) <= tol * scale
        assert rel_err(g[b].reshape(-1), gv) < tol * 10


@pytest.mark.parametrize("std", [False, True])
@pytest.mark.parametrize("use_slack", [False, True])
def test_first_order_check_large_batch_equals_small_batches(std, use_slack):
    """A batch large enough that each wavefront of the check kernel walks
    several stages (B T >= 2 * 16384; here B = 1536, T = 23: two stages per
    wave, the last wave of each problem one) gives, problem for problem
    and bit for bit, the values of small batches (one stage per wave).  Each
    problem gets its own NaN or infinite entry in some rows, so the per-wave
    folding of the stage maxima must keep what the per-stage atomics kept."""
    from helpers import random_qp
    from turbompc_amd.solvers.qp_data import QPCostBlocks, QPData, QPEqualityBlocks, QPInequalityBlocks
    from turbompc_amd.solvers.sqp_hip import first_order_check

    B, T, n, nx, m = 1536, 23, 9, 6, 5
    dtype = torch.float32
    qp = random_qp(B, T, n, nx, m, seed=23, std=std, diag=True).to("cuda", dtype)
    gen = torch.Generator(device="cpu").manual_seed(5)
    rnd = lambda *s: torch.randn(s, generator=gen, dtype=dtype).to("cuda")  # noqa: E731
    x, yg, y0, yf = rnd(B, T, n), rnd(B, T, m), rnd(B, nx), rnd(B, T - 1, nx)
    sl = rnd(B, T, m) * 0.3 if use_slack else None
    x[7, 3, 2] = float("nan")
    x[100, 20, 0] = float("inf")
    yg[901, 0, 1] = float("nan")
    big = first_order_check(qp, x, y0, yf, yg, sl, 2.5, std_dynamics=std, diag_cost=True)

    def part(t, lo, hi):
        return t[lo:hi].contiguous()

    def sub(lo, hi):
        c, e, i = qp.cost, qp.eq, qp.ineq
        q = QPData(cost=QPCostBlocks(part(c.D, lo, hi), part(c.E, lo, hi), part(c.q, lo, hi)),
                   eq=QPEqualityBlocks(part(e.A0, lo, hi), part(e.A_minus, lo, hi), part(e.A_plus, lo, hi),
                                       part(e.c0, lo, hi), part(e.c, lo, hi)),
                   ineq=QPInequalityBlocks(part(i.G, lo, hi), part(i.l, lo, hi), part(i.u, lo, hi),
                                           i.slack_penalization_weight, i.use_slack_variables))
        return first_order_check(q, part(x, lo, hi), part(y0, lo, hi), part(yf, lo, hi), part(yg, lo, hi),
                                 part(sl, lo, hi) if use_slack else None, 2.5, std_dynamics=std, diag_cost=True)

    for lo in range(0, B, 256):
        small = sub(lo, lo + 256)
        for a, b in zip(big, small):
            a, b = a[lo:lo + 256], b
            nan_a, nan_b = torch.isnan(a), torch.isnan(b)
            assert torch.equal(nan_a, nan_b) and torch.equal(a[~nan_a], b[~nan_b]), lo


def _random_state(qp, rng, dtype, use_slack):
    from turbompc_amd.solvers.admm.admm import ADMMState

    B, T, n, nx, n0, m = qp.dims
    dev = lambda a: torch.tensor(a, dtype=dtype, device="cuda")  # noqa: E731
    l, u = qp.ineq.l.numpy(), qp.ineq.u.numpy()
    return ADMMState(
        x_blocks=dev(rng.standard_normal((B, T, n))), y_g=dev(rng.standard_normal((B, T, m))),
        y_f_0=dev(rng.standard_normal((B, n0))), y_f_dyn=dev(rng.standard_normal((B, T - 1, nx))),
        z_g=dev(np.clip(rng.standard_normal((B, T, m)), l, u)),
        xi_g=dev(rng.standard_normal((B, T, m)) * 0.3 if use_slack else np.zeros((B, T, m))),
        rho_bar=dev(np.full(B, 0.1)))


# kernel: the check fused into the streaming kernel (explicit-integrator
# structure, P problems per wavefront) or the generic path (check kernel, then
# the activity test, then the generic ADMM kernel)
@pytest.mark.parametrize("kernel", ["stream-1", "stream-2", "stream-3", "generic-std", "generic"])
@pytest.mark.parametrize("use_slack", [False, True])
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_sqp_step_check_and_activity(kernel, use_slack, dtype):
    """tmpc_sqp_admm_step: the first-order check of the input iterate matches
    tmpc_sqp_first_order_*, the activity test is active & (conv > tol), stopped
    problems keep their state with zero iterations, and the others match a
    plain ADMM solve from the same state."""
    from helpers import random_qp, soften
    from turbompc_amd import _lib
    from turbompc_amd.solvers.admm.admm import ADMMSolver
    from turbompc_amd.solvers.linear_systems_solvers.backends import AdmmBackend
    from turbompc_amd.solvers.qp_utils import ZShape
    from turbompc_amd.solvers.sqp_hip import first_order_check

    std = kernel != "generic"
    B, T, n, nx, m = (13, 21, 6, 4, 2) if kernel.startswith("stream") else (7, 9, 9, 6, 11)
    if kernel == "stream-2":
        B, T, n, nx, m = 9, 11, 17, 13, 4
    qp = random_qp(B, T, n, nx, m, seed=71, std=std, diag=std)
    if use_slack:
        qp = soften(qp, 3.0, shrink=0.5)
    rng = np.random.default_rng(9)
    st = _random_state(qp, rng, dtype, use_slack)
    qpd = qp.to("cuda", dtype)
    flags = _lib.flag_stream_p(int(kernel[-1])) if kernel.startswith("stream") else _lib.FLAG_GENERIC_KERNEL
    solver = ADMMSolver(ZShape(T - 1, nx, n - nx), {"max_iter": 50, "tol_epsilon": 1e-8}, sigma=1e-6, max_iter=15,
                        eps_abs=1e-12, eps_rel=1e-12, check_termination_every=25, adapt_rho_every=0,
                        rho_f_factor=1000.0, admm_backend=AdmmBackend.HIP_DIRECT, use_slack=use_slack,
                        std_dynamics=std, kernel_flags=flags, diag_cost=std)
    sw = qpd.ineq.slack_penalization_weight
    x = st.x_blocks
    ref = first_order_check(qpd, x, st.y_f_0, st.y_f_dyn, st.y_g, st.xi_g if use_slack else None, float(sw),
                            std_dynamics=std, diag_cost=std)
    tol = float(ref[0].median())
    active = torch.tensor(rng.random(B) < 0.7, device="cuda")
    (_, _), stats, out, (cv, e, i, g), act = solver.sqp_step(qpd, st, active, tol, slack_weight=sw)
    (_, _), stats_p, out_p = solver.solve(qpd, st, slack_weight=sw)
    torch.cuda.synchronize()
    bar = 1e-12 if dtype == torch.float64 else 1e-5
    for got, want in zip((cv, e, i, g), ref):
        assert rel_err(got, want) < bar, rel_err(got, want)
    want_act = active & (ref[0] > tol)
    assert torch.equal(act, want_act)
    assert 0 < int(want_act.sum()) < B
    on = want_act.cpu().numpy()
    assert np.all(stats.num_iter.cpu().numpy()[~on] == 0)
    assert np.all(stats.num_iter.cpu().numpy()[on] == stats_p.num_iter.cpu().numpy()[on])
    for k in ("x_blocks", "z_g", "y_g", "y_f_0", "y_f_dyn", "xi_g", "rho_bar"):
        a, b0, p = getattr(out, k).cpu().numpy(), getattr(st, k).cpu().numpy(), getattr(out_p, k).cpu().numpy()
        np.testing.assert_array_equal(a[~on], b0[~on])
        np.testing.assert_array_equal(a[on], p[on])


@pytest.mark.parametrize("case", ["quadrotor", "config4", "config4-slack", "config4-built", "config4-built-slack"])
def test_sqp_warm_records_match_repacking(case):
    """FLAG_WARM_RECORDS: an SQP solve whose steps rewrite only the records
    that changed gives the same iterates, bit for bit, as one that repacks
    every record at every step.  The quadrotor's and config 4's steps write
    their relinearized rows (A_minus and c; the obstacle rows of G, l, u) into
    the records themselves and keep the rest (config 4's dynamics records with
    FLAG_WARM_SAME_DYNAMICS); "built": config 4 with each QP from build_qp,
    whose obstacle rows the step copies in (FLAG_WARM_INEQ)."""
    import turbompc_amd.solvers.turbompc_solver as ts
    from turbompc_amd.problems import configs

    B = 24
    if case == "quadrotor":
        prob, level, n_sqp, iters = make_quadrotor_config(B=B, seed=6, dtype=torch.float32, device="cuda"), \
            "dynamics", 4, 12
    else:
        prob = configs.config4(B=B, seed=6, use_slack_variables=case.endswith("slack"),
                               slack_penalization_weight=50.0).to("cuda", torch.float32)
        level, n_sqp, iters = "dynamics", 5, 15
        if "built" in case:
            prob.step_linearization = lambda: None  # noqa: E731
            level = "constraints"
    solver = TurboMPCSolver(prob, _params(n_sqp, iters))
    seen = []
    orig = ts._warm_level
    try:
        ts._warm_level = lambda qp, prev: seen.append(orig(qp, prev)) or seen[-1]
        warm = solver.solve(solver.initial_guess())
        ts._warm_level = lambda qp, prev: None
        cold = solver.solve(solver.initial_guess())
    finally:
        ts._warm_level = orig
    torch.cuda.synchronize()
    assert seen and all(v == level for v in seen), seen
    assert torch.equal(warm.states, cold.states) and torch.equal(warm.controls, cold.controls)
    assert torch.equal(warm.admm_state.y_f_dyn, cold.admm_state.y_f_dyn)
    assert torch.equal(warm.admm_state.y_g, cold.admm_state.y_g)
    assert torch.equal(warm.slack, cold.slack)
    assert torch.equal(warm.convergence_error, cold.convergence_error)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("with_dual", [True, False])
def test_kkt_active_sets_kernel_matches_torch(dtype, with_dual):
    """tmpc_kkt_active_sets_* against the elementwise torch form of
    identify_active_inequalities + the dual-sign rule (turbompc_solver.py:269-292,
    :1387-1439), value for value: rows drawn around the tolerance boundary on
    both sides (a contracted eps_abs + eps_rel |bound| would flip some of
    them), infinite and NaN bounds and values, duals at and around +-dual_tol."""
    from turbompc_amd.solvers.sqp_hip import kkt_active_sets
    from turbompc_amd.solvers.turbompc_solver import active_sets_torch

    gen = torch.Generator().manual_seed(7)
    B, T, m = 64, 21, 8
    ea, er, dtol = 1e-3, 1e-3, 1e-3
    l = -torch.rand((B, T, m), generator=gen, dtype=torch.float64) * 4.0
    u = torch.rand((B, T, m), generator=gen, dtype=torch.float64) * 4.0
    l, u = l.to(dtype), u.to(dtype)
    tol_l = ea + er * l.abs()
    tol_u = ea + er * u.abs()
    side = torch.rand((B, T, m), generator=gen) < 0.5
    spread = 2e-6 if dtype == torch.float32 else 4e-15  # a few dozen ulps of the tolerance
    jitter = (1.0 + (torch.rand((B, T, m), generator=gen, dtype=torch.float64) - 0.5) * spread).to(dtype)
    g = torch.where(side, l + tol_l * jitter, u - tol_u * jitter)  # within a few ulps of the boundary
    far = torch.rand((B, T, m), generator=gen) < 0.3
    g = torch.where(far, (l + u) / 2, g)
    # special rows: infinite bounds, NaN values and bounds, exact bounds, signed zeros
    g[0, 0, :] = torch.tensor([0.0, float("nan"), 1.0, -0.0, 2.0, float("inf"), -1.0, 0.5], dtype=dtype)
    l[0, 0, :] = torch.tensor([-float("inf"), -1.0, 1.0, 0.0, float("nan"), 0.0, -float("inf"), 0.5], dtype=dtype)
    u[0, 0, :] = torch.tensor([float("inf"), 1.0, 2.0, 0.0, 3.0, float("inf"), 0.0, float("inf")], dtype=dtype)
    y = None
    if with_dual:
        y = (torch.randn((B, T, m), generator=gen, dtype=torch.float64) * 2e-3).to(dtype)
        d = torch.tensor(dtol, dtype=dtype)
        y[1, 0, :] = torch.stack([d, -d, torch.nextafter(d, d * 2), -torch.nextafter(d, d * 2),
                                  torch.nextafter(d, d * 0), torch.tensor(0.0, dtype=dtype),
                                  torch.tensor(float("nan"), dtype=dtype), torch.tensor(-0.0, dtype=dtype)])
    gd, ld, ud = (t.to("cuda") for t in (g, l, u))
    yd = y.to("cuda") if y is not None else None
    lo, up = kkt_active_sets(gd, ld, ud, yd, ea, er, dtol)
    lo_t, up_t = active_sets_torch(gd, ld, ud, yd, ea, er, dtol)
    torch.cuda.synchronize()
    assert lo.dtype == torch.bool and lo.shape == g.shape
    assert torch.equal(lo, lo_t) and torch.equal(up, up_t)
    # the CPU evaluation of the same torch form agrees too
    lo_c, up_c = active_sets_torch(g, l, u, y, ea, er, dtol)
    assert torch.equal(lo.cpu(), lo_c) and torch.equal(up.cpu(), up_c)
    # the boundary draws exercise both outcomes
    n_lo, n_up = int(lo.sum()), int(up.sum())
    print(f"{dtype} dual={with_dual}: {n_lo} lower, {n_up} upper of {g.numel()}")
    assert 0 < n_lo < g.numel() and 0 < n_up < g.numel()
