"""SQP with the merit line search (linesearch=True, turbompc/solvers/linesearch.py:54-178)
on the GPU against the CPU restatement (oracle/sqp_cpu.py merit_linesearch) at
fixed iteration counts: the quadrotor (config 3 shapes) and the obstacle
workload (config 4 shapes) with hard and soft constraints.  The step chosen
for every problem and SQP iteration must be the same; the iterates agree to
the fp64 tolerance.  Also the quadrotor's RK4 step kernel
(tmpc_quadrotor_dynamics_*), which the equality residuals of the merit use,
against the CPU RK4."""
import copy

import numpy as np
import pytest
import torch

import oracle
from helpers import TOL, rel_err
from oracle.sqp_cpu import obstacle_sqp, quadrotor_sqp
from turbompc_amd.problems import configs
from turbompc_amd.problems.ocp import LinearOCP
from turbompc_amd.problems.quadrotor import hover_thrust, make_quadrotor_config
from turbompc_amd.solvers.turbompc_solver import DEFAULT_SOLVER_PARAMS, TurboMPCSolver

pytestmark = pytest.mark.gpu


def _params(n_sqp, admm_iters):
    p = copy.deepcopy(DEFAULT_SOLVER_PARAMS)
    p["num_sqp_iteration_max"] = n_sqp
    p["tol_convergence"] = 0.0
    p["admm"]["max_iter"] = admm_iters
    p["admm"]["adapt_rho_every"] = 0
    p["admm"]["relaxation_parameter"] = 1.0
    p["linesearch"] = True
    return p


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_quadrotor_dynamics_kernel_matches_cpu(dtype):
    B = 9
    prob = make_quadrotor_config(B=B, seed=2, dtype=torch.float64, device="cpu")
    rng = np.random.default_rng(3)
    T = prob.horizon + 1
    s = rng.standard_normal((B, T, 13))
    s[..., 3:7] /= np.linalg.norm(s[..., 3:7], axis=-1, keepdims=True)
    u = rng.uniform(0.0, 4.0, (B, T, 4))
    dev = make_quadrotor_config(B=B, seed=2, dtype=dtype, device="cuda")
    got = dev.next_states(torch.tensor(s, dtype=dtype, device="cuda"), torch.tensor(u, dtype=dtype, device="cuda"))
    torch.cuda.synchronize()
    c = lambda a: torch.tensor(a, dtype=dtype).double().numpy()  # noqa: E731
    xu = np.concatenate([c(s)[:, :-1], c(u)[:, :-1]], axis=-1).reshape(-1, 17)
    f, _ = oracle.quadrotor_rk4_jac(xu, float(prob.dt), prob.params)
    assert got.shape == (B, T - 1, 13)
    assert rel_err(got, f.reshape(B, T - 1, 13)) < (1e-13 if dtype == torch.float64 else 2e-6)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_linear_dynamics_kernel_matches_cpu(dtype):
    prob = configs.config4(B=7, seed=3)  # double integrator, nx = 6, nu = 3, per-problem A, B, b
    g = torch.Generator().manual_seed(5)
    s = torch.randn((7, prob.horizon + 1, 6), generator=g, dtype=torch.float64)
    u = torch.randn((7, prob.horizon + 1, 3), generator=g, dtype=torch.float64)
    prob.b = torch.randn(prob.b.shape, generator=g, dtype=torch.float64)
    ref = prob.next_states(s, u)  # the CPU path (einsum in fp64)
    dev = prob.to("cuda", dtype)
    got = dev.next_states(s.to("cuda", dtype), u.to("cuda", dtype))
    torch.cuda.synchronize()
    assert got.shape == ref.shape
    assert rel_err(got, ref.numpy()) < (1e-14 if dtype == torch.float64 else 1e-6)


def test_quadrotor_sqp_linesearch_fp64_matches_cpu():
    B, n_sqp, admm_iters = 8, 6, 20
    cpu = make_quadrotor_config(B=B, seed=0, dtype=torch.float64, device="cpu")
    D, E, q = (t.numpy() for t in cpu.cost_blocks())
    A0, c0 = (t.numpy() for t in cpu.initial_equality())
    G, l, u = (t.numpy() for t in cpu.inequality_blocks())
    static = dict(D=D, E=E, q=q, A0=A0, c0=c0, A_plus=cpu.a_plus().numpy(), G=G, l=l, u=u)
    xg, ug = (t.numpy() for t in cpu.initial_guess())
    cfg = oracle.OracleCfg(max_iter=admm_iters, check_every=25, adapt_rho_every=0, sigma=1e-6, eps_abs=1e-9,
                           eps_rel=1e-9, rho_f_factor=1000.0, alpha=1.0)
    xs, us, st, _, alphas = quadrotor_sqp(static, xg, ug, dt=cpu.dt, params=cpu.params, cfg=cfg, rho0=0.1,
                                          n_sqp=n_sqp, linesearch={})
    print(f"  CPU steps {alphas.tolist()}", flush=True)
    prob = make_quadrotor_config(B=B, seed=0, dtype=torch.float64, device="cuda")
    solver = TurboMPCSolver(prob, _params(n_sqp, admm_iters))
    sol = solver.solve(solver.initial_guess())
    torch.cuda.synchronize()
    np.testing.assert_array_equal(sol.linesearch_alphas.cpu().numpy(), alphas)
    assert rel_err(sol.states, xs) < TOL[torch.float64]
    assert rel_err(sol.controls, us) < TOL[torch.float64]
    assert rel_err(sol.admm_state.y_f_dyn, st.y_f_dyn) < 1e-8
    assert torch.all(sol.num_iter == n_sqp)
    assert len(set(alphas.ravel().tolist())) >= 2


@pytest.mark.parametrize("use_slack", [False, True])
def test_config4_sqp_linesearch_fp64_matches_cpu(use_slack):
    B, n_sqp, admm_iters, gamma = 6, 8, 30, 50.0
    prob = configs.config4(B=B, seed=0, use_slack_variables=use_slack, slack_penalization_weight=gamma)
    D, E, q = (t.numpy() for t in prob.cost_blocks())
    A0, c0 = (t.numpy() for t in prob.initial_equality())
    G, l, u = (t.numpy() for t in LinearOCP.inequality_blocks(prob))
    static = dict(D=D, E=E, q=q, A0=A0, c0=c0, A_plus=prob.a_plus().numpy(), G=G, l=l, u=u)
    xg, ug = (t.numpy() for t in prob.initial_guess())
    Am, c = (t.numpy() for t in prob.dynamics_blocks(*prob.initial_guess()))
    cfg = oracle.OracleCfg(max_iter=admm_iters, check_every=50, adapt_rho_every=0, sigma=1e-6, eps_abs=1e-9,
                           eps_rel=1e-9, rho_f_factor=1000.0, alpha=1.0)
    xs, us, st, sl, alphas = obstacle_sqp(static, xg, ug, A_minus=Am, c=c, centers=prob.centers.numpy(),
                                          radii=prob.radii.numpy(), dim=3, cfg=cfg, rho0=0.1, n_sqp=n_sqp,
                                          slack_weight=gamma, use_slack=use_slack, linesearch={})
    print(f"  CPU steps {alphas.tolist()}", flush=True)
    solver = TurboMPCSolver(prob.to("cuda"), _params(n_sqp, admm_iters))
    sol = solver.solve(solver.initial_guess())
    torch.cuda.synchronize()
    np.testing.assert_array_equal(sol.linesearch_alphas.cpu().numpy(), alphas)
    assert rel_err(sol.states, xs) < TOL[torch.float64]
    assert rel_err(sol.controls, us) < TOL[torch.float64]
    assert rel_err(sol.admm_state.y_g, st.y_g) < 1e-8
    # the returned slack is the ADMM state's (turbompc_solver.py:1747-1751)
    assert rel_err(sol.slack, st.xi_g) < 1e-8
    assert len(set(alphas.ravel().tolist())) >= 3


def _torch_terms(prob, s, c, sl, ds, dc, dsl):
    from turbompc_amd.solvers.linesearch import evaluate_constraints_with_bounds

    eq, iq, *_ = evaluate_constraints_with_bounds(prob, s, c, sl)
    dcost = prob.cost_directional_derivative(s, c, sl, ds, dc, dsl) if ds is not None else None
    return prob.cost(s, c, sl), eq, iq, dcost


def _merit_cases(dtype):
    """(name, problem): the quadrotor plain and with rescaling and the
    initial-control rows; config 1 (linear dynamics) with soft box rows."""
    hov = hover_thrust()
    lim = dict(rescale_optimization_variables=True,
               state_rescaling_min=torch.tensor([-5.0] * 3 + [-1.0] * 4 + [-3.0] * 3 + [-4.0] * 3, dtype=dtype),
               state_rescaling_max=torch.tensor([5.0] * 3 + [1.0] * 4 + [3.0] * 3 + [4.0] * 3, dtype=dtype),
               control_rescaling_min=torch.zeros(4, dtype=dtype),
               control_rescaling_max=torch.full((4,), 2.0 * hov, dtype=dtype))
    yield "quadrotor", make_quadrotor_config(B=6, seed=3, dtype=dtype, device="cuda")
    yield "quadrotor rescaled, u0 rows", make_quadrotor_config(
        B=6, seed=4, dtype=dtype, device="cuda", constrain_initial_control=True,
        initial_control=torch.full((6, 4), hov, dtype=dtype), **lim)
    yield "config 1 soft", configs.config1(B=6, seed=2, use_slack_variables=True,
                                           slack_penalization_weight=30.0).to("cuda", dtype)
    yield "config 4 (obstacle rows)", configs.config4(B=6, seed=1).to("cuda", dtype)
    lim4 = dict(rescale_optimization_variables=True,
                state_rescaling_min=torch.tensor([-4.0] * 3 + [-2.0] * 3, dtype=torch.float64),
                state_rescaling_max=torch.tensor([4.0, 5.0, 3.0] + [2.0] * 3, dtype=torch.float64),
                control_rescaling_min=torch.full((3,), -3.0, dtype=torch.float64),
                control_rescaling_max=torch.full((3,), 3.0, dtype=torch.float64))
    yield "config 4 soft rescaled", configs.config4(B=6, seed=2, use_slack_variables=True,
                                                    slack_penalization_weight=50.0, **lim4).to("cuda", dtype)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_fused_merit_terms_match_torch_forms(dtype):
    """QuadraticTrackingOCP.merit_terms (tmpc_ocp_merit_terms_*, one kernel)
    against cost, cost_directional_derivative and evaluate_constraints_with_bounds
    (linesearch.py:14-52): the same terms up to the order of the sums, for one
    batch and for four stacked copies (the line search's candidates); a NaN in
    an iterate reaches every term it enters; problems with other inequality
    rows than the fused form knows have none."""
    tol = 1e-12 if dtype == torch.float64 else 2e-5
    for name, prob in _merit_cases(dtype):
        gen = torch.Generator().manual_seed(5)
        s0, c0 = prob.initial_guess()
        B, T = s0.shape[:2]
        rnd = lambda shape, k: (k * torch.randn(shape, generator=gen, dtype=torch.float64)).to("cuda", dtype)  # noqa: E731
        s, c = s0 + rnd(s0.shape, 0.3), c0 + rnd(c0.shape, 0.5)
        m = prob.num_inequality_constraints
        sl = rnd((B, T, m), 0.2) if prob.use_slack_variables else torch.zeros((B, T, m), dtype=dtype, device="cuda")
        ds, dc, dsl = rnd(s.shape, 0.1), rnd(c.shape, 0.1), rnd((B, T, m), 0.1)
        got = prob.merit_terms(s, c, sl, ds, dc, dsl)
        want = _torch_terms(prob, s, c, sl, ds, dc, dsl)
        torch.cuda.synchronize()
        for k, g, w in zip(("cost", "eq", "iq", "dcost"), got, want):
            e = rel_err(g, w)
            print(f"{name} {dtype}: {k} rel err {e:.1e}", flush=True)
            assert g.shape == (B,) and e < tol, (name, k, e)
        assert float(want[2].abs().sum()) > 0  # some box row is violated, so iq is exercised
        # four stacked copies, as the line search's candidates
        A = 4
        a = torch.tensor([0.1, 0.3, 0.7, 1.0], dtype=dtype, device="cuda").view(A, 1, 1, 1)
        s4, c4, sl4 = ((z[None] + a * d[None]).flatten(0, 1) for z, d in ((s, ds), (c, dc), (sl, dsl)))
        got4 = prob.merit_terms(s4, c4, sl4, copies=A)
        want4 = _torch_terms(prob.tile(A), s4, c4, sl4, None, None, None)
        for k, g, w in zip(("cost", "eq", "iq"), got4[:3], want4[:3]):
            assert g.shape == (A * B,) and rel_err(g, w) < tol, (name, "copies", k)
        assert got4[3] is None
        if prob._merit_linear_dynamics() is not None:
            # the linear step formed in the kernel equals the one read from
            # next_states (tmpc_linear_dynamics_*), bit for bit
            ref = copy.copy(prob)
            ref._merit_linear_dynamics = lambda: None  # noqa: E731
            for g, r in zip(got4, ref.merit_terms(s4, c4, sl4, copies=A)):
                assert (g is None and r is None) or torch.equal(g, r), (name, "linear step")
    # NaN propagation: one problem's state
    prob = make_quadrotor_config(B=4, seed=1, dtype=dtype, device="cuda")
    s, c = prob.initial_guess()
    s = s.clone()
    s[2, 5, 1] = float("nan")
    cost, eq, iq, _ = prob.merit_terms(s, c, None)
    assert torch.isnan(cost[2]) and torch.isnan(eq[2]) and torch.isfinite(cost[[0, 1, 3]]).all()
    # no fused form for a problem that defines its inequality rows otherwise
    class OtherRows(type(prob)):
        def inequality_values(self, states, controls):
            return super().inequality_values(states, controls)

    other = copy.copy(prob)
    other.__class__ = OtherRows
    assert other.merit_terms(*other.initial_guess(), None) is None


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_fused_step_choice_matches_torch_form(dtype):
    """tmpc_linesearch_choose_* against the elementwise step choice of
    backtracking_linesearch (linesearch.py:54-178), value for value, on merit
    terms drawn so that candidates sit on both sides of the Armijo test within
    a few ulps, with NaN and infinite terms (a candidate that is not finite
    is never taken; none finite: alpha_0), equal merits (the first is taken)
    and a NaN or infinite mu (nan_to_num)."""
    from turbompc_amd.solvers.linesearch import _choose_fused, _choose_torch

    gen = torch.Generator().manual_seed(9)
    B, alphas = 4096, [0.1, 0.3, 0.7, 1.0]
    A = len(alphas)
    eta, mu_min, mu_max, floor = 1e-4, 0.1, 1.0e6, 1.0e-8
    f = lambda *s: torch.rand(s, generator=gen, dtype=torch.float64)  # noqa: E731
    cost, eq, iq = 10 * f(B), f(B), f(B)
    dcost = -(f(B) * 5)
    eq[:64] = 0.0
    iq[:64] = 0.0  # cl1 below the floor
    dcost[64:96] = float("nan")  # mu NaN -> mu_min
    dcost[96:128] = float("inf")  # mu +inf -> mu_max
    dcost[128:160] = -float("inf")
    cl1 = eq + iq
    mu = torch.clamp(torch.nan_to_num(dcost / (0.5 * cl1.clamp(min=floor)), nan=mu_min, posinf=mu_max,
                                      neginf=mu_min), mu_min, mu_max)
    merit, slope = cost + mu * cl1, dcost - mu * cl1
    # candidates around the Armijo line merit + eta alpha slope (a few ulps either side)
    tgt = torch.stack([merit + eta * a * slope for a in alphas])  # (A, B)
    jit = 1.0 + (f(A, B) - 0.5) * (4e-15 if dtype == torch.float64 else 8e-7)
    far = f(A, B) < 0.3
    cand = torch.where(far, tgt * (1.0 + 0.1 * (f(A, B) - 0.5)), tgt * jit)
    # split each candidate merit into cost_a + mu (eq_a + iq_a)
    eq_a, iq_a = 0.3 * f(A, B), 0.2 * f(A, B)
    cost_a = cand - mu[None] * (eq_a + iq_a)
    cost_a[0, 200:210] = float("nan")
    cost_a[:, 210:220] = float("nan")  # no finite candidate
    eq_a[2, 220:230] = float("inf")
    cost_a[:, 230:240] = cost_a[1, 230:240]  # equal merits
    eq_a[:, 230:240], iq_a[:, 230:240] = eq_a[1, 230:240], iq_a[1, 230:240]
    cost_a[:, 230:240] += 1e3  # and none passes
    d = lambda t: t.to("cuda", dtype).contiguous()  # noqa: E731
    base = (d(cost), d(eq), d(iq), d(dcost))
    ca, ea, ia = d(cost_a).flatten(), d(eq_a).flatten(), d(iq_a).flatten()
    got = _choose_fused(base, (ca, ea, ia, None), alphas, eta, mu_min, mu_max, floor)
    a_t = torch.tensor(alphas, dtype=dtype, device="cuda")
    want = _choose_torch(base[0], base[3], base[1], base[2],
                         lambda m: (ca + m.repeat(A) * (ea + ia)).view(A, B).t(), alphas, a_t, eta, mu_min,
                         mu_max, floor)
    torch.cuda.synchronize()
    assert torch.equal(got, want), int((got != want).sum())
    counts = {a: int((want == a).sum()) for a in alphas}
    print(f"{dtype}: steps taken {counts}")
    assert all(v > 0 for v in counts.values())
    assert torch.all(want[210:220] == alphas[0])
