"""TEST INFRASTRUCTURE ONLY — CPU restatement of the SQP loop for the quadrotor
and obstacle-avoidance workloads.

Restates TurboMPCSolver._solve_impl (turbompc/solvers/turbompc_solver.py:1519-1760)
with the first_order criterion at a fixed iteration count (tol_convergence = 0):
  linearize (RK4 Jacobians by complex step, liboracle; obstacle rows in numpy)
  -> ADMM (liboracle)
  -> relinearize at the new iterate, carrying the ADMM state (including rho)
Used by bench.py's cpu_baseline leg and by the SQP parity tests.

Pins: the loop itself (tests/test_oracle_sqp.py) -- on linear dynamics n_sqp
iterations of K ADMM steps equal one solve of n_sqp*K steps from the zero
state bit for bit (x starts at 0 once, z and the duals carry), and with
adaptive rho the chain of ADMM calls on the carried state, rho included; the
converged quadrotor SQP meets the NLP first-order conditions evaluated with an
independent numpy RK4 and complex-step Jacobians.  The quadrotor Jacobians are checked against central differences and
torch.func.jacfwd (tests/test_oracle_adjoint_quadrotor.py); the obstacle rows
against central differences of g, known answers on the sphere and the exactness
of the linearization at its own point, and their Hessian against differences
of the gradient and its null direction (tests/test_oracle_obstacle.py).
The rescaled QP (scale_qp_np) is pinned by the equivalence it must keep
(tests/test_rescaling.py): solved to convergence, S times its solution is the
unscaled QP's solution and its multipliers are the unscaled ones divided by
the row scales.
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


LINESEARCH_DEFAULTS = dict(eta=0.4, alphas=(0.1, 0.3, 0.7, 1.0), mu_min=0.1, mu_max=1.0e6, floor=1.0e-8)


class Merit:
    """The terms of the l1 merit function of one workload, in numpy.

    cost: the tracking cost from the QP's own blocks, 1/2 z'Dz + q'z per stage
    (it differs from the problem's cost by a constant, which no decision of
    the line search sees), plus gamma/2 |slack|^2 with soft constraints
    (cost_with_slack, optimal_control_problem.py:1504-1515).
    eq(states, controls) -> (B, ...) equality residuals h(z);
    ineq(states, controls) -> (g, l, u), each (B, ...)."""

    def __init__(self, D, q, eq, ineq, *, slack_weight=0.0, use_slack=False):
        self.D, self.q, self.eq, self.ineq = D, q, eq, ineq
        self.gamma, self.use_slack = float(slack_weight), bool(use_slack)

    def cost(self, s, u, sl):
        z = np.concatenate([s, u], axis=-1)
        c = 0.5 * np.einsum("bti,btij,btj->b", z, self.D, z) + np.einsum("bti,bti->b", self.q, z)
        if self.use_slack:
            c = c + 0.5 * self.gamma * np.sum(sl * sl, axis=(1, 2))
        return c

    def cost_derivative(self, s, u, sl, ds, du, dsl):
        z, dz = np.concatenate([s, u], axis=-1), np.concatenate([ds, du], axis=-1)
        grad = np.einsum("btij,btj->bti", self.D, z) + self.q
        d = np.einsum("bti,bti->b", grad, dz)
        if self.use_slack:
            d = d + self.gamma * np.sum(sl * dsl, axis=(1, 2))
        return d

    def constraint_l1(self, s, u, sl):
        """|h|_1 + |viol(g (+ slack))|_1 (evaluate_constraints_with_bounds, linesearch.py:14-52)."""
        B = s.shape[0]
        eq = np.sum(np.abs(self.eq(s, u)).reshape(B, -1), axis=1)
        g, lo, hi = self.ineq(s, u)
        if self.use_slack:
            g = g + sl
        viol = np.maximum(0.0, lo - g) + np.maximum(0.0, g - hi)
        return eq + np.sum(viol.reshape(B, -1), axis=1)


def merit_linesearch(merit: Merit, states, controls, slacks, s_new, c_new, sl_new, *, eta=0.4,
                     alphas=(0.1, 0.3, 0.7, 1.0), mu_min=0.1, mu_max=1.0e6, floor=1.0e-8):
    """backtracking_linesearch (turbompc/solvers/linesearch.py:54-178), one
    problem at a time for the choice of step.  Returns ((states, controls,
    slacks) at the accepted step, alpha (B,), mu (B,))."""
    ds, du, dsl = s_new - states, c_new - controls, sl_new - slacks
    B = states.shape[0]
    cost = merit.cost(states, controls, slacks)
    dcost = merit.cost_derivative(states, controls, slacks, ds, du, dsl)
    cl1 = merit.constraint_l1(states, controls, slacks)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        mu = np.clip(np.nan_to_num(dcost / (0.5 * np.maximum(cl1, floor)), nan=mu_min, posinf=mu_max,
                                   neginf=mu_min), mu_min, mu_max)
    merit0 = cost + mu * cl1
    slope = dcost - mu * cl1
    cand = np.stack([merit.cost(states + a * ds, controls + a * du, slacks + a * dsl)
                     + mu * merit.constraint_l1(states + a * ds, controls + a * du, slacks + a * dsl)
                     for a in alphas], axis=1)
    alpha = np.zeros(B)
    for b in range(B):
        dec = [cand[b, k] - (merit0[b] + eta * a * slope[b]) for k, a in enumerate(alphas)]
        finite = [bool(np.isfinite(a) and np.isfinite(cand[b, k]) and np.isfinite(dec[k]))
                  for k, a in enumerate(alphas)]
        passing = [k for k in range(len(alphas)) if finite[k] and dec[k] <= 0]
        if passing:  # the largest step that passes the Armijo test
            k = passing[-1]
        elif any(finite):  # else the finite candidate of least merit (first of equals)
            k = min((k for k in range(len(alphas)) if finite[k]), key=lambda j: cand[b, j])
        else:
            k = 0
        alpha[b] = alphas[k]
    a3 = alpha[:, None, None]
    return (states + a3 * ds, controls + a3 * du, slacks + a3 * dsl), alpha, mu


def scale_qp_np(qp, state_diff, control_diff, ineq_row_scale):
    """The QP in the scaled variables z_hat = z / [state_diff, control_diff]
    of the reference's variable rescaling: the problem scales its constraint
    rows (the initial rows by 1 / state_diff, then 1 / control_diff for u_0
    rows, optimal_control_problem.py:944-956; the dynamics rows by
    1 / state_diff, :1324-1332; the inequality rows by ineq_row_scale, :460-469,
    obstacle_avoidance.py:42-47), then scale_qp_data scales the columns by
    S = diag(state_diff, control_diff) (qp_data.py:178-211)."""
    sd, cd = np.asarray(state_diff, dtype=np.float64), np.asarray(control_diff, dtype=np.float64)
    sc = np.concatenate([sd, cd])
    r0 = 1.0 / sc[: qp.eq.A0.shape[-2]]
    rd, rg = 1.0 / sd, np.asarray(ineq_row_scale, dtype=np.float64)
    return QPNS(
        _ns(D=qp.cost.D * sc[:, None] * sc, E=qp.cost.E * sc[:, None] * sc, q=qp.cost.q * sc),
        _ns(A0=qp.eq.A0 * r0[:, None] * sc, A_minus=qp.eq.A_minus * rd[:, None] * sc,
            A_plus=qp.eq.A_plus * rd[:, None] * sc, c0=qp.eq.c0 * r0, c=qp.eq.c * rd),
        _ns(G=qp.ineq.G * rg[:, None] * sc, l=qp.ineq.l * rg, u=qp.ineq.u * rg,
            slack_penalization_weight=qp.ineq.slack_penalization_weight,
            use_slack_variables=qp.ineq.use_slack_variables),
    )


def _scaled_merit_terms(eq, ineq, n0, scaling):
    """The merit's residuals with the rows scaled as in scale_qp_np (the
    reference's equality_constraints and inequality values with rescaling,
    optimal_control_problem.py:892-910, :460-469)."""
    sd, cd, rg = (np.asarray(a, dtype=np.float64) for a in scaling)
    r0 = 1.0 / np.concatenate([sd, cd])[:n0]

    def eq_s(s, u):
        h = eq(s, u)
        B = h.shape[0]
        return np.concatenate([h[:, :n0] * r0, (h[:, n0:].reshape(B, -1, sd.size) / sd).reshape(B, -1)], axis=1)

    def ineq_s(s, u):
        g, lo, hi = ineq(s, u)
        return g * rg, lo * rg, hi * rg
    return eq_s, ineq_s


def sqp_fixed(qp_at, x_guess, u_guess, *, n, m, n0, cfg: "ora.OracleCfg", rho0, n_sqp, dtype=np.float64,
              nthreads=None, merit: "Merit | None" = None, linesearch=None, state0=None, scaling=None):
    """Fixed-count SQP: qp_at(states, controls) -> QP; the ADMM state (including
    rho and the slack) carries across iterations; x starts at 0
    (turbompc_solver.py:1545-1551), or the solve is warm-started from the
    ADMM state `state0` (an OracleState, the admm_state of a previous solve,
    turbompc_solver.py:1032-1037; then rho0 is not used, and the iterate's
    slack starts at state0's).  With `merit`, each QP solution is a step
    direction scaled by merit_linesearch (options `linesearch`, defaults
    LINESEARCH_DEFAULTS) and the next linearization is at the blended iterate;
    the ADMM state is carried unblended (turbompc_solver.py:1591-1604).
    scaling: (state_diff, control_diff, ineq_row_scale) to solve each QP in
    the rescaled variables (scale_qp_np) and unscale its solution
    (turbompc_solver.py:1151-1155, :1582-1585); the ADMM state stays scaled.
    Returns (states, controls, admm_state), plus (slacks, alphas (B, n_sqp))
    with `merit`."""
    states, controls = x_guess.astype(np.float64), u_guess.astype(np.float64)
    B, T, nx = states.shape
    qp_raw = qp_at
    if scaling is not None:
        qp_at = lambda s_, u_: scale_qp_np(qp_raw(s_, u_), *scaling)  # noqa: E731
    qp = qp_at(states, controls)
    if state0 is None:
        z0 = np.clip(np.zeros((B, T, m)), qp.ineq.l, qp.ineq.u)
        st = ora.OracleState(np.zeros((B, T, n)), np.zeros((B, T, m)), np.zeros((B, n0)),
                             np.zeros((B, T - 1, nx)), z0, np.zeros((B, T, m)), np.full((B,), float(rho0)))
    else:
        st = ora.OracleState(*[np.array(a, dtype=np.float64) for a in state0])
    slacks = st.xi_g.copy()
    alphas = np.zeros((B, n_sqp))
    ls = dict(LINESEARCH_DEFAULTS, **(linesearch or {}))
    for it in range(n_sqp):
        st, _, _ = ora.admm_solve(qp, st, cfg, schur="direct", dtype=dtype, nthreads=nthreads)
        st = ora.OracleState(*[np.asarray(a, dtype=np.float64) for a in st])
        s_new, c_new, sl_new = st.x_blocks[..., :nx], st.x_blocks[..., nx:], st.xi_g
        if scaling is not None:
            s_new, c_new = s_new * np.asarray(scaling[0]), c_new * np.asarray(scaling[1])
        if merit is not None:
            (s_new, c_new, sl_new), alphas[:, it], _ = merit_linesearch(merit, states, controls, slacks, s_new,
                                                                        c_new, sl_new, **ls)
        states, controls, slacks = s_new, c_new, sl_new
        if it + 1 < n_sqp:
            qp = qp_at(states, controls)
    if merit is not None:
        return states, controls, st, slacks, alphas
    return states, controls, st


def obstacle_values(states, centers, radii, dim):
    """g_k = 1 - |p - c_k| / (r_k + 0.001) (B,T,K) (obstacle_avoidance.py:28-41)."""
    d = states[..., None, :dim] - centers[:, None]
    return 1.0 - np.sqrt(np.sum(d * d, axis=-1)) / (radii[:, None] + OBSTACLE_MARGIN)


def _linear_dynamics_residual(static, A_minus, c):
    """h(z) of linear dynamics from the QP's own rows: A0 z_0 - c0, then
    A_minus z_t + A_plus z_{t+1} - c_t (exact when the dynamics are linear)."""
    def eq(s, u):
        z = np.concatenate([s, u], axis=-1)
        h0 = np.einsum("bij,bj->bi", static["A0"], z[:, 0]) - static["c0"]
        hd = (np.einsum("btij,btj->bti", A_minus, z[:, :-1]) + np.einsum("btij,btj->bti", static["A_plus"], z[:, 1:])
              - c)
        return np.concatenate([h0.reshape(h0.shape[0], -1), hd.reshape(hd.shape[0], -1)], axis=1)
    return eq


def _box_values(static):
    def box(s, u):
        z = np.concatenate([s, u], axis=-1)
        return np.einsum("btij,btj->bti", static["G"], z), static["l"], static["u"]
    return box


def _no_cross_terms(static):
    if np.any(static["E"] != 0):
        raise ValueError("the merit cost here covers stage-separable costs (E = 0)")


def obstacle_sqp(static, x_guess, u_guess, *, A_minus, c, centers, radii, dim, cfg: "ora.OracleCfg", rho0, n_sqp,
                 slack_weight=0.0, use_slack=False, dtype=np.float64, nthreads=None, linesearch=None, state0=None,
                 scaling=None):
    """static: numpy QP blocks that do not change (D, E, q, A0, c0, A_plus) and
    the box rows (G, l, u) (B,T,mb,n); the obstacle rows follow the box rows.
    linesearch: None, or a dict of line-search options (possibly empty) to run
    the merit line search (then also returns slacks and alphas).  state0: a
    starting ADMM state (sqp_fixed)."""
    Gb, lb, ub = static["G"], static["l"], static["u"]
    B, T, mb, n = Gb.shape
    K = centers.shape[1]
    merit = None
    if linesearch is not None:
        _no_cross_terms(static)
        box = _box_values(static)

        def ineq(s, u):
            g, lo, hi = box(s, u)
            go = obstacle_values(s, centers, radii, dim)
            return (np.concatenate([g, go], axis=2), np.concatenate([lo, np.full_like(go, OBSTACLE_LOWER)], axis=2),
                    np.concatenate([hi, np.zeros_like(go)], axis=2))

        eq = _linear_dynamics_residual(static, A_minus, c)
        if scaling is not None:
            eq, ineq = _scaled_merit_terms(eq, ineq, static["A0"].shape[-2], scaling)
        merit = Merit(static["D"], static["q"], eq, ineq, slack_weight=slack_weight, use_slack=use_slack)

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
                     n_sqp=n_sqp, dtype=dtype, nthreads=nthreads, merit=merit, linesearch=linesearch, state0=state0,
                     scaling=scaling)


def quadrotor_dynamics_residual(static, dt, params, nthreads=None):
    """h(z): A0 z_0 - c0, then f(x_t, u_t) - x_{t+1} with the RK4 step f
    (equality_constraints, optimal_control_problem.py:841-912)."""
    def eq(s, u):
        B, T, nx = s.shape
        xu = np.concatenate([s[:, :-1], u[:, :-1]], axis=-1).reshape(-1, 17)
        f, _ = ora.quadrotor_rk4_jac(xu, dt, params, nthreads=nthreads)
        h0 = np.einsum("bij,bj->bi", static["A0"], np.concatenate([s[:, 0], u[:, 0]], axis=-1)) - static["c0"]
        return np.concatenate([h0, (f.reshape(B, T - 1, nx) - s[:, 1:]).reshape(B, -1)], axis=1)
    return eq


def quadrotor_sqp(static, x_guess, u_guess, *, dt, params, cfg: "ora.OracleCfg", rho0, n_sqp, dtype=np.float64,
                  nthreads=None, linesearch=None, state0=None, scaling=None):
    """static: dict of numpy QP blocks that do not change (D, E, q, A0, c0, A_plus, G, l, u).
    Returns (states, controls, admm_state); with `linesearch` (a dict of
    options, possibly empty) runs the merit line search and also returns
    slacks and alphas.  state0: a starting ADMM state (sqp_fixed)."""
    n = static["D"].shape[-1]
    m = static["G"].shape[-2]
    merit = None
    if linesearch is not None:
        _no_cross_terms(static)
        eq, ineq = quadrotor_dynamics_residual(static, dt, params, nthreads), _box_values(static)
        if scaling is not None:
            eq, ineq = _scaled_merit_terms(eq, ineq, static["A0"].shape[-2], scaling)
        merit = Merit(static["D"], static["q"], eq, ineq)

    def qp_at(s, u):
        Am, c = linearize_quadrotor(s, u, dt, params)
        return QPNS(
            _ns(D=static["D"], E=static["E"], q=static["q"]),
            _ns(A0=static["A0"], A_minus=Am, A_plus=static["A_plus"], c0=static["c0"], c=c),
            _ns(G=static["G"], l=static["l"], u=static["u"], slack_penalization_weight=0.0,
                use_slack_variables=False),
        )

    return sqp_fixed(qp_at, x_guess, u_guess, n=n, m=m, n0=static["A0"].shape[-2], cfg=cfg, rho0=rho0,
                     n_sqp=n_sqp, dtype=dtype, nthreads=nthreads, merit=merit, linesearch=linesearch, state0=state0,
                     scaling=scaling)
