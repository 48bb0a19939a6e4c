"""Pins the CPU restatement of the merit line search (oracle/sqp_cpu.py,
after turbompc/solvers/linesearch.py:54-178) by known answers, and checks the
host line search (turbompc_amd/solvers/linesearch.py, torch) against it.

Known answers: along an exact Newton direction of a quadratic the full step
passes the Armijo test with eta = 0.4; along three times that direction the
largest passing step is 0.3; along an ascent direction no step passes and the
least merit (the shortest step) is taken; with every step failing but a
longer step of less merit, the fallback takes that step, not the first; steps
whose merit is not finite are never taken; mu at its clip points and in
between.  The constraint term is checked against a brute-force sum."""
import numpy as np
import pytest
import torch

from oracle.sqp_cpu import OBSTACLE_LOWER, Merit, merit_linesearch, obstacle_values
from turbompc_amd.problems import configs
from turbompc_amd.problems.obstacle import ObstacleOCP
from turbompc_amd.problems.ocp import LinearOCP
from turbompc_amd.solvers.linesearch import backtracking_linesearch, evaluate_constraints_with_bounds

B, T, NX, NU = 3, 4, 2, 1


def _no_constraints(s, u):
    return np.zeros((s.shape[0], 1))


def _no_ineq(s, u):
    z = np.zeros(s.shape[:2] + (0,))
    return z, z, z


def _quadratic(seed=0):
    rng = np.random.default_rng(seed)
    n = NX + NU
    w = rng.uniform(0.5, 2.0, (B, T, n))
    D = np.zeros((B, T, n, n))
    idx = np.arange(n)
    D[..., idx, idx] = w
    q = rng.standard_normal((B, T, n))
    z = rng.standard_normal((B, T, n))
    newton = -(w * z + q) / w  # to the minimizer of 1/2 z'Dz + q'z
    return Merit(D, q, _no_constraints, _no_ineq), z, newton


def _run(merit, z, dz, sl=None, dsl=None, **kw):
    sl = np.zeros(z.shape[:2] + (0,)) if sl is None else sl
    dsl = np.zeros_like(sl) if dsl is None else dsl
    return merit_linesearch(merit, z[..., :NX], z[..., NX:], sl, (z + dz)[..., :NX], (z + dz)[..., NX:], sl + dsl,
                            **kw)


def test_newton_step_is_taken_whole():
    merit, z, newton = _quadratic()
    (s, u, _), alpha, _ = _run(merit, z, newton)
    np.testing.assert_array_equal(alpha, 1.0)
    np.testing.assert_allclose(np.concatenate([s, u], axis=-1), z + newton, rtol=0, atol=1e-15)


def test_overlong_step_backtracks_to_largest_passing():
    # phi(a) = phi0 + a g + a^2 h / 2 with g = -h/3: a = 1 and 0.7 fail the
    # Armijo test (0.6 g + h/2 > 0, 0.42 g + 0.245 h > 0), a = 0.3 passes
    merit, z, newton = _quadratic(1)
    (s, u, _), alpha, _ = _run(merit, z, 3.0 * newton)
    np.testing.assert_array_equal(alpha, 0.3)
    np.testing.assert_allclose(np.concatenate([s, u], axis=-1), z + 0.9 * newton, rtol=0, atol=1e-14)


def test_ascent_direction_takes_least_merit():
    merit, z, newton = _quadratic(2)
    _, alpha, _ = _run(merit, z, -newton)
    np.testing.assert_array_equal(alpha, 0.1)


def _eq_square(s, u):
    """h(z) = z_0^2 per problem: moving z_0 from 1 by -a gives |h| = (1 - a)^2."""
    return s[:, :1, 0] ** 2


def test_fallback_takes_least_merit_not_first_step():
    # zero cost, |h|(a) = (1 - a)^2: mu = mu_min, merit(a) = 0.1 (1 - a)^2 and
    # the slope is -0.1; with eta = 2.5 every step fails (0.81 - 1 + 0.25 > 0 ...)
    # and the least merit is at a = 1
    n = NX + NU
    merit = Merit(np.zeros((B, T, n, n)), np.zeros((B, T, n)), _eq_square, _no_ineq)
    z = np.zeros((B, T, n))
    z[:, 0, 0] = 1.0
    dz = np.zeros_like(z)
    dz[:, 0, 0] = -1.0
    _, alpha, mu = _run(merit, z, dz, eta=2.5)
    np.testing.assert_array_equal(mu, 0.1)
    np.testing.assert_array_equal(alpha, 1.0)
    # with eta = 0.4 the Armijo test passes everywhere: the longest step
    _, alpha, _ = _run(merit, z, dz, eta=0.4)
    np.testing.assert_array_equal(alpha, 1.0)


def test_non_finite_candidates_are_never_taken():
    # |h| = |log z_0| is infinite at z_0 = 0 (a = 1) and NaN beyond
    def eq_log(s, u):
        with np.errstate(divide="ignore", invalid="ignore"):
            return np.log(s[:, :1, 0])

    n = NX + NU
    merit = Merit(np.zeros((B, T, n, n)), np.zeros((B, T, n)), eq_log, _no_ineq)
    z = np.zeros((B, T, n))
    z[:, 0, 0] = 2.0
    dz = np.zeros_like(z)
    dz[:, 0, 0] = -2.0  # a = 1 reaches z_0 = 0
    _, alpha, _ = _run(merit, z, dz)
    assert np.all(alpha < 1.0)
    # the largest finite passing step: |log(2 - 2a)| at a = 0.7 is 0.51 < log 2 - ...
    cl0 = np.log(2.0)
    expect = max(a for a in (0.1, 0.3, 0.7) if 0.1 * abs(np.log(2 - 2 * a)) <= 0.1 * cl0 - 0.4 * a * 0.1 * cl0)
    np.testing.assert_array_equal(alpha, expect)
    # nothing finite at all: the first candidate
    merit_nan = Merit(np.zeros((B, T, n, n)), np.zeros((B, T, n)), lambda s, u: np.full((s.shape[0], 1), np.nan),
                      _no_ineq)
    _, alpha, _ = _run(merit_nan, z, dz)
    np.testing.assert_array_equal(alpha, 0.1)


def test_mu_clip_points_and_interior():
    n = NX + NU
    D = np.zeros((B, T, n, n))
    q = np.zeros((B, T, n))
    q[:, 0, 0] = 1.0  # dcost = dz_00
    z = np.zeros((B, T, n))
    z[:, 0, 0] = 2.0  # |h| = |z_00| = 2 -> cl1 = 2
    merit = Merit(D, q, lambda s, u: s[:, :1, 0], _no_ineq)
    for dz00, mu_expect in ((-1.0, 0.1), (0.4, 0.4), (0.0, 0.1), (3.0e6, 1.0e6)):
        dz = np.zeros_like(z)
        dz[:, 0, 0] = dz00
        _, _, mu = _run(merit, z, dz)
        np.testing.assert_allclose(mu, mu_expect, rtol=1e-15)
    # no violation (cl1 = 0 -> the floor 1e-8): mu = dcost / 5e-9, clipped
    merit0 = Merit(D, q, _no_constraints, _no_ineq)
    for dz00, mu_expect in ((1e-3, 2.0e5), (1e-2, 1.0e6)):
        dz = np.zeros_like(z)
        dz[:, 0, 0] = dz00
        _, _, mu = _run(merit0, z, dz)
        np.testing.assert_allclose(mu, mu_expect, rtol=1e-12)


def test_constraint_l1_and_slack_cost_brute_force():
    rng = np.random.default_rng(3)
    n, m = NX + NU, 2
    s, u = rng.standard_normal((B, T, NX)), rng.standard_normal((B, T, NU))
    sl = rng.standard_normal((B, T, m))
    lo, hi = -0.5 * np.ones((B, T, m)), 0.5 * np.ones((B, T, m))
    G = rng.standard_normal((B, T, m, n))
    merit = Merit(np.zeros((B, T, n, n)), np.zeros((B, T, n)), lambda a, b: np.ones((a.shape[0], 3)),
                  lambda a, b: (np.einsum("btij,btj->bti", G, np.concatenate([a, b], -1)), lo, hi),
                  slack_weight=7.0, use_slack=True)
    got = merit.constraint_l1(s, u, sl)
    for b in range(B):
        tot = 3.0
        for t in range(T):
            for i in range(m):
                g = float(G[b, t, i] @ np.concatenate([s[b, t], u[b, t]])) + sl[b, t, i]
                tot += max(0.0, -0.5 - g) + max(0.0, g - 0.5)
        assert abs(got[b] - tot) < 1e-12
    np.testing.assert_allclose(merit.cost(s, u, sl), 3.5 * np.sum(sl * sl, axis=(1, 2)), rtol=1e-15)
    dsl = rng.standard_normal(sl.shape)
    h = 1e-6
    fd = (merit.cost(s, u, sl + h * dsl) - merit.cost(s, u, sl - h * dsl)) / (2 * h)
    np.testing.assert_allclose(merit.cost_derivative(s, u, sl, 0 * s, 0 * u, dsl), fd, rtol=1e-8)


# ------------------------------------------- host line search vs oracle ----
def _oracle_merit(prob, states, controls, use_slack=False, gamma=0.0):
    D, E, q = (t.numpy() for t in prob.cost_blocks())
    A0, c0 = (t.numpy() for t in prob.initial_equality())
    Am, c = (t.numpy() for t in prob.dynamics_blocks(states, controls))
    Ap = prob.a_plus().numpy()

    def eq(s, u):
        z = np.concatenate([s, u], axis=-1)
        h0 = np.einsum("bij,bj->bi", A0, z[:, 0]) - c0
        hd = np.einsum("btij,btj->bti", Am, z[:, :-1]) + np.einsum("btij,btj->bti", Ap, z[:, 1:]) - c
        return np.concatenate([h0, hd.reshape(hd.shape[0], -1)], axis=1)

    G, lo, hi = (t.numpy() for t in LinearOCP.inequality_blocks(prob))

    def ineq(s, u):
        g = np.einsum("btij,btj->bti", G, np.concatenate([s, u], axis=-1))
        if not isinstance(prob, ObstacleOCP):
            return g, lo, hi
        go = obstacle_values(s, prob.centers.numpy(), prob.radii.numpy(), prob.obstacles_dimension)
        return (np.concatenate([g, go], axis=2), np.concatenate([lo, np.full_like(go, OBSTACLE_LOWER)], axis=2),
                np.concatenate([hi, np.zeros_like(go)], axis=2))

    return Merit(D, q, eq, ineq, slack_weight=gamma, use_slack=use_slack)


@pytest.mark.parametrize("case", ["config1", "config4", "config4_slack"])
def test_host_linesearch_matches_oracle(case):
    Bc = 24
    if case == "config1":
        prob = configs.config1(B=Bc, seed=4)
    else:
        prob = configs.config4(B=Bc, seed=4, use_slack_variables=case.endswith("slack"),
                               slack_penalization_weight=30.0)
    use_slack = bool(prob.use_slack_variables)
    s0, u0 = prob.initial_guess()
    g = torch.Generator().manual_seed(11)
    r = lambda t: torch.randn(t.shape, generator=g, dtype=torch.float64)  # noqa: E731
    states, controls = s0 + 0.5 * r(s0), u0 + 0.5 * r(u0)
    m = prob.num_inequality_constraints
    slacks = 0.1 * torch.randn((Bc, s0.shape[1], m), generator=g, dtype=torch.float64) if use_slack else \
        torch.zeros((Bc, s0.shape[1], m), dtype=torch.float64)
    # directions of mixed lengths, so that different steps get taken
    scale = torch.logspace(-2, 1, Bc, dtype=torch.float64).view(-1, 1, 1)
    s_new, c_new = states + scale * r(states), controls + scale * r(controls)
    sl_new = slacks + scale * 0.1 * r(slacks) if use_slack else slacks.clone()
    params = dict(linesearch_eta=0.4, linesearch_alphas=[0.1, 0.3, 0.7, 1.0])
    (s, u, sl), alpha = backtracking_linesearch(prob, None, params, states, controls, slacks, s_new, c_new, sl_new)
    merit = _oracle_merit(prob, states, controls, use_slack, 30.0)
    n = lambda t: t.numpy()  # noqa: E731
    (s_o, u_o, sl_o), alpha_o, _ = merit_linesearch(merit, n(states), n(controls), n(slacks), n(s_new), n(c_new),
                                                    n(sl_new))
    np.testing.assert_array_equal(alpha.numpy(), alpha_o)
    assert len(set(alpha_o.tolist())) >= 2, alpha_o  # more than one outcome is exercised
    np.testing.assert_allclose(s.numpy(), s_o, rtol=0, atol=1e-13)
    np.testing.assert_allclose(u.numpy(), u_o, rtol=0, atol=1e-13)
    np.testing.assert_allclose(sl.numpy(), sl_o, rtol=0, atol=1e-13)
    # the constraint norms of both sides at the start point
    e, i, *_ = evaluate_constraints_with_bounds(prob, states, controls, slacks)
    np.testing.assert_allclose((e + i).numpy(), merit.constraint_l1(n(states), n(controls), n(slacks)),
                               rtol=1e-12)
    # the cost differs from the QP-block cost by a constant only
    dc = prob.cost(s_new, c_new, sl_new) - prob.cost(states, controls, slacks)
    dc_o = merit.cost(n(s_new), n(c_new), n(sl_new)) - merit.cost(n(states), n(controls), n(slacks))
    np.testing.assert_allclose(dc.numpy(), dc_o, rtol=1e-10, atol=1e-9)
