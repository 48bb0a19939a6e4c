"""Backtracking line search on the l1 merit function, batched over problems.

Follows backtracking_linesearch / evaluate_constraints_with_bounds
(turbompc/solvers/linesearch.py:14-178), which the reference applies per
problem under vmap:
  merit(z)  = cost(z) + mu * (|h(z)|_1 + |viol(g(z))|_1)
  mu        = clip(nan_to_num(dcost / (0.5 max(|c|_1, floor))), mu_min, mu_max)
  accept the largest alpha of `linesearch_alphas` with
      merit(z + alpha dz) <= merit(z) + eta alpha (dcost - mu |c|_1)
  and, when no finite candidate passes, the finite candidate of least merit
  (the first candidate if none is finite).
The problem supplies cost, cost_directional_derivative, equality_residuals
and inequality_values (problems/ocp.py); problem_params, when given, are
applied with program.with_params as in the solver.
"""
from __future__ import annotations

import ctypes
from typing import Any, Dict, Tuple

import torch


def _with_params(program, problem_params):
    return program.with_params(problem_params) if problem_params else program


def evaluate_constraints_with_bounds(program, states, controls, slacks, problem_params=None):
    """(|h|_1 (B,), |viol|_1 (B,), g, l, u (B, T, m)), with g + slack for soft
    constraints (evaluate_constraints_with_bounds, linesearch.py:14-52)."""
    program = _with_params(program, problem_params)
    eq = program.equality_residuals(states, controls).abs().flatten(1).sum(dim=1)
    g, lo, hi = program.inequality_values(states, controls)
    if getattr(program, "use_slack_variables", False) and slacks is not None and slacks.numel():
        g = g + slacks
    if g.shape[-1] == 0:
        return eq, torch.zeros_like(eq), g, lo, hi
    viol = torch.clamp(lo - g, min=0.0) + torch.clamp(g - hi, min=0.0)
    return eq, viol.flatten(1).sum(dim=1), g, lo, hi


def _merit_terms(program, states, controls, slacks, ds=None, dc=None, dsl=None, copies=1):
    """(cost, |h|_1, |viol|_1, dcost or None) from the problem's fused
    evaluation (QuadraticTrackingOCP.merit_terms: one kernel), or None where
    it has none for this problem."""
    fn = getattr(program, "merit_terms", None)
    return fn(states, controls, slacks, ds, dc, dsl, copies=copies) if fn is not None else None


def _candidate_merits(program, alphas, a_t, states, controls, slacks, ds, dc, dsl, mu):
    """(B, n_alpha): merit(z + alpha dz) for every candidate.  A program that
    can tile its batch (QuadraticTrackingOCP.tile) evaluates all candidates in
    one pass over n_alpha B problems, candidate j at rows j B .. j B + B - 1
    (its terms in one kernel where the problem has one); others are evaluated
    one candidate at a time."""
    A, B = len(alphas), states.shape[0]
    if hasattr(program, "tile"):
        stack = lambda z, dz: (z[None] + a_t.view(A, *([1] * z.dim())) * dz[None]).flatten(0, 1)  # noqa: E731
        s_a, c_a, sl_a = stack(states, ds), stack(controls, dc), stack(slacks, dsl)
        fused = _merit_terms(program, s_a, c_a, sl_a, copies=A)
        if fused is not None:
            cost_a, e_a, i_a, _ = fused
            return (cost_a + mu.repeat(A) * (e_a + i_a)).view(A, B).t()
        tiled = program.tile(A)
        e_a, i_a, *_ = evaluate_constraints_with_bounds(tiled, s_a, c_a, sl_a)
        m = tiled.cost(s_a, c_a, sl_a) + mu.repeat(A) * (e_a + i_a)
        return m.view(A, B).t()
    cand = []
    for a in alphas:
        s_a, c_a, sl_a = states + a * ds, controls + a * dc, slacks + a * dsl
        e_a, i_a, *_ = evaluate_constraints_with_bounds(program, s_a, c_a, sl_a)
        cand.append(program.cost(s_a, c_a, sl_a) + mu * (e_a + i_a))
    return torch.stack(cand, dim=1)


def _choose_fused(base, cand, alphas, eta, mu_min, mu_max, floor):
    """alpha (B,): the step choice below in one kernel (tmpc_linesearch_choose_*)
    from the merit terms of the base point and of the stacked candidates."""
    from .. import _lib

    cost, eq, iq, dcost = base
    cost_a, eq_a, iq_a, _ = cand
    B, dt, dev = cost.shape[0], cost.dtype, cost.device
    alpha = torch.empty(B, dtype=dt, device=dev)
    fn = f"tmpc_linesearch_choose_{_lib.suffix(dt)}"
    p = _lib.ptr
    _lib.check(fn, getattr(_lib.load(), fn)(
        _lib.stream_handle(dev), B, len(alphas), p(cost), p(dcost), p(eq), p(iq), p(cost_a), p(eq_a), p(iq_a),
        (ctypes.c_double * len(alphas))(*alphas), eta, mu_min, mu_max, floor, p(alpha), None))
    return alpha


def backtracking_linesearch(program, problem_params, solver_params: Dict[str, Any], states, controls, slacks,
                            states_new, controls_new, slacks_new
                            ) -> Tuple[Tuple[torch.Tensor, torch.Tensor, torch.Tensor], torch.Tensor]:
    """Returns ((states, controls, slacks) at the accepted step, alpha (B,))."""
    program = _with_params(program, problem_params)
    eta = float(solver_params["linesearch_eta"])
    alphas = [float(a) for a in solver_params["linesearch_alphas"]]
    mu_min = float(solver_params.get("linesearch_mu_min", 0.1))
    mu_max = float(solver_params.get("linesearch_mu_max", 1.0e6))
    floor = float(solver_params.get("linesearch_constraint_floor", 1.0e-8))
    ds, dc, dsl = states_new - states, controls_new - controls, slacks_new - slacks

    fused = _merit_terms(program, states, controls, slacks, ds, dc, dsl)
    if fused is not None and hasattr(program, "tile") and 1 <= len(alphas) <= 8:
        # the candidates' terms and the choice among them in two kernels
        A = len(alphas)
        a_t = torch.tensor(alphas, dtype=states.dtype).to(states.device, non_blocking=True)
        stack = lambda z, dz: (z[None] + a_t.view(A, *([1] * z.dim())) * dz[None]).flatten(0, 1)  # noqa: E731
        cand = _merit_terms(program, stack(states, ds), stack(controls, dc), stack(slacks, dsl), copies=A)
        if cand is not None:
            alpha = _choose_fused(fused, cand, alphas, eta, mu_min, mu_max, floor)
            al = alpha.view(-1, 1, 1)
            return (states + al * ds, controls + al * dc, slacks + al * dsl), alpha
    if fused is not None:
        cost, eq, iq, dcost = fused
    else:
        cost = program.cost(states, controls, slacks)
        dcost = program.cost_directional_derivative(states, controls, slacks, ds, dc, dsl)
        eq, iq, *_ = evaluate_constraints_with_bounds(program, states, controls, slacks)
    a_t = torch.tensor(alphas, dtype=states.dtype).to(states.device, non_blocking=True)
    alpha = _choose_torch(cost, dcost, eq, iq,
                          lambda mu: _candidate_merits(program, alphas, a_t, states, controls, slacks, ds, dc, dsl, mu),
                          alphas, a_t, eta, mu_min, mu_max, floor)
    al = alpha.view(-1, 1, 1)
    return (states + al * ds, controls + al * dc, slacks + al * dsl), alpha


def _choose_torch(cost, dcost, eq, iq, candidate_merits, alphas, a_t, eta, mu_min, mu_max, floor):
    """alpha (B,): the step choice of backtracking_linesearch (linesearch.py:54-178)
    in elementwise torch operations; candidate_merits(mu) gives the (B,
    n_alpha) merits of the candidates."""
    cl1 = eq + iq
    mu_raw = dcost / (0.5 * torch.clamp(cl1, min=floor))
    mu = torch.clamp(torch.nan_to_num(mu_raw, nan=mu_min, posinf=mu_max, neginf=mu_min), mu_min, mu_max)
    merit = cost + mu * cl1
    merit_deriv = dcost - mu * cl1
    cand = candidate_merits(mu)  # (B, n_alpha)
    # eta alpha rounded from its double product, as a Python scalar would be
    ea_t = torch.tensor([eta * a for a in alphas], dtype=cost.dtype).to(cost.device, non_blocking=True)
    dec = cand - (merit[:, None] + ea_t[None] * merit_deriv[:, None])
    finite = torch.isfinite(a_t)[None] & torch.isfinite(cand) & torch.isfinite(dec)
    valid = finite & (dec <= 0)
    idx = torch.arange(len(alphas), device=cand.device).expand_as(cand)
    valid_index = torch.where(valid, idx, torch.full_like(idx, -1)).amax(dim=1)
    best_finite = torch.where(finite, cand, torch.full_like(cand, float("inf"))).argmin(dim=1)
    fallback = torch.where(finite.any(dim=1), best_finite, torch.zeros_like(best_finite))
    index = torch.where(valid_index >= 0, valid_index, fallback)
    return a_t[index]
