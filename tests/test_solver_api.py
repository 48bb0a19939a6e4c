"""Host-side solver API (CPU): the reference's construction and parameter
helpers (turbompc_solver.py:441-526, :1480-1501) and the batched candidate
merits of the line search against the one-candidate-at-a-time form."""
import pytest
import torch

from turbompc_amd.problems import configs
from turbompc_amd.solvers.linear_systems_solvers.backends import AdmmBackend, SchurSolverBackend
from turbompc_amd.solvers.linesearch import _candidate_merits
from turbompc_amd.solvers.turbompc_solver import (BackwardBackend, ForwardBackend, TurboMPCSolver,
                                                  parse_backward_backend, parse_forward_backend)


def test_backend_names_and_components():
    assert parse_forward_backend("admm_hip_direct") == ForwardBackend.ADMM_HIP_DIRECT
    assert parse_backward_backend("direct_hip_kkt") == BackwardBackend.DIRECT_HIP_KKT
    with pytest.raises(ValueError):
        parse_forward_backend("no_such_backend")
    solver = TurboMPCSolver(configs.config1(B=2), forward_backend="admm_hip_pcg")
    assert solver.forward_admm_backend == AdmmBackend.HIP_PCG
    assert solver.forward_schur_backend == SchurSolverBackend.IGNORED
    # the direct adjoint solve runs no ADMM (the reference's direct backends report the same)
    assert solver.backward_admm_backend == AdmmBackend.JAX_LOOP
    assert solver.backward_schur_backend == SchurSolverBackend.IGNORED
    with pytest.raises(ValueError):
        TurboMPCSolver(configs.config1(B=2), forward_backend="admm_fused_cudss")


def test_make_params_with_weights_routes_weights_to_the_program():
    prob = configs.config1(B=3, seed=1)
    solver = TurboMPCSolver(prob)
    wx = torch.full((3, 4), 7.0, dtype=torch.float64)
    x0 = torch.zeros((3, 4), dtype=torch.float64)
    params = solver.make_params_with_weights({"weights_penalization_reference_state_trajectory": wx},
                                             {"initial_state": x0})
    assert set(params) == {"initial_state", "weights_penalization_reference_state_trajectory"}
    p, w = solver._split_params(params, None)
    assert set(p) == {"initial_state"} and set(w) == {"weights_penalization_reference_state_trajectory"}
    program = solver._program_for(params, None)
    assert torch.equal(program.wx, wx) and torch.equal(program.x0, x0)
    assert torch.equal(prob.wx, configs.config1(B=3, seed=1).wx)  # the solver's own problem is untouched
    # nested dictionaries merge key by key
    merged = solver.make_params_with_weights({"a": {"y": 2}}, {"a": {"x": 1}, "b": 0})
    assert merged == {"a": {"x": 1, "y": 2}, "b": 0}


@pytest.mark.parametrize("case", ["config1", "config4", "config4_slack"])
def test_tiled_candidates_equal_the_candidate_loop(case):
    B = 5
    if case == "config1":
        prob = configs.config1(B=B, seed=2)
    else:
        prob = configs.config4(B=B, seed=2, use_slack_variables=case.endswith("slack"), slack_penalization_weight=20.0)
    g = torch.Generator().manual_seed(3)
    s0, u0 = prob.initial_guess()
    r = lambda t: torch.randn(t.shape, generator=g, dtype=torch.float64)  # noqa: E731
    states, controls = s0 + r(s0), u0 + r(u0)
    m = prob.num_inequality_constraints
    slacks = 0.1 * torch.randn((B, s0.shape[1], m), generator=g, dtype=torch.float64)
    ds, dc, dsl = r(states), r(controls), 0.1 * r(slacks)
    mu = torch.rand(B, generator=g, dtype=torch.float64) + 0.5
    alphas = [0.1, 0.3, 0.7, 1.0]
    a_t = torch.tensor(alphas, dtype=torch.float64)
    tiled = _candidate_merits(prob, alphas, a_t, states, controls, slacks, ds, dc, dsl, mu)

    class Untiled:  # the same problem without tile(): the one-candidate loop
        def __getattr__(self, name):
            if name == "tile":
                raise AttributeError(name)
            return getattr(prob, name)

    loop = _candidate_merits(Untiled(), alphas, a_t, states, controls, slacks, ds, dc, dsl, mu)
    assert tiled.shape == (B, len(alphas))
    torch.testing.assert_close(tiled, loop, rtol=1e-15, atol=0)
    # the tiled problem repeats every per-problem tensor, copy j at rows j B ..
    t4 = prob.tile(4)
    assert t4.B == 4 * B and prob.tile(4) is t4
    for name in prob.PER_PROBLEM:
        v, tv = getattr(prob, name), getattr(t4, name)
        assert tv.shape[0] == 4 * B and torch.equal(tv[2 * B:3 * B], v), name
