"""Host-side solver API (CPU): the reference's construction and parameter
helpers (turbompc_solver.py:441-526, :1480-1501) and the batched candidate
merits of the line search against the one-candidate-at-a-time form."""
import pytest
import torch

from turbompc_amd.problems import configs
from turbompc_amd.problems.ocp import LinearOCP
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
    # nested dictionaries merge key by key, into a copy: the caller's
    # dictionaries are unchanged (turbompc_solver.py:511-526 deep-copies)
    base = {"a": {"x": 1}, "b": 0}
    merged = solver.make_params_with_weights({"a": {"y": 2}}, base)
    assert merged == {"a": {"x": 1, "y": 2}, "b": 0}
    assert base == {"a": {"x": 1}, "b": 0}
    w = {"weights_penalization_control_squared": torch.ones((3, 2), dtype=torch.float64)}
    merged = solver.make_params_with_weights(w, {"initial_state": x0})
    merged["weights_penalization_control_squared"][0, 0] = 5.0
    merged["initial_state"][0, 0] = 5.0
    assert float(w["weights_penalization_control_squared"][0, 0]) == 1.0 and float(x0[0, 0]) == 0.0
    # without problem_params the program's own parameters are the base
    own = solver.make_params_with_weights({"weights_penalization_reference_state_trajectory": wx})
    assert torch.equal(own["initial_state"], prob.x0) and own["initial_state"] is not prob.x0
    assert torch.equal(own["weights_penalization_control_squared"], prob.wu)
    assert torch.equal(own["weights_penalization_reference_state_trajectory"], wx)


def test_linear_ocp_expands_shared_blocks_and_checks_shapes():
    """Blocks shared by the batch are expanded to one per problem (the device
    step kernel indexes them per problem); shapes that do not broadcast, and
    trajectories of the wrong length, are refused."""
    ref = configs.config1(B=3, seed=4)
    A, Bm = ref.A[0], ref.Bm[0]
    kw = dict(horizon=ref.horizon, num_states=4, num_controls=2, initial_state=ref.x0, weights_state=ref.wx,
              weights_control=ref.wu, weights_final=ref.wf)
    b = torch.tensor([[0.1, -0.2, 0.3, 0.0]], dtype=torch.float64)  # (1, nx)
    prob = LinearOCP(A=A, Bm=Bm, b=b, **kw)
    assert prob.A.shape == (3, 4, 4) and prob.Bm.shape == (3, 4, 2) and prob.b.shape == (3, 4)
    s, u = prob.initial_guess()
    xn = prob.next_states(s, u)
    assert torch.allclose(xn[2], s[2, :-1] @ A.T + u[2, :-1] @ Bm.T + b[0])
    assert prob.tile(2).b.shape == (6, 4)
    with pytest.raises(ValueError, match="does not broadcast"):
        LinearOCP(A=A, Bm=Bm, b=torch.zeros((2, 4), dtype=torch.float64), **kw)
    with pytest.raises(ValueError, match="states has shape"):
        prob.next_states(s[:, :-1], u)
    with pytest.raises(ValueError, match="A has shape"):
        prob.next_states(s[:2], u[:2])  # 2 problems' trajectories for a problem of 3


def test_initial_control_rows():
    """constrain_initial_control (optimal_control_problem.py:958-978, :897-910):
    A0 = [I 0; 0 I], c0 = [x0; u0]; the equality residual ends with u_0 - u0;
    initial_control is required, and problem_params may set it."""
    B = 3
    u0 = torch.tensor([[0.1, -0.2], [0.0, 0.3], [0.5, 0.5]], dtype=torch.float64)
    prob = configs.config1(B=B, seed=5, constrain_initial_control=True, initial_control=u0)
    A0, c0 = prob.initial_equality()
    assert A0.shape == (B, 6, 6) and torch.equal(A0[0], torch.eye(6, dtype=torch.float64))
    assert torch.equal(c0, torch.cat([prob.x0, u0], dim=1))
    qp = prob.build_qp(*prob.initial_guess())
    assert qp.dims[4] == 6
    s, u = prob.initial_guess()
    h = prob.equality_residuals(s, u)
    assert h.shape == (B, 21 * 4 + 2)
    assert torch.equal(h[:, -2:], u[:, 0] - u0)
    assert torch.equal(h[:, :4], s[:, 0] - prob.x0)
    assert set(prob.problem_params) >= {"initial_state", "initial_control"}
    other = prob.with_params({"initial_control": torch.zeros(2, dtype=torch.float64)})
    assert torch.equal(other.initial_equality()[1][:, 4:], torch.zeros((B, 2), dtype=torch.float64))
    assert torch.equal(prob.u0, u0)  # the original is untouched
    with pytest.raises(ValueError, match="initial_control must be provided"):
        configs.config1(B=B, seed=5, constrain_initial_control=True)
    with pytest.raises(ValueError, match="initial_control has shape"):
        configs.config1(B=B, seed=5, constrain_initial_control=True, initial_control=torch.zeros(3))
    plain = configs.config1(B=B, seed=5)
    assert plain.initial_equality()[0].shape == (B, 4, 6)
    assert plain.equality_residuals(s, u).shape == (B, 21 * 4)


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


def test_fused_merit_terms_are_a_gpu_form():
    """QuadraticTrackingOCP.merit_terms has no CPU path: off the GPU it
    returns None and the line search evaluates the torch forms."""
    from turbompc_amd.problems import configs

    prob = configs.config1(B=2)
    s, c = prob.initial_guess()
    assert prob.merit_terms(s, c, None) is None
