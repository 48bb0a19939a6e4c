"""Robustness of the device solve: determinism and non-finite detection.

Determinism (reference: tests/cuda/backends/test_admm_math_cuda_vs_python.py:195-215,
the fused kernel run twice agrees to 1e-12): the benchmark's SQP solve and a
PCG solve, run twice on the same inputs, must agree bit for bit.  No kernel
uses atomics or order-dependent reductions across launches.

Non-finite detection: the ADMM entry points set TMPC_ITERS_NONFINITE in
iters_out for a problem whose output state holds a NaN or an infinity.  A NaN
planted in one problem's data must mark exactly that problem (the problems of a
batch never share arithmetic), on every kernel path, and leave the iteration
counts intact.
"""
import copy

import pytest
import torch

from helpers import random_qp
from turbompc_amd import _lib
from turbompc_amd.problems import configs
from turbompc_amd.problems.quadrotor import make_quadrotor_config
from turbompc_amd.solvers.admm.admm import ADMMSolver
from turbompc_amd.solvers.linear_systems_solvers.backends import AdmmBackend
from turbompc_amd.solvers.qp_data import QPCostBlocks, QPData
from turbompc_amd.solvers.qp_utils import ZShape
from turbompc_amd.solvers.turbompc_solver import DEFAULT_SOLVER_PARAMS, TurboMPCSolver

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _bench_params(n_sqp=5, admm_iters=20):
    p = copy.deepcopy(DEFAULT_SOLVER_PARAMS)
    p["num_sqp_iteration_max"] = n_sqp
    p["tol_convergence"] = 0.0
    p["admm"]["max_iter"] = admm_iters
    p["admm"]["adapt_rho_every"] = 0
    p["admm"]["relaxation_parameter"] = 1.0
    return p


def test_benchmark_solve_is_bitwise_reproducible():
    prob = make_quadrotor_config(B=4096, seed=0, dtype=torch.float32, device=DEV)
    solver = TurboMPCSolver(prob, _bench_params())
    a = solver.solve(solver.initial_guess())
    b = solver.solve(solver.initial_guess())
    torch.cuda.synchronize()
    assert torch.equal(a.states, b.states) and torch.equal(a.controls, b.controls)
    for fa, fb in zip(a.admm_state, b.admm_state):
        assert torch.equal(fa, fb)
    assert torch.equal(a.admm_iters, b.admm_iters)
    assert not bool(a.nonfinite.any())


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_pcg_solve_is_bitwise_reproducible(dtype):
    prob = configs.config2(B=256, seed=0).to(DEV, dtype)
    qp = prob.build_qp(*prob.initial_guess())
    B, T, n, nx, n0, m = qp.dims
    solver = ADMMSolver(ZShape(T - 1, nx, n - nx), {"max_iter": 50, "tol_epsilon": 1e-6}, sigma=1e-6, max_iter=20,
                        eps_abs=1e-9, eps_rel=1e-9, check_termination_every=25, adapt_rho_every=0,
                        admm_backend=AdmmBackend.HIP_PCG)
    runs = [solver.solve(qp, solver.initial_state(qp, rho_bar=0.1)) for _ in range(2)]
    torch.cuda.synchronize()
    (_, sa, xa), (_, sb, xb) = runs
    for fa, fb in zip(xa, xb):
        assert torch.equal(fa, fb)
    assert torch.equal(sa.num_pcg_iters, sb.num_pcg_iters)


def _poisoned(qp: QPData, b: int) -> QPData:
    q = qp.cost.q.clone()
    q[b, 2, 1] = float("nan")
    return QPData(cost=QPCostBlocks(qp.cost.D, qp.cost.E, q), eq=qp.eq, ineq=qp.ineq)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("path", ["stream", "generic", "pcg"])
def test_nonfinite_flag_marks_exactly_the_poisoned_problem(dtype, path):
    B, T, n, nx, m = 7, 9, 6, 4, 2  # nx + m <= n: the streaming kernel's shape
    qp = random_qp(B, T, n, nx, m, seed=5, std=True, diag=True).to(DEV, dtype)
    bad = 4
    qp = _poisoned(qp, bad)
    flags = _lib.FLAG_GENERIC_KERNEL if path == "generic" else 0
    backend = AdmmBackend.HIP_PCG if path == "pcg" else AdmmBackend.HIP_DIRECT
    solver = ADMMSolver(ZShape(T - 1, nx, n - nx), {"max_iter": 20, "tol_epsilon": 1e-8}, sigma=1e-6, max_iter=12,
                        eps_abs=1e-30, eps_rel=1e-30, check_termination_every=5, adapt_rho_every=0,
                        admm_backend=backend, kernel_flags=flags, diag_cost=True, std_dynamics=True)
    print(f"non-finite flag: path {path}, {dtype}, NaN in q of problem {bad}", flush=True)
    (_, _), stats, st = solver.solve(qp, solver.initial_state(qp, rho_bar=0.1))
    torch.cuda.synchronize()
    expect = torch.zeros(B, dtype=torch.bool)
    expect[bad] = True
    assert torch.equal(stats.nonfinite.cpu(), expect)
    # counts intact under the flag bit; a NaN residual passes the termination
    # test (NaN > eps is false), so the poisoned problem may stop early, as the
    # reference's loop would
    good = ~expect.to(stats.num_iter.device)
    assert torch.all(stats.num_iter[good] == 12) and torch.all(stats.num_iter >= 0)
    finite = torch.stack([torch.isfinite(t).flatten(1).all(1) for t in (st.x_blocks, st.y_f_dyn, st.y_g)]).all(0)
    assert torch.equal(~finite.cpu(), expect)  # the flag says what the state shows


def test_nonfinite_flag_reaches_the_sqp_solution():
    prob = make_quadrotor_config(B=6, seed=2, dtype=torch.float32, device=DEV)
    wu = prob.wu.clone()
    wu[1, 0] = float("inf")
    solver = TurboMPCSolver(prob.with_weights({"weights_penalization_control_squared": wu}), _bench_params(3, 10))
    sol = solver.solve(solver.initial_guess())
    torch.cuda.synchronize()
    assert sol.nonfinite.tolist() == [False, True, False, False, False, False]
    assert bool(torch.isfinite(sol.states[[0, 2, 3, 4, 5]]).all())


def test_fill_zero_entry_point():
    """tmpc_fill_zero (a kernel, no memset node): zeroes exactly the words asked for."""
    lib = _lib.load()
    x = torch.full((1000,), 7.0, dtype=torch.float32, device=DEV)
    st = lib.tmpc_fill_zero(_lib.stream_handle(x.device), _lib.ptr(x), 999 * 4)
    assert st == 0
    torch.cuda.synchronize()
    assert bool((x[:999] == 0).all()) and float(x[999]) == 7.0
