"""GPU parity of the fused ADMM (direct and PCG Schur solves), the adjoint KKT
and the quadrotor linearization against the CPU oracle, through the C ABI.

Parity protocol (fixed iteration counts, adapt_rho_every = 0): fp64 must match
the fp64 oracle to 1e-9 (normwise relative); fp32 must match the fp64 oracle to
1e-4.  The fp32 kernels factor in fp64, so they sit closer to the fp64 result
than the fp32 oracle does (quadrotor QP states: 2.5e-5 against the fp32
oracle's 8.0e-5).

Adaptive rho is tested separately with a looser bar: the rho candidate
rho * sqrt(r_p / r_d) is a ratio of residual norms that cancel, so two correct
implementations summing in different orders move rho by ~1e-9 relative and the
iterates after the change by up to ~1e-6 (measured: oracle vs GPU rho differ by
2e-9, states by 4e-7 one iteration later).
"""
import dataclasses

import numpy as np
import pytest
import torch

import oracle
from helpers import TOL, np_qp, random_qp, rel_err, soften, zero_state
from turbompc_amd import _lib
from turbompc_amd.problems import configs
from turbompc_amd.problems.quadrotor import QUAD_PARAMS, make_quadrotor_config
from turbompc_amd.solvers.admm.admm import ADMMSolver, ADMMState
from turbompc_amd.solvers.backward.backward_kkt_hip import solve_backward_kkt_hip
from turbompc_amd.solvers.linear_systems_solvers.backends import AdmmBackend
from turbompc_amd.solvers.qp_utils import ZShape

pytestmark = pytest.mark.gpu
DEV = "cuda"
FIELDS = ("x_blocks", "z_g", "y_g", "y_f_0", "y_f_dyn", "xi_g", "rho_bar")


def _solver(qp, cfg, backend=AdmmBackend.HIP_DIRECT, **kw):
    B, T, n, nx, n0, m = qp.dims
    return ADMMSolver(
        ZShape(T - 1, nx, n - nx),
        {"max_iter": cfg.pcg_max_iter, "tol_epsilon": cfg.pcg_eps},
        sigma=cfg.sigma, max_iter=cfg.max_iter, eps_abs=cfg.eps_abs, eps_rel=cfg.eps_rel, rho_min=cfg.rho_min,
        rho_max=cfg.rho_max, check_termination_every=cfg.check_every, adapt_rho_every=cfg.adapt_rho_every,
        adaptive_rho_tolerance=cfg.adaptive_rho_tolerance, rho_f_factor=cfg.rho_f_factor, admm_backend=backend,
        **kw,
    )


def _state_to_dev(st, dtype):
    return ADMMState(**{k: torch.as_tensor(np.asarray(getattr(st, k)), dtype=dtype, device=DEV) for k in FIELDS})


def _run_pair(qp, cfg, dtype, backend=AdmmBackend.HIP_DIRECT, rho0=0.1, schur="direct", **kw):
    st0 = zero_state(qp, rho0)
    ref, it_ref, pcg_ref = oracle.admm_solve(qp, st0, cfg, schur=schur, dtype=np.float64)
    qpd = qp.to(DEV, dtype)
    solver = _solver(qp, cfg, backend, **kw)
    (_, _), stats, out = solver.solve(qpd, _state_to_dev(st0, dtype), alpha=cfg.alpha,
                                      slack_weight=qpd.ineq.slack_penalization_weight)
    torch.cuda.synchronize()
    return ref, it_ref, pcg_ref, out, stats


def _oracle_full_batch(qp, cfg, rho0=0.1):
    """The fp64 oracle on a whole device batch (the same fp32-valued inputs)."""
    qc = qp.to("cpu", torch.float64)
    ref, it_ref, _ = oracle.admm_solve(qc, zero_state(qc, rho0), cfg, dtype=np.float64)
    return ref, it_ref


def _assert_batch_matches_oracle(name, out, ref, tol):
    for k in ("x_blocks", "y_f_dyn", "y_g", "z_g", "y_f_0"):
        e = rel_err(getattr(out, k), getattr(ref, k))
        print(f"{name} {k}: rel err vs fp64 oracle {e:.2e}")
        assert e < tol, (name, k, e)


def _assert_state_close(out, ref, tol):
    for k in FIELDS:
        a, b = getattr(out, k), getattr(ref, k)
        if np.asarray(b).size:
            assert rel_err(a, b) < tol, (k, rel_err(a, b))


@pytest.mark.parametrize("std", [True, False])
@pytest.mark.parametrize("shape", [(9, 21, 6, 4, 2), (7, 11, 17, 13, 4), (5, 13, 9, 6, 11), (4, 8, 5, 3, 2), (3, 6, 4, 2, 0)])
def test_admm_direct_fp64_fixed_iterations(std, shape):
    B, T, n, nx, m = shape
    qp = random_qp(B, T, n, nx, m, seed=41, std=std)
    cfg = oracle.OracleCfg(max_iter=30, check_every=25, adapt_rho_every=0, sigma=1e-6, eps_abs=1e-9,
                           eps_rel=1e-9, rho_f_factor=1000.0, alpha=1.0)
    ref, it_ref, _, out, stats = _run_pair(qp, cfg, torch.float64)
    np.testing.assert_array_equal(stats.num_iter.cpu().numpy(), it_ref)
    _assert_state_close(out, ref, 1e-9)


# soft constraints (slack variables): generic kernel with general and
# explicit-integrator structure, streaming kernel with 1 and 2 problems per
# wavefront; the residual sweep (with its slack terms) runs every 4 iterations
@pytest.mark.parametrize("kernel", ["generic", "generic-std", "stream-1", "stream-2"])
def test_admm_slack_fp64_fixed_iterations(kernel):
    if kernel.startswith("stream"):
        shape, flags, std = (13, 21, 6, 4, 2), _lib.flag_stream_p(int(kernel[-1])), True
    else:
        shape, flags, std = (5, 13, 9, 6, 11), _lib.FLAG_GENERIC_KERNEL, kernel.endswith("std")
    B, T, n, nx, m = shape
    qp = soften(random_qp(B, T, n, nx, m, seed=61, std=std), 20.0, shrink=0.3)
    cfg = oracle.OracleCfg(max_iter=30, check_every=4, adapt_rho_every=0, sigma=1e-6, eps_abs=1e-12,
                           eps_rel=1e-12, rho_f_factor=1000.0, alpha=1.6)
    ref, it_ref, _, out, stats = _run_pair(qp, cfg, torch.float64, use_slack=True, kernel_flags=flags)
    np.testing.assert_array_equal(stats.num_iter.cpu().numpy(), it_ref)
    assert float(np.max(np.abs(ref.xi_g))) > 1e-3  # rows are softened
    _assert_state_close(out, ref, 1e-9)


def test_admm_slack_converges_with_termination_and_adaptive_rho():
    qp = soften(random_qp(9, 9, 6, 4, 3, seed=62, std=True), 5.0, shrink=0.3)
    cfg = oracle.OracleCfg(max_iter=300, check_every=2, adapt_rho_every=4, sigma=1e-6, eps_abs=1e-6, eps_rel=1e-6,
                           rho_f_factor=50.0, alpha=1.0, adaptive_rho_tolerance=1.5)
    ref, it_ref, _, out, stats = _run_pair(qp, cfg, torch.float64, use_slack=True)
    np.testing.assert_array_equal(stats.num_iter.cpu().numpy(), it_ref)
    assert np.all(it_ref < cfg.max_iter)
    assert rel_err(out.rho_bar, ref.rho_bar) < 1e-7
    _assert_state_close(out, ref, 1e-5)


@pytest.mark.parametrize("alpha", [1.0, 1.6])
def test_admm_direct_fp64_adaptive_rho_and_termination(alpha):
    # residual checks every 2 iterations, rho adapted every 4: per-problem
    # termination and refactorizations inside one call
    qp = random_qp(11, 9, 6, 4, 3, seed=42, std=False)
    cfg = oracle.OracleCfg(max_iter=200, check_every=2, adapt_rho_every=4, sigma=1e-6, eps_abs=1e-6, eps_rel=1e-6,
                           rho_f_factor=50.0, alpha=alpha, adaptive_rho_tolerance=1.5)
    ref, it_ref, _, out, stats = _run_pair(qp, cfg, torch.float64)
    np.testing.assert_array_equal(stats.num_iter.cpu().numpy(), it_ref)
    assert len(set(it_ref.tolist())) > 1  # problems stop at different iterations
    assert rel_err(out.rho_bar, ref.rho_bar) < 1e-7
    assert np.any(ref.rho_bar != 0.1)  # rho did adapt
    _assert_state_close(out, ref, 1e-5)


def test_admm_direct_config1_fp32():
    prob = configs.config1(B=64, seed=0)
    qp = prob.build_qp(*prob.initial_guess())
    cfg = oracle.OracleCfg(max_iter=50, check_every=25, adapt_rho_every=0, sigma=1e-6, eps_abs=1e-9, eps_rel=1e-9,
                           rho_f_factor=1000.0, alpha=1.0)
    ref, it_ref, _, out, stats = _run_pair(qp, cfg, torch.float32)
    for k in ("x_blocks", "y_f_dyn", "y_g", "z_g", "y_f_0"):
        e = rel_err(getattr(out, k), getattr(ref, k))
        print(f"config1 fp32 {k}: rel err vs fp64 oracle {e:.2e}")
        assert e < TOL[torch.float32], (k, e)


def test_admm_direct_quadrotor_qp_fp32_and_fp64():
    prob = make_quadrotor_config(B=8, seed=0, dtype=torch.float64, device=DEV)
    qp = prob.build_qp(*prob.initial_guess()).to("cpu")
    cfg = oracle.OracleCfg(max_iter=20, check_every=25, adapt_rho_every=0, sigma=1e-6, eps_abs=1e-9, eps_rel=1e-9,
                           rho_f_factor=1000.0, alpha=1.0)
    ref, it_ref, _, out64, _ = _run_pair(qp, cfg, torch.float64)
    _assert_state_close(out64, ref, 1e-9)
    _, _, _, out32, _ = _run_pair(qp, cfg, torch.float32)
    for k in ("x_blocks", "y_f_dyn", "y_g"):
        e = rel_err(getattr(out32, k), getattr(ref, k))
        print(f"quadrotor QP fp32 {k}: rel err vs fp64 oracle {e:.2e}")
        assert e < TOL[torch.float32], (k, e)


def test_admm_direct_warm_start_and_in_place_state():
    qp = random_qp(6, 10, 6, 4, 3, seed=43, std=True)
    cfg = oracle.OracleCfg(max_iter=15, check_every=5, adapt_rho_every=0, sigma=1e-6, eps_abs=1e-12, eps_rel=1e-12,
                           rho_f_factor=100.0, alpha=1.6)
    st0 = zero_state(qp, 0.1)
    mid, _, _ = oracle.admm_solve(qp, st0, cfg)
    ref, it_ref, _ = oracle.admm_solve(qp, mid, cfg)
    solver = _solver(qp, cfg)
    qpd = qp.to(DEV, torch.float64)
    _, _, s1 = solver.solve(qpd, _state_to_dev(st0, torch.float64), alpha=1.6)
    _, stats, s2 = solver.solve(qpd, s1, alpha=1.6)
    np.testing.assert_array_equal(stats.num_iter.cpu().numpy(), it_ref)
    _assert_state_close(s2, ref, 1e-9)


# PCG Schur solve on explicit-integrator QPs: "dpp" is the one-launch kernel
# with a stage per 16-lane row (admm_pcg_dpp_kernel), "lds" the one-launch
# kernel with the problem resident in LDS (admm_pcg_lds_kernel), "chunk" the
# kernel that streams S and Phiinv (admm_pcg_chunk_kernel).
PCG_KERNELS = {"dpp": _lib.flag_pcg_kernel(_lib.PCG_KERNEL_DPP), "lds": _lib.flag_pcg_kernel(_lib.PCG_KERNEL_LDS),
               "chunk": _lib.FLAG_GENERIC_KERNEL}


@pytest.mark.parametrize("kernel", list(PCG_KERNELS))
def test_admm_pcg_config2_fp64(kernel):
    prob = configs.config2(B=6, seed=0)
    qp = prob.build_qp(*prob.initial_guess())
    cfg = oracle.OracleCfg(max_iter=12, check_every=25, adapt_rho_every=0, sigma=1e-6, eps_abs=1e-9, eps_rel=1e-9,
                           rho_f_factor=1000.0, alpha=1.0, pcg_eps=1e-6, pcg_max_iter=50)
    ref, it_ref, pcg_ref, out, stats = _run_pair(qp, cfg, torch.float64, backend=AdmmBackend.HIP_PCG, schur="pcg",
                                                 kernel_flags=PCG_KERNELS[kernel])
    np.testing.assert_array_equal(stats.num_iter.cpu().numpy(), it_ref)
    # the tolerance stop can flip by one iteration between two summation orders
    assert np.all(np.abs(stats.num_pcg_iters.sum(1).cpu().numpy() - pcg_ref) <= 2)
    _assert_state_close(out, ref, 1e-6)


@pytest.mark.parametrize("kernel", list(PCG_KERNELS))
def test_admm_pcg_fixed_pcg_iterations_fp64(kernel):
    # pcg_eps = 0 runs exactly pcg_max_iter PCG iterations per ADMM iteration
    prob = configs.config2(B=5, seed=1)
    qp = prob.build_qp(*prob.initial_guess())
    cfg = oracle.OracleCfg(max_iter=6, check_every=25, adapt_rho_every=0, sigma=1e-6, eps_abs=1e-9, eps_rel=1e-9,
                           rho_f_factor=1000.0, alpha=1.0, pcg_eps=0.0, pcg_max_iter=6)
    ref, it_ref, pcg_ref, out, stats = _run_pair(qp, cfg, torch.float64, backend=AdmmBackend.HIP_PCG, schur="pcg",
                                                 kernel_flags=PCG_KERNELS[kernel])
    np.testing.assert_array_equal(stats.num_pcg_iters.sum(1).cpu().numpy(), pcg_ref)
    _assert_state_close(out, ref, 1e-9)


@pytest.mark.parametrize("kernel", list(PCG_KERNELS))
def test_admm_pcg_config2_fp32(kernel):
    """Config 2 in fp32 on the PCG backend, tolerance-stopped (pcg_eps 1e-6,
    at most 50 PCG iterations, as the workload specifies) against the fp64
    oracle."""
    prob = configs.config2(B=6, seed=0)
    qp = prob.build_qp(*prob.initial_guess())
    cfg = oracle.OracleCfg(max_iter=12, check_every=25, adapt_rho_every=0, sigma=1e-6, eps_abs=1e-9, eps_rel=1e-9,
                           rho_f_factor=1000.0, alpha=1.0, pcg_eps=1e-6, pcg_max_iter=50)
    ref, it_ref, pcg_ref, out, stats = _run_pair(qp, cfg, torch.float32, backend=AdmmBackend.HIP_PCG, schur="pcg",
                                                 kernel_flags=PCG_KERNELS[kernel])
    np.testing.assert_array_equal(stats.num_iter.cpu().numpy(), it_ref)
    assert np.all(np.abs(stats.num_pcg_iters.sum(1).cpu().numpy() - pcg_ref) <= 2)
    for k in ("x_blocks", "y_f_dyn", "y_g"):
        e = rel_err(getattr(out, k), getattr(ref, k))
        print(f"config2 PCG fp32 ({kernel}) {k}: rel err vs fp64 oracle {e:.2e}")
        assert e < TOL[torch.float32], (k, e)


@pytest.mark.parametrize("kernel", list(PCG_KERNELS))
def test_admm_pcg_fixed_pcg_iterations_fp32(kernel):
    prob = configs.config2(B=5, seed=1)
    qp = prob.build_qp(*prob.initial_guess())
    cfg = oracle.OracleCfg(max_iter=6, check_every=25, adapt_rho_every=0, sigma=1e-6, eps_abs=1e-9, eps_rel=1e-9,
                           rho_f_factor=1000.0, alpha=1.0, pcg_eps=0.0, pcg_max_iter=6)
    ref, it_ref, pcg_ref, out, stats = _run_pair(qp, cfg, torch.float32, backend=AdmmBackend.HIP_PCG, schur="pcg",
                                                 kernel_flags=PCG_KERNELS[kernel])
    np.testing.assert_array_equal(stats.num_pcg_iters.sum(1).cpu().numpy(), pcg_ref)
    for k in ("x_blocks", "y_f_dyn", "y_g"):
        e = rel_err(getattr(out, k), getattr(ref, k))
        print(f"config2 PCG fixed-count fp32 ({kernel}) {k}: rel err vs fp64 oracle {e:.2e}")
        assert e < TOL[torch.float32], (k, e)


# every n the one-launch kernels are built for, with m = 0, n0 < nx, a single
# stage pair and 1024 = 16 T (a full workgroup for the row-broadcast kernel);
# fixed PCG counts (pcg_eps = 0) so that the iteration is fully determined,
# residual checks every 4 iterations
@pytest.mark.parametrize("shape", [(5, 21, 6, 4, 2, 4), (4, 13, 9, 6, 11, 6), (3, 9, 16, 12, 16, 12),
                                   (3, 7, 17, 13, 4, 13), (2, 64, 16, 12, 0, 12), (4, 2, 6, 4, 3, 2)])
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("kernel", ["dpp", "lds"])
def test_admm_pcg_one_launch_kernel_shapes(kernel, shape, dtype):
    B, T, n, nx, m, n0 = shape
    if kernel == "dpp" and n > 16:
        pytest.skip("the row-broadcast kernel covers n <= 16")
    qp = random_qp(B, T, n, nx, m, seed=71, std=True, n0=n0)
    cfg = oracle.OracleCfg(max_iter=9, check_every=4, adapt_rho_every=0, sigma=1e-6, eps_abs=1e-12, eps_rel=1e-12,
                           rho_f_factor=100.0, alpha=1.6, pcg_eps=0.0, pcg_max_iter=5)
    ref, it_ref, pcg_ref, out, stats = _run_pair(qp, cfg, dtype, backend=AdmmBackend.HIP_PCG, schur="pcg",
                                                 kernel_flags=PCG_KERNELS[kernel])
    np.testing.assert_array_equal(stats.num_iter.cpu().numpy(), it_ref)
    np.testing.assert_array_equal(stats.num_pcg_iters.sum(1).cpu().numpy(), pcg_ref)
    _assert_state_close(out, ref, 1e-9 if dtype == torch.float64 else TOL[torch.float32])


@pytest.mark.parametrize("kernel", list(PCG_KERNELS))
def test_admm_pcg_slack_fp64(kernel):
    qp = soften(random_qp(5, 13, 9, 6, 11, seed=72, std=True), 20.0, shrink=0.3)
    cfg = oracle.OracleCfg(max_iter=12, check_every=4, adapt_rho_every=0, sigma=1e-6, eps_abs=1e-12, eps_rel=1e-12,
                           rho_f_factor=100.0, alpha=1.6, pcg_eps=0.0, pcg_max_iter=8)
    ref, it_ref, pcg_ref, out, stats = _run_pair(qp, cfg, torch.float64, backend=AdmmBackend.HIP_PCG, schur="pcg",
                                                 use_slack=True, kernel_flags=PCG_KERNELS[kernel])
    np.testing.assert_array_equal(stats.num_pcg_iters.sum(1).cpu().numpy(), pcg_ref)
    assert float(np.max(np.abs(ref.xi_g))) > 1e-3  # rows are softened
    _assert_state_close(out, ref, 1e-9)


@pytest.mark.parametrize("kernel", list(PCG_KERNELS))
def test_admm_pcg_adaptive_rho_and_termination(kernel):
    # residual checks every 2 iterations, rho adapted every 4: per-problem
    # termination and S / Phiinv rebuilt inside one call; PCG run to its
    # absolute floor so that the PCG solve equals the direct one
    qp = random_qp(11, 9, 6, 4, 3, seed=43, std=True)
    cfg = oracle.OracleCfg(max_iter=200, check_every=2, adapt_rho_every=4, sigma=1e-6, eps_abs=1e-6, eps_rel=1e-6,
                           rho_f_factor=50.0, alpha=1.6, adaptive_rho_tolerance=1.5, pcg_eps=1e-26, pcg_max_iter=200)
    ref, it_ref, _, out, stats = _run_pair(qp, cfg, torch.float64, backend=AdmmBackend.HIP_PCG, schur="pcg",
                                           kernel_flags=PCG_KERNELS[kernel])
    np.testing.assert_array_equal(stats.num_iter.cpu().numpy(), it_ref)
    assert len(set(it_ref.tolist())) > 1  # problems stop at different iterations
    assert np.any(ref.rho_bar != 0.1)  # rho did adapt
    # each PCG solve stops at |eta| < 1e-12 rather than at the exact solution,
    # and rho (a ratio of residual norms) carries that error: measured 1.1e-7
    # (chunk kernel) against the oracle
    assert rel_err(out.rho_bar, ref.rho_bar) < 1e-6
    _assert_state_close(out, ref, 1e-5)


def test_admm_pcg_matches_direct_when_tight():
    qp = random_qp(4, 12, 6, 4, 3, seed=44, std=True)
    cfg = oracle.OracleCfg(max_iter=10, check_every=25, adapt_rho_every=0, sigma=1e-6, eps_abs=1e-9, eps_rel=1e-9,
                           rho_f_factor=100.0, alpha=1.0, pcg_eps=1e-26, pcg_max_iter=400)
    ref, _, _ = oracle.admm_solve(qp, zero_state(qp, 0.1), cfg, schur="direct")
    _, _, _, out, _ = _run_pair(qp, cfg, torch.float64, backend=AdmmBackend.HIP_PCG, schur="pcg")
    # PCG stops once |eta| < 1e-12 (absolute floor of pcg_primal.py:113)
    assert rel_err(out.x_blocks, ref.x_blocks) < 1e-6


def test_adjoint_kkt_matches_dense_oracle_fp64():
    prob = configs.config5(B=3, seed=0)
    qp = prob.build_qp(*prob.initial_guess())
    rng = np.random.default_rng(5)
    sign = rng.choice([-1.0, 0.0, 1.0], size=tuple(qp.ineq.l.shape), p=[0.2, 0.6, 0.2])
    G = qp.ineq.G * torch.tensor(sign).unsqueeze(-1)
    qb = qp.replace_ineq(G=G).replace_cost(q=torch.tensor(rng.standard_normal(tuple(qp.cost.q.shape))))
    dz_ref, mult_ref = oracle.adjoint_kkt(qb)
    dz, mult = solve_backward_kkt_hip(qb.to(DEV, torch.float64))
    assert rel_err(dz, dz_ref) < 1e-9
    assert rel_err(mult, mult_ref) < 1e-9


# the rows-in-lanes KKT factorization and solve (n <= 16, nb <= 32) against the
# dense oracle and the generic kernels: config 5 (nb = 18), config 4 (nb = 26),
# and random QPs with n = 12 (nb = 24) and with E != 0 (the coupling block's E part)
@pytest.mark.parametrize("case", ["config5", "config4", "random12", "random-E"])
def test_adjoint_kkt_rows_kernels_match_generic_and_oracle(case):
    rng = np.random.default_rng(7)
    if case == "config5":
        prob = configs.config5(B=5, seed=1)
        qp = prob.build_qp(*prob.initial_guess())
    elif case == "config4":
        prob = configs.config4(B=5, seed=1).to(DEV, torch.float64)  # its linearization runs on the device
        qp = prob.build_qp(*prob.initial_guess()).to("cpu", torch.float64)
    elif case == "random12":
        # n0 + m <= n: the initial-state rows and the active rows of stage 0
        # both sit on z_0 alone, and more of them than n makes the multipliers
        # non-unique (dz stays unique)
        qp = random_qp(5, 9, 12, 8, 4, seed=91, std=True)
    else:
        qp = random_qp(5, 9, 9, 6, 3, seed=92, std=False)
    sign = rng.choice([-1.0, 0.0, 1.0], size=tuple(qp.ineq.l.shape), p=[0.3, 0.4, 0.3])
    if case == "config4":
        # box rows only: the obstacle rows act on the position, which the
        # initial-state rows already pin at stage 0 (a rank-deficient KKT)
        sign[..., prob.num_box_constraints:] = 0.0
    G = qp.ineq.G * torch.tensor(sign).unsqueeze(-1)
    qb = qp.replace_ineq(G=G).replace_cost(q=torch.tensor(rng.standard_normal(tuple(qp.cost.q.shape))))
    dz_ref, mult_ref = oracle.adjoint_kkt(qb)
    qd = qb.to(DEV, torch.float64)
    # four refinement rounds: with this many active rows two rounds against
    # the shifted factor leave about 2e-9 in the multipliers (either kernel)
    dz, mult = solve_backward_kkt_hip(qd, refine_steps=4)
    dz_g, mult_g = solve_backward_kkt_hip(qd, refine_steps=4, kernel_flags=_lib.FLAG_GENERIC_KERNEL)
    errs = {k: rel_err(a, b) for k, (a, b) in {"dz": (dz, dz_ref), "mult": (mult, mult_ref), "dz generic": (dz_g, dz_ref),
                                             "mult generic": (mult_g, mult_ref)}.items()}
    print(case, {k: f"{v:.2e}" for k, v in errs.items()})
    assert all(v < 1e-10 for v in errs.values()), errs
    assert not torch.equal(dz, dz_g)  # two different factorizations ran


# the rows-in-lanes kernels with two and three problems per wavefront (the
# batch sets how many: ceil(B / 1024)), last wavefront partly filled, in the
# three (NC, NBC) forms; T = 6 keeps the dense oracle cheap at B = 2049
@pytest.mark.parametrize("shape", [(2049, 9, 6, 3), (1100, 9, 6, 3), (1100, 9, 6, 14), (2049, 12, 8, 4)])
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_adjoint_kkt_rows_kernels_packed_wavefronts(shape, dtype):
    B, n, nx, m = shape
    rng = np.random.default_rng(11)
    qp = random_qp(B, 6, n, nx, m, seed=94, std=False)
    # at most n - nx - 1 active rows per stage: each stage's controls leave
    # n - nx directions free, so the multipliers stay unique and the batch's
    # KKT condition numbers stay below about 1e6 (n - nx active rows reach
    # 1e9 in a batch this size)
    k = rng.integers(0, n - nx, size=(B, 6))
    order = np.argsort(rng.random((B, 6, m)), axis=-1)
    sign = np.where(order < k[..., None], rng.choice([-1.0, 1.0], size=(B, 6, m)), 0.0)
    G = qp.ineq.G * torch.tensor(sign).unsqueeze(-1)
    qb = qp.replace_ineq(G=G).replace_cost(q=torch.tensor(rng.standard_normal(tuple(qp.cost.q.shape))))
    dz_ref, mult_ref = oracle.adjoint_kkt(qb)
    qd = qb.to(DEV, dtype)
    dz, mult = solve_backward_kkt_hip(qd, refine_steps=4)
    dz_g, mult_g = solve_backward_kkt_hip(qd, refine_steps=4, kernel_flags=_lib.FLAG_GENERIC_KERNEL)
    tol = 1e-9 if dtype == torch.float64 else 1e-4
    errs = {"dz": rel_err(dz, dz_ref), "mult": rel_err(mult, mult_ref), "dz generic": rel_err(dz_g, dz_ref),
            "mult generic": rel_err(mult_g, mult_ref)}
    errs["rows vs generic"] = rel_err(dz, dz_g)
    print(shape, dtype, {k: f"{v:.2e}" for k, v in errs.items()})
    # max-abs errors over the whole batch: every problem counts, the last
    # (partly filled) wavefront's included
    assert all(v < tol for v in errs.values()), errs


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_quadrotor_linearization_matches_complex_step(dtype):
    prob = make_quadrotor_config(B=16, seed=1, dtype=dtype, device=DEV)
    g = torch.Generator().manual_seed(3)
    st = (prob.initial_guess()[0].cpu().double() + 0.2 * torch.randn(prob.initial_guess()[0].shape, generator=g))
    ct = torch.rand((16, 41, 4), generator=g, dtype=torch.float64) * 4.0
    Am, c = prob.dynamics_blocks(st.to(DEV, dtype), ct.to(DEV, dtype))
    xu = torch.cat([st[:, :-1], ct[:, :-1]], dim=-1).numpy().reshape(-1, 17)
    f, J = oracle.quadrotor_rk4_jac(xu, prob.dt, QUAD_PARAMS)
    Jr = J.reshape(16, 40, 13, 17)
    cr = (-f + np.einsum("kij,kj->ki", J, xu)).reshape(16, 40, 13)
    tol = 1e-12 if dtype == torch.float64 else 1e-5
    assert rel_err(Am, Jr) < tol
    assert rel_err(c, cr) < (1e-11 if dtype == torch.float64 else 1e-5)
    # the same iterate packed as z rows [x; u] (an ADMM state's layout): read in
    # place through the row strides, the blocks are the same bit for bit
    z = torch.cat([st, ct], dim=-1).to(DEV, dtype)
    zs, zc = z[..., :13], z[..., 13:]
    assert not zs.is_contiguous() and zs.stride(1) == 17
    Am2, c2 = prob.dynamics_blocks(zs, zc)
    assert torch.equal(Am2, Am) and torch.equal(c2, c)
    # rows that are not evenly strided are copied first; wrong shapes are refused
    Am3, c3 = prob.dynamics_blocks(st.to(DEV, dtype).transpose(0, 1).contiguous().transpose(0, 1), ct.to(DEV, dtype))
    assert torch.equal(Am3, Am) and torch.equal(c3, c)
    with pytest.raises(ValueError, match="expected"):
        prob.dynamics_blocks(zs[:, :-1], zc[:, :-1])


# ---- streaming kernel (explicit-integrator structure, stage records) ---------
# B is chosen so that the last wavefront is partially filled for P = 2 and 3.

# "rows": the factorization with a problem per 16-lane row (the default);
# "groups": the lane-group factorization (TMPC_FLAG_FACTOR_GROUPS)
@pytest.mark.parametrize("factor", ["rows", "groups"])
@pytest.mark.parametrize("P", [1, 2, 3])
@pytest.mark.parametrize("shape", [(13, 21, 6, 4, 2), (8, 11, 17, 13, 4), (7, 13, 9, 6, 5), (5, 9, 16, 12, 0)])
def test_admm_stream_kernel_fp64_matches_oracle(P, shape, factor):
    B, T, n, nx, m = shape
    qp = random_qp(B, T, n, nx, m, seed=51, std=True)
    # residual pass every 3 iterations (no adaptation): exercises the
    # residual sweep without changing the fixed-iteration trajectory
    cfg = oracle.OracleCfg(max_iter=20, check_every=3, adapt_rho_every=0, sigma=1e-6, eps_abs=1e-12,
                           eps_rel=1e-12, rho_f_factor=1000.0, alpha=1.6)
    flags = _lib.flag_stream_p(P) | (_lib.FLAG_FACTOR_GROUPS if factor == "groups" else 0)
    ref, it_ref, _, out, stats = _run_pair(qp, cfg, torch.float64, kernel_flags=flags)
    np.testing.assert_array_equal(stats.num_iter.cpu().numpy(), it_ref)
    _assert_state_close(out, ref, 1e-9)


@pytest.mark.parametrize("alpha", [1.0, 1.6])
def test_admm_stream_kernel_adaptive_rho_and_termination(alpha):
    qp = random_qp(11, 9, 6, 4, 3, seed=42, std=True)
    cfg = oracle.OracleCfg(max_iter=200, check_every=2, adapt_rho_every=4, sigma=1e-6, eps_abs=1e-6, eps_rel=1e-6,
                           rho_f_factor=50.0, alpha=alpha, adaptive_rho_tolerance=1.5)
    ref, it_ref, _, out, stats = _run_pair(qp, cfg, torch.float64, kernel_flags=_lib.flag_stream_p(2))
    np.testing.assert_array_equal(stats.num_iter.cpu().numpy(), it_ref)
    assert len(set(it_ref.tolist())) > 1
    assert np.any(ref.rho_bar != 0.1)
    assert rel_err(out.rho_bar, ref.rho_bar) < 1e-7
    _assert_state_close(out, ref, 1e-5)


def test_admm_stream_kernel_matches_generic_on_bench_batch():
    # the benchmark's shapes at a batch that selects P = 2 with a partial last
    # wavefront: streaming and generic kernels run the same fp32 iteration
    B = 4099
    prob = make_quadrotor_config(B=B, seed=5, dtype=torch.float32, device=DEV)
    qp = prob.build_qp(*prob.initial_guess())
    cfg = oracle.OracleCfg(max_iter=20, check_every=25, adapt_rho_every=0, sigma=1e-6, eps_abs=1e-9, eps_rel=1e-9,
                           rho_f_factor=1000.0, alpha=1.0)
    outs = []
    for flags in (0, _lib.FLAG_GENERIC_KERNEL):
        solver = _solver(qp, cfg, kernel_flags=flags)
        st0 = solver.initial_state(qp, rho_bar=0.1)
        _, stats, out = solver.solve(qp, st0)
        outs.append((stats, out))
    torch.cuda.synchronize()
    (s_a, o_a), (s_b, o_b) = outs
    assert torch.equal(s_a.num_iter, s_b.num_iter)
    for k in ("x_blocks", "y_f_dyn", "y_g", "z_g", "y_f_0"):
        assert rel_err(getattr(o_a, k), getattr(o_b, k)) < TOL[torch.float32], k
    # and both against the fp64 oracle on the whole batch
    ref, it_ref = _oracle_full_batch(qp, cfg)
    np.testing.assert_array_equal(s_a.num_iter.cpu().numpy(), it_ref)
    _assert_batch_matches_oracle("config 3 B=4099 stream", o_a, ref, TOL[torch.float32])
    _assert_batch_matches_oracle("config 3 B=4099 generic", o_b, ref, TOL[torch.float32])


@pytest.mark.parametrize("P", [1, 2, 3])
@pytest.mark.parametrize("shape", [(13, 21, 6, 4, 2), (8, 11, 17, 13, 4), (7, 13, 9, 6, 3)])
def test_admm_stream_kernel_structured_records_fp64_matches_oracle(P, shape):
    # diagonal D_t declared to the kernel: it then streams diag(D_t)
    B, T, n, nx, m = shape
    qp = random_qp(B, T, n, nx, m, seed=61, std=True, diag=True)
    cfg = oracle.OracleCfg(max_iter=20, check_every=3, adapt_rho_every=0, sigma=1e-6, eps_abs=1e-12,
                           eps_rel=1e-12, rho_f_factor=1000.0, alpha=1.6)
    ref, it_ref, _, out, stats = _run_pair(qp, cfg, torch.float64, kernel_flags=_lib.flag_stream_p(P),
                                           diag_cost=True)
    np.testing.assert_array_equal(stats.num_iter.cpu().numpy(), it_ref)
    _assert_state_close(out, ref, 1e-9)


# the wide form: n = 9 with more stacked rows than n (the obstacle workload's
# 6 + 11 rows), up to 17 row lanes per problem; 11 rows exercise the rows past
# the block that the column products read
@pytest.mark.parametrize("P", [1, 2, 3])
@pytest.mark.parametrize("shape", [(7, 13, 9, 6, 11), (10, 9, 9, 6, 5)])
@pytest.mark.parametrize("variant", ["dense", "diag", "slack-diag"])
def test_admm_stream_kernel_wide_rows_fp64_matches_oracle(P, shape, variant):
    B, T, n, nx, m = shape
    diag = variant.endswith("diag")
    qp = random_qp(B, T, n, nx, m, seed=71, std=True, diag=diag)
    kw = {"diag_cost": True} if diag else {}
    if variant.startswith("slack"):
        qp = soften(qp, 20.0, shrink=0.3)
        kw["use_slack"] = True
    cfg = oracle.OracleCfg(max_iter=20, check_every=3, adapt_rho_every=0, sigma=1e-6, eps_abs=1e-12,
                           eps_rel=1e-12, rho_f_factor=1000.0, alpha=1.6)
    ref, it_ref, _, out, stats = _run_pair(qp, cfg, torch.float64, kernel_flags=_lib.flag_stream_p(P), **kw)
    np.testing.assert_array_equal(stats.num_iter.cpu().numpy(), it_ref)
    _assert_state_close(out, ref, 1e-9)
    if variant.startswith("slack"):
        assert float(np.max(np.abs(ref.xi_g))) > 1e-6  # the soft rows are in play


def test_admm_stream_kernel_wide_rows_adaptive_rho_and_termination():
    qp = random_qp(11, 9, 9, 6, 11, seed=43, std=True, diag=True)
    cfg = oracle.OracleCfg(max_iter=200, check_every=2, adapt_rho_every=4, sigma=1e-6, eps_abs=1e-6, eps_rel=1e-6,
                           rho_f_factor=50.0, alpha=1.6, adaptive_rho_tolerance=1.5)
    ref, it_ref, _, out, stats = _run_pair(qp, cfg, torch.float64, kernel_flags=_lib.flag_stream_p(3),
                                           diag_cost=True)
    np.testing.assert_array_equal(stats.num_iter.cpu().numpy(), it_ref)
    assert len(set(it_ref.tolist())) > 1
    assert rel_err(out.rho_bar, ref.rho_bar) < 1e-7
    _assert_state_close(out, ref, 1e-5)


def test_admm_stream_kernel_wide_rows_match_generic_on_config4_batch():
    # config 4 at a batch that selects P = 2 with a partial last wavefront:
    # the wide streaming kernel and the generic kernel run the same fp32 iteration
    prob = configs.config4(B=4099, seed=2).to(DEV, torch.float32)
    qp = prob.build_qp(*prob.initial_guess())
    cfg = oracle.OracleCfg(max_iter=30, check_every=25, adapt_rho_every=0, sigma=1e-6, eps_abs=1e-9, eps_rel=1e-9,
                           rho_f_factor=1000.0, alpha=1.0)
    outs = []
    for flags in (0, _lib.FLAG_GENERIC_KERNEL):
        solver = _solver(qp, cfg, kernel_flags=flags, diag_cost=True)
        st0 = solver.initial_state(qp, rho_bar=0.1)
        _, stats, out = solver.solve(qp, st0)
        outs.append((stats, out))
    torch.cuda.synchronize()
    (s_a, o_a), (s_b, o_b) = outs
    assert torch.equal(s_a.num_iter, s_b.num_iter)
    for k in ("x_blocks", "y_f_dyn", "y_g", "z_g", "y_f_0"):
        assert rel_err(getattr(o_a, k), getattr(o_b, k)) < TOL[torch.float32], k
    assert not torch.equal(o_a.x_blocks, o_b.x_blocks)  # two different kernels ran
    ref, it_ref = _oracle_full_batch(qp, cfg)
    np.testing.assert_array_equal(s_a.num_iter.cpu().numpy(), it_ref)
    _assert_batch_matches_oracle("config 4 B=4099 wide stream", o_a, ref, TOL[torch.float32])
    _assert_batch_matches_oracle("config 4 B=4099 generic", o_b, ref, TOL[torch.float32])


# block widths outside {6, 9, 16, 17}: the streaming path rounds n up to the
# next width it is built for (n = 4 -> 6, 7 -> 9, 8 with 11 stacked rows -> the
# wide 9, 12 and 14 -> 16, 14 with 20 stacked rows -> the wide 16); the extra
# variables are decoupled dummies in the stage records and never reach the
# state.  (5, 9, 16, 12, 16) is the linear workload's widths (box constraints
# on all 16 variables): the wide 16 form, a half-wave per problem.
PADDED_SHAPES = [(9, 11, 4, 2, 2), (10, 13, 7, 4, 3), (7, 9, 8, 5, 6), (6, 9, 12, 8, 4), (5, 7, 14, 10, 5),
                 (5, 9, 16, 12, 16), (6, 7, 14, 10, 10)]


def _wide16(shape):
    _, _, n, nx, m = shape
    return nx + m > 16 and n > 9


def _gpu_solve(qp, cfg, dtype, **kw):
    qpd = qp.to(DEV, dtype)
    solver = _solver(qp, cfg, **kw)
    (_, _), stats, out = solver.solve(qpd, solver.initial_state(qpd, rho_bar=0.1), alpha=cfg.alpha)
    torch.cuda.synchronize()
    return stats, out


@pytest.mark.parametrize("P", [1, 2, 3])
@pytest.mark.parametrize("shape", PADDED_SHAPES)
@pytest.mark.parametrize("variant", ["dense", "diag", "groups"])
def test_admm_stream_kernel_padded_width_fp64_matches_oracle(P, shape, variant):
    if P == 3 and _wide16(shape):
        pytest.skip("three 32-lane groups do not fit a wavefront (the wide 16 form runs P = 1, 2)")
    B, T, n, nx, m = shape
    diag = variant == "diag"
    qp = random_qp(B, T, n, nx, m, seed=81, std=True, diag=diag)
    cfg = oracle.OracleCfg(max_iter=20, check_every=3, adapt_rho_every=0, sigma=1e-6, eps_abs=1e-12,
                           eps_rel=1e-12, rho_f_factor=1000.0, alpha=1.6)
    kw = {"diag_cost": True} if diag else {}
    flags = _lib.flag_stream_p(P) | (_lib.FLAG_FACTOR_GROUPS if variant == "groups" else 0)
    ref, it_ref, _, out, stats = _run_pair(qp, cfg, torch.float64, kernel_flags=flags, **kw)
    np.testing.assert_array_equal(stats.num_iter.cpu().numpy(), it_ref)
    _assert_state_close(out, ref, 1e-9)
    # the streaming kernels ran, not the generic one (same iterate, other rounding)
    _, out_g = _gpu_solve(qp, cfg, torch.float64, kernel_flags=_lib.FLAG_GENERIC_KERNEL, **kw)
    assert rel_err(out.x_blocks, out_g.x_blocks) < 1e-9
    assert not torch.equal(out.x_blocks, out_g.x_blocks)


def test_admm_stream_kernel_wide16_config2_direct_backend():
    # the linear workload (n = 16, nx = 12, m = 16) on the direct backend at a
    # batch with a partial last wavefront: the wide 16 streaming kernel and the
    # generic kernel run the same fp32 iteration, both against the fp64 oracle
    prob = configs.config2(B=515, seed=4).to(DEV, torch.float32)
    qp = prob.build_qp(*prob.initial_guess())
    cfg = oracle.OracleCfg(max_iter=40, check_every=41, adapt_rho_every=0, sigma=1e-6, eps_abs=1e-9, eps_rel=1e-9,
                           rho_f_factor=1000.0, alpha=1.6)
    outs = []
    for flags in (0, _lib.FLAG_GENERIC_KERNEL):
        outs.append(_gpu_solve(qp, cfg, torch.float32, kernel_flags=flags))
    (s_a, o_a), (s_b, o_b) = outs
    assert torch.equal(s_a.num_iter, s_b.num_iter)
    assert not torch.equal(o_a.x_blocks, o_b.x_blocks)  # two different kernels ran
    ref, it_ref = _oracle_full_batch(qp, cfg)
    np.testing.assert_array_equal(s_a.num_iter.cpu().numpy(), it_ref)
    _assert_batch_matches_oracle("config 2 B=515 wide stream", o_a, ref, TOL[torch.float32])
    _assert_batch_matches_oracle("config 2 B=515 generic", o_b, ref, TOL[torch.float32])


@pytest.mark.parametrize("shape", [(10, 13, 7, 4, 3), (6, 9, 12, 8, 4)])
def test_admm_stream_kernel_padded_width_adaptive_rho_fp32(shape):
    B, T, n, nx, m = shape
    qp = random_qp(B, T, n, nx, m, seed=82, std=True)
    cfg = oracle.OracleCfg(max_iter=200, check_every=2, adapt_rho_every=4, sigma=1e-6, eps_abs=1e-6, eps_rel=1e-6,
                           rho_f_factor=50.0, alpha=1.6, adaptive_rho_tolerance=1.5)
    ref, it_ref, _, out, stats = _run_pair(qp, cfg, torch.float64, kernel_flags=_lib.flag_stream_p(2))
    np.testing.assert_array_equal(stats.num_iter.cpu().numpy(), it_ref)
    assert rel_err(out.rho_bar, ref.rho_bar) < 1e-7
    _assert_state_close(out, ref, 1e-5)
    # fp32 against the fp64 oracle at a fixed iteration count
    cfg32 = oracle.OracleCfg(max_iter=30, check_every=31, adapt_rho_every=0, sigma=1e-6, eps_abs=1e-9,
                             eps_rel=1e-9, rho_f_factor=1000.0, alpha=1.0)
    ref32, _, _, out32, _ = _run_pair(qp, cfg32, torch.float32, kernel_flags=_lib.flag_stream_p(2))
    _assert_state_close(out32, ref32, TOL[torch.float32])


@pytest.mark.parametrize("shape", [(10, 13, 7, 4, 3), (7, 9, 8, 5, 6), (5, 7, 14, 10, 5), (6, 7, 14, 10, 10)])
@pytest.mark.parametrize("ineq", [False, True])
@pytest.mark.parametrize("same_dyn", [False, True])
def test_admm_stream_kernel_padded_width_warm_records(shape, ineq, same_dyn):
    """An SQP step whose QP differs from the previous call's in A_minus and c
    (and with ineq in G, l, u), on padded records: rewriting only those records
    gives the iterate of a step that repacks everything, bit for bit.  With
    same_dyn the QP keeps the previous A_minus and c (FLAG_WARM_SAME_DYNAMICS:
    their records are kept as well; without ineq no record is rewritten)."""
    from turbompc_amd.solvers.admm.admm_hip_backend import direct_workspace

    B, T, n, nx, m = shape
    qp1 = random_qp(B, T, n, nx, m, seed=83, std=True).to(DEV, torch.float64)
    qp2 = random_qp(B, T, n, nx, m, seed=84, std=True).to(DEV, torch.float64)
    # qp2 keeps qp1's cost, initial rows and (without ineq) inequality rows
    eq2 = dataclasses.replace(qp2.eq, A0=qp1.eq.A0, c0=qp1.eq.c0)
    if same_dyn:
        eq2 = dataclasses.replace(eq2, A_minus=qp1.eq.A_minus, c=qp1.eq.c)
    qp2 = dataclasses.replace(qp2, cost=qp1.cost, eq=eq2, ineq=qp2.ineq if ineq else qp1.ineq)
    cfg = oracle.OracleCfg(max_iter=15, check_every=16, adapt_rho_every=0, sigma=1e-6, eps_abs=1e-12,
                           eps_rel=1e-12, rho_f_factor=1000.0, alpha=1.0)
    solver = _solver(qp1, cfg)
    st0 = solver.initial_state(qp1, rho_bar=0.1)
    outs = []
    for warm in (True, False):
        ws = direct_workspace(qp1)
        (_, _), _, st1 = solver.solve(qp1, st0, workspace=ws)
        active = torch.ones(B, dtype=torch.bool, device=DEV)
        (_, _), stats, st2, _, _ = solver.sqp_step(qp2, st1, active, 0.0, rho_bar=0.1, workspace=ws,
                                                   warm_records=warm, warm_ineq=warm and ineq,
                                                   same_dynamics=same_dyn)
        outs.append((stats, st2))
    torch.cuda.synchronize()
    (s_w, o_w), (s_c, o_c) = outs
    assert torch.equal(s_w.num_iter, s_c.num_iter)
    for k in ("x_blocks", "z_g", "y_g", "y_f_0", "y_f_dyn", "xi_g"):
        assert torch.equal(getattr(o_w, k), getattr(o_c, k)), k


@pytest.mark.parametrize("kernel", ["stream", "generic"])
def test_admm_config5_large_rho_stays_with_oracle(kernel):
    # the reference's default adaptation on config 5 raises rho ~2000x at
    # iteration 25 (rho_f ~ 2.4e5, cond(Theta) ~ 1e9); the stored stage
    # inverses must be the symmetric part of the computed inverses: mirroring
    # one triangle made both kernels diverge (x off by 1e-2 one iteration
    # later, 1e13 after fifteen)
    prob = configs.config5(B=2, seed=3)
    qp = prob.build_qp(*prob.initial_guess())
    cfg = oracle.OracleCfg(max_iter=60, check_every=25, adapt_rho_every=25, sigma=1e-6, eps_abs=1e-13, eps_rel=1e-13,
                           rho_f_factor=1000.0, alpha=1.6, adaptive_rho_tolerance=5.0)
    flags = _lib.FLAG_GENERIC_KERNEL if kernel == "generic" else 0
    ref, it_ref, _, out, stats = _run_pair(qp, cfg, torch.float64, diag_cost=True, kernel_flags=flags)
    np.testing.assert_array_equal(stats.num_iter.cpu().numpy(), it_ref)
    assert np.all(ref.rho_bar > 100.0)
    assert rel_err(out.rho_bar, ref.rho_bar) < 1e-4
    assert rel_err(out.x_blocks, ref.x_blocks) < 1e-5
    assert rel_err(out.y_f_dyn, ref.y_f_dyn) < 1e-4


@pytest.mark.parametrize("seed", [0, 3])
def test_admm_config5_first_rho_update_matches_oracle(seed):
    # config 5 (dt = 10, rho_f / sigma = 1e8 at the start): the dual residual
    # is a cancellation of terms ~1e2 down to ~1e-6, so the first adaptive rho
    # update (iteration 25) follows the factorization's accuracy; a closed-form
    # 2x2 block inverse in the Gauss-Jordan steps moved it by 40%
    prob = configs.config5(B=2, seed=seed)
    qp = prob.build_qp(*prob.initial_guess())
    cfg = oracle.OracleCfg(max_iter=26, check_every=25, adapt_rho_every=25, sigma=1e-6, eps_abs=1e-13, eps_rel=1e-13,
                           rho_f_factor=1000.0, alpha=1.6, adaptive_rho_tolerance=5.0)
    ref, it_ref, _, out, stats = _run_pair(qp, cfg, torch.float64, diag_cost=True)
    np.testing.assert_array_equal(stats.num_iter.cpu().numpy(), it_ref)
    assert np.all(ref.rho_bar > 100.0)  # the update fired
    # rho is a ratio of cancelled residuals: ~1e-5 apart between two summation orders
    assert rel_err(out.rho_bar, ref.rho_bar) < 1e-4
    for k in FIELDS[:-1]:  # the state after one iteration at the new rho
        if np.asarray(getattr(ref, k)).size:
            assert rel_err(getattr(out, k), getattr(ref, k)) < 1e-5, k


@pytest.mark.parametrize("alpha", [1.0, 1.6])
def test_admm_stream_kernel_structured_records_adaptive_rho(alpha):
    # termination and rho adaptation read the residuals of the structured path
    qp = random_qp(11, 9, 6, 4, 3, seed=42, std=True, diag=True)
    cfg = oracle.OracleCfg(max_iter=200, check_every=2, adapt_rho_every=4, sigma=1e-6, eps_abs=1e-6, eps_rel=1e-6,
                           rho_f_factor=50.0, alpha=alpha, adaptive_rho_tolerance=1.5)
    ref, it_ref, _, out, stats = _run_pair(qp, cfg, torch.float64, kernel_flags=_lib.flag_stream_p(2),
                                           diag_cost=True)
    np.testing.assert_array_equal(stats.num_iter.cpu().numpy(), it_ref)
    assert len(set(it_ref.tolist())) > 1
    assert rel_err(out.rho_bar, ref.rho_bar) < 1e-7
    _assert_state_close(out, ref, 1e-5)


def test_admm_stream_kernel_structured_records_match_dense_on_bench_batch():
    # the benchmark QP (quadrotor: diagonal weights) solved with the structure
    # declared and with dense D_t records
    B = 4099
    prob = make_quadrotor_config(B=B, seed=7, dtype=torch.float32, device=DEV)
    qp = prob.build_qp(*prob.initial_guess())
    cfg = oracle.OracleCfg(max_iter=20, check_every=1, adapt_rho_every=0, sigma=1e-6, eps_abs=1e-9, eps_rel=1e-9,
                           rho_f_factor=1000.0, alpha=1.6)
    outs = []
    for kw in ({}, {"diag_cost": True}):
        solver = _solver(qp, cfg, **kw)
        st0 = solver.initial_state(qp, rho_bar=0.1)
        _, stats, out = solver.solve(qp, st0, alpha=cfg.alpha)
        outs.append((stats, out))
    torch.cuda.synchronize()
    (s_a, o_a), (s_b, o_b) = outs
    assert torch.equal(s_a.num_iter, s_b.num_iter)
    for k in ("x_blocks", "y_f_dyn", "y_g", "z_g", "y_f_0"):
        assert rel_err(getattr(o_a, k), getattr(o_b, k)) < 1e-5, k
    ref, it_ref = _oracle_full_batch(qp, cfg)
    np.testing.assert_array_equal(s_b.num_iter.cpu().numpy(), it_ref)
    _assert_batch_matches_oracle("config 3 B=4099 diagonal records", o_b, ref, TOL[torch.float32])


# ---- G rows resident in LDS (TMPC_FLAG_CONST_G: the same G_t for every stage
# and problem, as box rows are): the backward sweep streams only the A_minus
# rows; the products are the same, so the iterates are bit for bit those of
# the form that streams the whole records, and match the oracle.
def _shared_g(qp, seed=0):
    """qp with one G_t (problem 0's stage 0) for every stage and problem, and
    bounds around G z at a point z that satisfies the equality constraints
    (least squares on the dense C), so that the QP stays feasible."""
    from helpers import dense_C

    G = qp.ineq.G[:1, :1].expand_as(qp.ineq.G).contiguous()
    a = np_qp(qp)
    B, T, m, n = G.shape
    rng = np.random.default_rng(seed)
    l, u = np.empty((B, T, m)), np.empty((B, T, m))
    for b in range(B):
        C = dense_C(a["A0"][b], a["Am"][b], a["Ap"][b])
        z = np.linalg.lstsq(C, np.concatenate([a["c0"][b], a["c"][b].reshape(-1)]), rcond=None)[0].reshape(T, n)
        gz = np.einsum("tij,tj->ti", G[b].numpy(), z)
        l[b] = gz - rng.uniform(0.05, 0.5, size=(T, m))
        u[b] = gz + rng.uniform(0.05, 0.5, size=(T, m))
    return qp.replace_ineq(G=G, l=torch.tensor(l), u=torch.tensor(u))


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("P", [1, 2])
# n = 17 records run the resident-G form (nx + m = 17, 17 and 16 below);
# elsewhere the flag is ignored (n = 6)
@pytest.mark.parametrize("shape", [(8, 11, 17, 13, 4), (5, 9, 17, 12, 5), (6, 7, 17, 13, 3), (13, 21, 6, 4, 2)])
def test_admm_stream_kernel_const_g_rows(shape, P, dtype):
    B, T, n, nx, m = shape
    qp = _shared_g(random_qp(B, T, n, nx, m, seed=57, std=True, diag=True))
    cfg = oracle.OracleCfg(max_iter=20, check_every=3, adapt_rho_every=0, sigma=1e-6, eps_abs=1e-12,
                           eps_rel=1e-12, rho_f_factor=1000.0, alpha=1.6)
    outs = []
    for const_g in (False, True):
        ref, it_ref, _, out, stats = _run_pair(qp, cfg, dtype, kernel_flags=_lib.flag_stream_p(P), diag_cost=True,
                                               const_g=const_g)
        np.testing.assert_array_equal(stats.num_iter.cpu().numpy(), it_ref)
        outs.append(out)
    for k in FIELDS:
        assert torch.equal(getattr(outs[0], k), getattr(outs[1], k)), k
    assert float(np.max(np.abs(ref.y_g))) > 0  # some rows are active
    # fp32 on these random QPs (cond(Theta) up to ~1e6 at rho_f = 100, the
    # inverse rounded to fp32 on store): measured up to 1.3e-4 against the fp64
    # oracle in either form; the workload tests hold fp32 to 1e-4
    _assert_state_close(outs[1], ref, 1e-9 if dtype == torch.float64 else 5e-4)


def test_quadrotor_sqp_const_g_rows_bit_equal():
    """The benchmark's solve with and without the resident G rows (the
    solver sets the flag for box rows): the same iterates bit for bit."""
    prob = make_quadrotor_config(B=300, seed=9, dtype=torch.float32, device=DEV)
    import copy as _copy

    from turbompc_amd.solvers.turbompc_solver import DEFAULT_SOLVER_PARAMS, TurboMPCSolver

    params = _copy.deepcopy(DEFAULT_SOLVER_PARAMS)
    params["num_sqp_iteration_max"], params["tol_convergence"] = 3, 0.0
    params["admm"].update(max_iter=20, adapt_rho_every=0, relaxation_parameter=1.0)
    sols = []
    for const_g in (True, False):
        p2 = _copy.copy(prob)
        p2.const_g = const_g
        solver = TurboMPCSolver(p2, params)
        assert bool(solver._admm_solver_fwd._kernel_flags & _lib.FLAG_CONST_G) == const_g
        sols.append(solver.solve(solver.initial_guess()))
    torch.cuda.synchronize()
    for k in ("states", "controls"):
        assert torch.equal(getattr(sols[0], k), getattr(sols[1], k)), k
    for k in sols[0].admm_state._fields:
        assert torch.equal(getattr(sols[0].admm_state, k), getattr(sols[1].admm_state, k)), k
