"""The workloads of configs 2 and 5 at their own iteration counts against the
fp64 oracle (the other GPU tests run them shorter).

Config 2 (random stable LTI, nx=12, nu=4, N=50) on the PCG backend at its 100
ADMM iterations, in fp32 and fp64, on each PCG kernel:
  * fixed count (pcg_eps = 0, 10 PCG iterations per ADMM iteration, which
    never reach the |eta| < 1e-12 floor): every iteration is determined, so
    the bars are the parity bars, 1e-9 (fp64) and 1e-4 (fp32);
  * the workload's tolerance stop (pcg_eps = 1e-6, at most 50): two correct
    implementations may stop a PCG solve one iteration apart, so the bar is
    what the tolerance itself allows.  Both iterates lie within the distance
    d of the fp64 oracle's tolerance-stopped run from the same ADMM with exact
    Schur solves (the direct backend), so fp64 is held to 2 d (measured:
    d = 3.5e-6 on seed 0); fp32 to the 1e-4 parity bar (the fp32 oracle
    itself sits 8e-6 from the fp64 one).
Config 5 (Clohessy-Wiltshire, fp64) at its 200 ADMM iterations with a fixed
rho, on the streaming and the generic kernels, held to 1e-9.
Reference semantics: admm.py:795-1049, pcg_primal.py:70-175; the reference's
own comparison of its backends is tests/cuda/backends/
test_admm_math_cuda_vs_python.py:195-253.
"""
import numpy as np
import pytest
import torch

import oracle
from helpers import TOL, rel_err, zero_state
from test_gpu_admm import PCG_KERNELS, _assert_state_close, _run_pair
from turbompc_amd import _lib
from turbompc_amd.problems import configs
from turbompc_amd.solvers.linear_systems_solvers.backends import AdmmBackend

pytestmark = pytest.mark.gpu

K2 = 100  # config 2's ADMM iterations


def _cfg2(pcg_eps, pcg_max_iter):
    return oracle.OracleCfg(max_iter=K2, check_every=200, adapt_rho_every=0, sigma=1e-6, eps_abs=1e-9,
                            eps_rel=1e-9, rho_f_factor=1000.0, alpha=1.0, pcg_eps=pcg_eps,
                            pcg_max_iter=pcg_max_iter)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("kernel", list(PCG_KERNELS))
def test_config2_pcg_fixed_count_at_100_iterations(kernel, dtype):
    prob = configs.config2(B=8, seed=0)
    qp = prob.build_qp(*prob.initial_guess())
    cfg = _cfg2(0.0, 10)
    print(f"config 2 PCG ({kernel}, {dtype}): {K2} ADMM x 10 PCG iterations, B=8", flush=True)
    ref, it_ref, pcg_ref, out, stats = _run_pair(qp, cfg, dtype, backend=AdmmBackend.HIP_PCG, schur="pcg",
                                                 kernel_flags=PCG_KERNELS[kernel])
    assert np.all(pcg_ref == K2 * 10)  # the count is fixed: the floor never stops a solve
    np.testing.assert_array_equal(stats.num_iter.cpu().numpy(), it_ref)
    np.testing.assert_array_equal(stats.num_pcg_iters.sum(1).cpu().numpy(), pcg_ref)
    if dtype == torch.float64:
        _assert_state_close(out, ref, 1e-9)
    else:
        for k in ("x_blocks", "z_g", "y_g", "y_f_0", "y_f_dyn"):
            e = rel_err(getattr(out, k), getattr(ref, k))
            print(f"  {k}: rel err vs fp64 oracle {e:.2e}")
            assert e < TOL[torch.float32], (k, e)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("kernel", list(PCG_KERNELS))
def test_config2_pcg_tolerance_stopped_at_100_iterations(kernel, dtype):
    prob = configs.config2(B=8, seed=0)
    qp = prob.build_qp(*prob.initial_guess())
    cfg = _cfg2(1e-6, 50)
    print(f"config 2 PCG ({kernel}, {dtype}): {K2} ADMM iterations, PCG to 1e-6 (at most 50), B=8", flush=True)
    ref, it_ref, pcg_ref, out, stats = _run_pair(qp, cfg, dtype, backend=AdmmBackend.HIP_PCG, schur="pcg",
                                                 kernel_flags=PCG_KERNELS[kernel])
    exact, _, _ = oracle.admm_solve(qp, zero_state(qp, 0.1), cfg, schur="direct", dtype=np.float64)
    np.testing.assert_array_equal(stats.num_iter.cpu().numpy(), it_ref)
    pcg = stats.num_pcg_iters.sum(1).cpu().numpy()
    # the stopping iteration of a solve may differ by one now and then
    print(f"  PCG iterations: oracle {pcg_ref.tolist()}, GPU {pcg.tolist()}")
    assert np.all(np.abs(pcg - pcg_ref) <= 0.02 * pcg_ref)
    for k in ("x_blocks", "z_g", "y_g", "y_f_0", "y_f_dyn"):
        d = rel_err(getattr(ref, k), getattr(exact, k))
        bar = 2.0 * d if dtype == torch.float64 else TOL[torch.float32]
        e = rel_err(getattr(out, k), getattr(ref, k))
        print(f"  {k}: rel err vs fp64 oracle {e:.2e} (tolerance spread d {d:.2e}, bar {bar:.2e})")
        assert e < bar, (k, e, bar)


@pytest.mark.parametrize("kernel", ["stream", "generic"])
def test_config5_fixed_rho_at_200_iterations_fp64(kernel):
    prob = configs.config5(B=64, seed=0)
    qp = prob.build_qp(*prob.initial_guess())
    cfg = oracle.OracleCfg(max_iter=200, check_every=25, adapt_rho_every=0, sigma=1e-6, eps_abs=1e-9,
                           eps_rel=1e-9, rho_f_factor=1000.0, alpha=1.6)
    flags = _lib.FLAG_GENERIC_KERNEL if kernel == "generic" else 0
    print(f"config 5 ({kernel}): 200 ADMM iterations, fixed rho, B=64, fp64", flush=True)
    ref, it_ref, _, out, stats = _run_pair(qp, cfg, torch.float64, kernel_flags=flags, diag_cost=True)
    np.testing.assert_array_equal(stats.num_iter.cpu().numpy(), it_ref)
    assert np.all(it_ref == 200)
    x = out.x_blocks.cpu().numpy()
    worst = max(rel_err(x[b], ref.x_blocks[b]) for b in range(x.shape[0]))
    print(f"  worst-problem x rel err {worst:.2e}")
    assert worst < 1e-9
    _assert_state_close(out, ref, 1e-9)
