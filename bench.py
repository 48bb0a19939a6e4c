#!/usr/bin/env python3
"""MPC solves/sec at B=4096 on one MI355X (benchmark config 3: quadrotor SQP).

One step = one full batched MPC solve: 5 SQP iterations, each = on-device RK4
linearization + ADMM (block-tridiagonal factorization + 20 fused iterations)
+ the first-order convergence check, from the same initial guess every step.
Inputs are resident on the GPU before timing starts.

Prints one JSON line with the metric, a roofline entry for the dominant kernel
(admm_stream_kernel: 20 ADMM iterations of the batch per launch, timed live
with HIP events the library records around every launch on the solve stream;
the whole QP solve is reported beside it) and the CPU baseline (the liboracle
restatement of the reference CPU path on a bounded sample of the same workload).

--workload config4 measures the obstacle-avoidance workload instead (B=16384,
8 SQP x 30 ADMM, fp32), a secondary line; the default is the metric's config 3.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E


def bytes_per_qp(T, n, nx, n0, m, K, w, m_g=0):
    """Algorithmic HBM bytes of one QP solve: w * (F + K * I), the streaming
    model of the survey (factor written once and read once per iteration;
    QP data and iterates read/written once per iteration; A_plus, A0 and
    box-selector G rows are constants and not counted)."""
    N = T - 1
    fac = T * n * (n + 1) // 2 + N * n * n
    F = T * n * n + N * n * n + N * nx * n + T * m_g * n + fac
    It = fac + N * nx * n + T * m_g * n + T * n + (N * nx + n0) + 2 * T * m \
        + 2 * (T * n + (N * nx + n0) + T * m + T * m)
    return w * (F + K * It), w * F, w * It


def make_solver(prob, n_sqp, admm_iters):
    from turbompc_amd.solvers.turbompc_solver import DEFAULT_SOLVER_PARAMS, TurboMPCSolver
    import copy

    params = copy.deepcopy(DEFAULT_SOLVER_PARAMS)
    params["num_sqp_iteration_max"] = n_sqp
    params["tol_convergence"] = 0.0  # fixed SQP iteration count
    params["admm"]["max_iter"] = admm_iters
    params["admm"]["adapt_rho_every"] = 0  # fixed-iteration protocol
    params["admm"]["relaxation_parameter"] = 1.0
    return TurboMPCSolver(prob, params, forward_backend="admm_hip_direct", backward_backend="direct_hip_kkt")


def cpu_baseline(B_gpu, n_sqp, admm_iters, seed, budget_s, workload="config3"):
    import numpy as np
    import torch

    import oracle
    from oracle.sqp_cpu import obstacle_sqp, quadrotor_sqp
    from turbompc_amd.problems import configs
    from turbompc_amd.problems.ocp import LinearOCP
    from turbompc_amd.problems.quadrotor import make_quadrotor_config

    cores = len(os.sched_getaffinity(0))

    def run_config4(Bs):
        prob = configs.config4(B=Bs, seed=seed)
        D, E, q = (t.numpy() for t in prob.cost_blocks())
        A0, c0 = (t.numpy() for t in prob.initial_equality())
        G, l, u = (t.numpy() for t in LinearOCP.inequality_blocks(prob))
        static = dict(D=D, E=E, q=q, A0=A0, c0=c0, A_plus=prob.a_plus().numpy(), G=G, l=l, u=u)
        xg, ug = (t.numpy() for t in prob.initial_guess())
        Am, c = (t.numpy() for t in prob.dynamics_blocks(*prob.initial_guess()))
        cfg = oracle.OracleCfg(max_iter=admm_iters, check_every=50, adapt_rho_every=0, sigma=1e-6, eps_abs=1e-9,
                               eps_rel=1e-9, rho_f_factor=1000.0, alpha=1.0)
        t0 = time.perf_counter()
        obstacle_sqp(static, xg, ug, A_minus=Am, c=c, centers=prob.centers.numpy(), radii=prob.radii.numpy(), dim=3,
                     cfg=cfg, rho0=0.1, n_sqp=n_sqp, dtype=np.float32, nthreads=cores)
        return time.perf_counter() - t0

    def run(Bs):
        if workload == "config4":
            return run_config4(Bs)
        prob = make_quadrotor_config(B=Bs, seed=seed, dtype=torch.float64, device="cpu")
        D, E, q = (t.numpy() for t in prob.cost_blocks())
        A0, c0 = (t.numpy() for t in prob.initial_equality())
        G, l, u = (t.numpy() for t in prob.inequality_blocks())
        static = dict(D=D, E=E, q=q, A0=A0, c0=c0, A_plus=prob.a_plus().numpy(), G=G, l=l, u=u)
        xg, ug = (t.numpy() for t in prob.initial_guess())
        cfg = oracle.OracleCfg(max_iter=admm_iters, check_every=25, adapt_rho_every=0, sigma=1e-6, eps_abs=1e-9,
                               eps_rel=1e-9, rho_f_factor=1000.0, alpha=1.0)
        t0 = time.perf_counter()
        quadrotor_sqp(static, xg, ug, dt=prob.dt, params=prob.params, cfg=cfg, rho0=0.1, n_sqp=n_sqp,
                      dtype=np.float32, nthreads=cores)
        return time.perf_counter() - t0

    t_cal = run(64)
    Bs = int(min(B_gpu, max(64, budget_s / max(t_cal, 1e-6) * 64)))
    dt = run(Bs) if Bs > 64 else t_cal
    if workload == "config4":
        sample = (f"{Bs} obstacle problems (config 4 shapes, seed {seed}), {n_sqp} SQP x {admm_iters} ADMM, "
                  f"fp32 ADMM (liboracle, OpenMP over the batch) + numpy obstacle rows, {dt:.2f} s wall")
    else:
        sample = (f"{Bs} quadrotor problems (config 3 shapes, seed {seed}), {n_sqp} SQP x {admm_iters} ADMM, "
                  f"fp32 ADMM (liboracle, OpenMP over the batch) + fp64 complex-step RK4 linearization, "
                  f"{dt:.2f} s wall")
    return {"value": Bs / dt, "unit": "MPC solves/s", "cores": cores, "kind": "port", "sample": sample}


TRAFFIC_FILE = ROOT / "profiles" / "admm_stream_kernel_config3_pmc.txt"


def measured_traffic():
    """HBM bytes per launch of the iteration kernel from the committed
    rocprofv3 --pmc summary (FETCH_SIZE + WRITE_SIZE, copy-calibrated), or None."""
    try:
        for line in TRAFFIC_FILE.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch"):
                return float(line.split("=")[1])
    except (OSError, ValueError, IndexError):
        pass
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", choices=("config3", "config4"), default="config3",
                    help="config3 (the metric's workload) or the obstacle workload config4 (a secondary line)")
    ap.add_argument("--batch", type=int, default=None, help="default 4096 (config3), 16384 (config4)")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--sqp", type=int, default=None, help="default 5 (config3), 8 (config4)")
    ap.add_argument("--admm-iters", type=int, default=None, help="default 20 (config3), 30 (config4)")
    ap.add_argument("--cpu-baseline", type=int, default=1)
    ap.add_argument("--cpu-budget", type=float, default=15.0, help="seconds of CPU work for the baseline sample")
    ap.add_argument("--copy-calibration", type=int, default=0,
                    help="after timing, copy this many MiB device-to-device (counter calibration under rocprofv3)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build measures one GPU only (the batch of independent MPC problems would shard "
              "across GPUs with no communication in the forward solve); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    from turbompc_amd import _lib
    from turbompc_amd.problems import configs
    from turbompc_amd.problems.quadrotor import make_quadrotor_config
    from turbompc_amd.solvers.admm import admm as admm_mod

    c4 = args.workload == "config4"
    args.batch = args.batch or (16384 if c4 else 4096)
    args.sqp = args.sqp or (8 if c4 else 5)
    args.admm_iters = args.admm_iters or (30 if c4 else 20)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    B = args.batch
    if c4:
        prob = configs.config4(B=B, seed=args.seed).to(dev, torch.float32)
    else:
        prob = make_quadrotor_config(B=B, seed=args.seed, dtype=torch.float32, device=dev)
    solver = make_solver(prob, args.sqp, args.admm_iters)
    guess = solver.initial_guess()

    # every ADMM solve (the first SQP iteration's solve and every later SQP
    # step) is timed twice with HIP events on the stream the library launches
    # on: the whole QP solve (pack or record rewrite + factorization +
    # iterations + unpack) and, through the library's hook, the iteration phase
    # alone (the single admm_stream_kernel launch of a fixed-iteration solve)
    solve_events = []
    iter_timer = _lib.IterationTimer()
    orig, orig_step = admm_mod.ADMMSolver.solve, admm_mod.ADMMSolver.sqp_step

    def timed(fn):
        def wrapper(self, *a, **kw):
            s = torch.cuda.current_stream(dev)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(s)
            with iter_timer:
                out = fn(self, *a, **kw)
            e1.record(s)
            solve_events.append((e0, e1))
            return out
        return wrapper

    admm_mod.ADMMSolver.solve = timed(orig)
    admm_mod.ADMMSolver.sqp_step = timed(orig_step)
    for _ in range(args.warmup):
        solver.solve(guess)
    torch.cuda.synchronize()
    solve_events.clear()
    iter_timer.clear()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        sol = solver.solve(guess)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    admm_mod.ADMMSolver.solve, admm_mod.ADMMSolver.sqp_step = orig, orig_step
    solve_ms = [a.elapsed_time(b) for a, b in solve_events]
    iter_ms = iter_timer.results()
    solve_avg_s = sum(solve_ms) / len(solve_ms) / 1e3
    iter_avg_s = sum(iter_ms) / len(iter_ms) / 1e3
    if args.copy_calibration:
        x = torch.ones(args.copy_calibration * (1 << 18), dtype=torch.float32, device=dev)
        y = torch.empty_like(x)
        y.copy_(x)
        torch.cuda.synchronize()

    T = prob.horizon + 1
    if c4:  # n = 9, nx = n0 = 6, 3 box rows and 8 obstacle rows (data-carrying)
        per_qp, F, It = bytes_per_qp(T, 9, 6, 6, 11, args.admm_iters, 4, m_g=8)
    else:  # n = 17, nx = n0 = 13, 4 box rows
        per_qp, F, It = bytes_per_qp(T, 17, 13, 13, 4, args.admm_iters, 4)
    iter_bytes = B * args.admm_iters * It  # algorithmic bytes of one iteration-kernel launch
    achieved = iter_bytes / iter_avg_s / 1e9
    qp_achieved = per_qp * B / solve_avg_s / 1e9
    finite = bool(torch.isfinite(sol.states).all() and torch.isfinite(sol.controls).all())
    traffic = None if c4 else measured_traffic()

    value = B * args.steps / elapsed
    if c4:
        workload = (f"config 4: obstacle avoidance, double integrator nx=6 nu=3 N={prob.horizon}, 8 spheres "
                    f"(linearized rows), |u| <= 3, {args.sqp} SQP x {args.admm_iters} ADMM, ADMM state carried "
                    f"across SQP iterations, direct block-tridiagonal KKT backend")
        data = "synthetic (seeded obstacle fields: 8 spheres, start and goal on opposite faces of [-4,4]^3)"
    else:
        workload = ("config 3: quadrotor nonlinear SQP, nx=13 nu=4 N=40, RK4 dt=0.02, 5 SQP x 20 ADMM, "
                    "direct block-tridiagonal KKT backend")
        data = "synthetic (seeded quadrotor fleet: random goals, perturbed hover starts)"
    line = {
        "metric": f"MPC solves/sec at B={B}{', config 4' if c4 else ''} (1 MI355X)",
        "value": value,
        "unit": "MPC solves/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": elapsed / args.steps * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": data,
        "config": {
            "workload": workload,
            "batch": B,
            "horizon": prob.horizon,
            "sqp_iterations": args.sqp,
            "admm_iterations": args.admm_iters,
            "parallelism": "single GPU, batch-parallel",
            "solution_finite": finite,
            "kernel_only_solves_per_s": B / (args.sqp * solve_avg_s),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": traffic,
            "kernel": f"admm_stream_kernel (one launch = {args.admm_iters} ADMM iterations of the batch)",
            "algorithmic_bytes_per_launch": iter_bytes,
            "avg_launch_ms": iter_avg_s * 1e3,
            "qp_solve": {
                "kernels": "stage_pack + factor_std + admm_stream + stage_unpack",
                "algorithmic_bytes": per_qp * B,
                "avg_ms": solve_avg_s * 1e3,
                "achieved": qp_achieved,
                "frac": qp_achieved / HBM_PEAK_GBS,
            },
        },
    }
    if args.cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(B, args.sqp, args.admm_iters, args.seed, args.cpu_budget,
                                            args.workload)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
