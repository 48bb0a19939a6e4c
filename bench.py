#!/usr/bin/env python3
"""MPC solves/sec at B=4096 on one MI355X (benchmark config 3: quadrotor SQP).

One step = one full batched MPC solve: 5 SQP iterations, each = on-device RK4
linearization + ADMM (block-tridiagonal factorization + 20 fused iterations)
+ the first-order convergence check, from the same initial guess every step.
Inputs are resident on the GPU before timing starts.

Prints one JSON line with the metric, a roofline entry for the dominant kernel
(timed live with HIP events the library records around every iteration phase
on the solve stream; the whole QP solve is reported beside it) and the CPU
baseline (the oracle's restatement of the reference CPU path, compiled with
-march=native on this host, on a bounded sample of the same workload, on all
cores and on one).

The default run (config 3, no --batch/--sqp/--admm-iters/--linesearch) also
reports configs 4, 5 and 2 (fp32 and fp64) under "secondary" (short runs:
--secondary-steps timed steps and a --secondary-cpu-budget CPU sample each;
--secondary 0 skips them).  Each can also run alone as the line's workload:
  --workload config4  obstacle avoidance, B=16384, 8 SQP x 30 ADMM, fp32
  --workload config5  spacecraft rendezvous, B=2048, fp64: 200 ADMM iterations
                      and the implicit-differentiation backward pass (gradients
                      of sum |x_N|^2 with respect to Q, R and x0)
  --workload config2  random stable LTI, B=1024, 100 ADMM iterations on the PCG
                      Schur solve (tolerance 1e-6, at most 50 PCG iterations),
                      --dtype f32 or f64
Every workload follows the fixed-iteration protocol: rho is not adapted and
the convergence tests cannot stop a solve early.
"""
from __future__ import annotations

import argparse
import copy
import json
import os
import sys
import tempfile
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
# MI355X vector (VALU) FMA rate, fp64 and fp32 without packed math (the
# library is built with packed-fp32 instructions disabled): 256 CUs x 4 SIMDs
# x 16 lanes x 2 flop x 2.4 GHz
VALU_PEAK_TFLOPS = 78.6


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


def bytes_pcg(T, n, nx, n0, m, K, pcg_iters, w, m_g=0):
    """The PCG variant of the model: F reads D, E and A_minus and writes S and
    Phiinv (2 (3T - 2) n^2 words); each ADMM iteration moves I of the direct
    model without its factor read, plus 2 (3T - 2) n^2 + 9 T n words per
    PCG iteration actually run (S and Phiinv streamed, the CG vectors).
    Returns (bytes of the solve, bytes of its iteration phase)."""
    N = T - 1
    sp = 2 * (3 * T - 2) * n * n
    F = T * n * n + N * n * n + N * nx * n + T * m_g * n + sp
    It = N * nx * n + T * m_g * n + T * n + (N * nx + n0) + 2 * T * m \
        + 2 * (T * n + (N * nx + n0) + T * m + T * m)
    per_pcg = sp + 9 * T * n
    phase = K * It + pcg_iters * per_pcg
    return w * (F + phase), w * phase


def flops_pcg_iteration(T, n):
    """Algorithmic flops of one PCG iteration of one problem on the
    block-tridiagonal Schur system (pcg_primal.py:70-175): the products with S
    and with the block preconditioner Phiinv, (3T - 2) n x n blocks each at 2
    flop per entry, two dot products and three vector updates of length T n."""
    return 4 * (3 * T - 2) * n * n + 10 * T * n


def sqp_params(n_sqp, admm_iters):
    from turbompc_amd.solvers.turbompc_solver import DEFAULT_SOLVER_PARAMS

    params = copy.deepcopy(DEFAULT_SOLVER_PARAMS)
    params["num_sqp_iteration_max"] = n_sqp
    params["tol_convergence"] = 0.0  # fixed SQP iteration count
    params["admm"]["max_iter"] = admm_iters
    params["admm"]["adapt_rho_every"] = 0  # fixed-iteration protocol
    params["admm"]["relaxation_parameter"] = 1.0
    return params


def make_solver(prob, n_sqp, admm_iters, linesearch=False):
    from turbompc_amd.solvers.turbompc_solver import TurboMPCSolver

    params = sqp_params(n_sqp, admm_iters)
    params["linesearch"] = bool(linesearch)
    return TurboMPCSolver(prob, params, forward_backend="admm_hip_direct", backward_backend="direct_hip_kkt")


# ------------------------------------------------------------ CPU baseline ----
def cpu_baseline(workload, B_gpu, args):
    """The oracle (the restated reference CPU path) on a bounded sample of the
    workload, built with -march=native on this host: all cores (value), then
    one thread (single_thread)."""
    import numpy as np
    import torch

    import oracle
    from oracle.sqp_cpu import obstacle_sqp, quadrotor_sqp
    from turbompc_amd.problems import configs
    from turbompc_amd.problems.ocp import LinearOCP
    from turbompc_amd.problems.quadrotor import make_quadrotor_config

    build = "g++ -O3 -march=native (oracle/Makefile native, built on this host)"
    try:
        oracle.use_native_build(tempfile.mkdtemp(prefix="tmpc_oracle_native_"))
    except Exception as e:  # keep the portable build
        build = f"portable x86-64-v2 build (native build failed: {type(e).__name__})"
    cores = len(os.sched_getaffinity(0))
    n_sqp, K, seed = args.sqp, args.admm_iters, args.seed

    def cfg(**kw):
        base = dict(max_iter=K, check_every=K + 1, adapt_rho_every=0, sigma=1e-6, eps_abs=1e-30, eps_rel=1e-30,
                    rho_f_factor=1000.0, alpha=1.0)
        base.update(kw)
        return oracle.OracleCfg(**base)

    def static_of(prob):
        D, E, q = (t.numpy() for t in prob.cost_blocks())
        A0, c0 = (t.numpy() for t in prob.initial_equality())
        G, l, u = (t.numpy() for t in LinearOCP.inequality_blocks(prob))
        return dict(D=D, E=E, q=q, A0=A0, c0=c0, A_plus=prob.a_plus().numpy(), G=G, l=l, u=u)

    def run(Bs, threads):
        if workload == "config4":
            prob = configs.config4(B=Bs, seed=seed)
            xg, ug = (t.numpy() for t in prob.initial_guess())
            Am, c = (t.numpy() for t in prob.dynamics_blocks(*prob.initial_guess()))
            t0 = time.perf_counter()
            obstacle_sqp(static_of(prob), xg, ug, A_minus=Am, c=c, centers=prob.centers.numpy(),
                         radii=prob.radii.numpy(), dim=3, cfg=cfg(), rho0=0.1, n_sqp=n_sqp, dtype=np.float32,
                         nthreads=threads)
            return time.perf_counter() - t0
        if workload == "config3":
            prob = make_quadrotor_config(B=Bs, seed=seed, dtype=torch.float64, device="cpu")
            xg, ug = (t.numpy() for t in prob.initial_guess())
            t0 = time.perf_counter()
            quadrotor_sqp(static_of(prob), xg, ug, dt=prob.dt, params=prob.params, cfg=cfg(), rho0=0.1,
                          n_sqp=n_sqp, dtype=np.float32, nthreads=threads)
            return time.perf_counter() - t0
        if workload == "config2":
            prob = configs.config2(B=Bs, seed=seed)
            qp = prob.build_qp(*prob.initial_guess())
            st0 = _zero_state_np(qp)
            dt = np.float64 if args.dtype == "f64" else np.float32
            t0 = time.perf_counter()
            oracle.admm_solve(qp, st0, cfg(pcg_eps=1e-6, pcg_max_iter=50), schur="pcg", dtype=dt, nthreads=threads)
            return time.perf_counter() - t0
        # config5: forward ADMM, then the dense adjoint KKT of the reference's
        # pure-JAX backward pass (backward_kkt_jax.py:177-198)
        prob = configs.config5(B=Bs, seed=seed)
        qp = prob.build_qp(*prob.initial_guess())
        t0 = time.perf_counter()
        st, _, _ = oracle.admm_solve(qp, _zero_state_np(qp), cfg(), nthreads=threads)
        oracle.adjoint_kkt(_adjoint_qp_np(qp, st, prob.num_state_variables), nthreads=threads)
        return time.perf_counter() - t0

    def sample(threads, budget):
        t_cal = run(8, threads)
        Bs = int(min(B_gpu, max(8, budget / max(t_cal, 1e-6) * 8)))
        dt = run(Bs, threads) if Bs > 8 else t_cal
        return Bs, dt

    Bs, dt = sample(cores, args.cpu_budget)
    B1, dt1 = sample(1, args.cpu_budget / 3)
    what = {
        "config3": f"quadrotor problems (config 3 shapes), {n_sqp} SQP x {K} ADMM, fp32 ADMM + fp64 complex-step "
                   "RK4 linearization",
        "config4": f"obstacle problems (config 4 shapes), {n_sqp} SQP x {K} ADMM, fp32 ADMM + numpy obstacle rows",
        "config2": f"LTI problems (config 2 shapes), {K} ADMM iterations on PCG (tol 1e-6, <= 50), {args.dtype}",
        "config5": f"spacecraft problems (config 5 shapes), {K} ADMM iterations + dense adjoint KKT, fp64",
    }[workload]
    return {
        "value": Bs / dt, "unit": "MPC solves/s", "cores": cores, "kind": "port",
        "sample": f"{Bs} {what} (seed {seed}), OpenMP over the batch on {cores} threads, {dt:.2f} s wall; {build}",
        "single_thread": {"value": B1 / dt1, "sample": f"{B1} problems on 1 thread, {dt1:.2f} s wall"},
    }


def _zero_state_np(qp):
    import numpy as np

    import oracle

    B, T, n, nx, n0, m = qp.dims
    f = lambda t: np.asarray(t, dtype=np.float64)  # noqa: E731
    z = np.clip(np.zeros((B, T, m)), f(qp.ineq.l), f(qp.ineq.u))
    return oracle.OracleState(np.zeros((B, T, n)), np.zeros((B, T, m)), np.zeros((B, n0)), np.zeros((B, T - 1, nx)),
                              z, np.zeros((B, T, m)), np.full((B,), 0.1))


def _adjoint_qp_np(qp, st, nx):
    """The adjoint QP of the loss sum |x_N|^2 at an ADMM solution, for the CPU
    baseline: q = -dL/dz, homogeneous constraints, the active rows of G signed
    by the dual sign (turbompc_solver.py:544-618, :1387-1439)."""
    from types import SimpleNamespace as NS

    import numpy as np

    f = lambda t: np.asarray(t, dtype=np.float64)  # noqa: E731
    x = st.x_blocks
    dl = np.zeros_like(x)
    dl[:, -1, :nx] = 2 * x[:, -1, :nx]
    sign = (st.y_g < -1e-9).astype(np.float64) - (st.y_g > 1e-9).astype(np.float64)
    return NS(cost=NS(D=f(qp.cost.D), E=f(qp.cost.E), q=-dl),
              eq=NS(A0=f(qp.eq.A0), A_minus=f(qp.eq.A_minus), A_plus=f(qp.eq.A_plus),
                    c0=np.zeros_like(f(qp.eq.c0)), c=np.zeros_like(f(qp.eq.c))),
              ineq=NS(G=f(qp.ineq.G) * sign[..., None], l=np.zeros_like(st.y_g), u=np.zeros_like(st.y_g),
                      slack_penalization_weight=0.0, use_slack_variables=False))


# ----------------------------------------------------------------- helpers ----
TRAFFIC_FILE = ROOT / "profiles" / "admm_stream_kernel_config3_pmc.txt"


def measured_traffic(batch, admm_iters):
    """HBM bytes per launch of the iteration kernel from the committed
    rocprofv3 --pmc summary (FETCH_SIZE + WRITE_SIZE, copy-calibrated), when
    the run has the shape that summary profiled (its `profiled_shape` line),
    else None."""
    traffic, shape = None, None
    try:
        for line in TRAFFIC_FILE.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch"):
                traffic = float(line.split("=")[1])
            elif line.startswith("profiled_shape"):
                f = line.split("=")[1].split()
                shape = dict(zip(f[0::2], f[1::2]))
    except (OSError, ValueError, IndexError):
        return None
    if not shape or int(shape.get("batch", -1)) != batch or int(shape.get("admm_iters", -1)) != admm_iters:
        return None
    return traffic


class SolveTimer:
    """Times ADMMSolver.solve / sqp_step calls with HIP events on the solve
    stream: the iteration phase alone (through the library's hook: two event
    records per call, the only ones in the timed region, their events made
    beforehand) and, while `whole` is set (the last warm-up step), the whole
    QP solve."""

    def __init__(self, dev):
        import torch

        from turbompc_amd import _lib
        from turbompc_amd.solvers.admm import admm as admm_mod

        self.mod, self.dev, self.torch = admm_mod, dev, torch
        self.solves = []
        self.whole = True
        self.calls = 0  # QP solves since the last clear()
        self.iters = _lib.IterationTimer()
        self.orig = (admm_mod.ADMMSolver.solve, admm_mod.ADMMSolver.sqp_step)

    def __enter__(self):
        torch = self.torch

        def timed(fn):
            def wrapper(solver, *a, **kw):
                self.calls += 1
                if not self.whole:
                    with self.iters:
                        return fn(solver, *a, **kw)
                s = torch.cuda.current_stream(self.dev)
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(s)
                with self.iters:
                    out = fn(solver, *a, **kw)
                e1.record(s)
                self.solves.append((e0, e1))
                return out
            return wrapper

        self.mod.ADMMSolver.solve = timed(self.orig[0])
        self.mod.ADMMSolver.sqp_step = timed(self.orig[1])
        return self

    def __exit__(self, *exc):
        self.mod.ADMMSolver.solve, self.mod.ADMMSolver.sqp_step = self.orig
        return False

    def clear(self):
        self.solves.clear()
        self.iters.clear()
        self.calls = 0

    def averages_s(self):
        solve_ms = [a.elapsed_time(b) for a, b in self.solves]
        iter_ms = self.iters.results()
        return sum(solve_ms) / len(solve_ms) / 1e3, sum(iter_ms) / len(iter_ms) / 1e3


def timed_steps(step, steps, warmup, timer):
    """Times `steps` calls of step() after `warmup` untimed ones.  The whole
    QP solves are timed in the last warm-up step (with no warm-up, in the
    timed steps); the timed region records only the library's iteration
    events, whose HIP events are made before it."""
    import torch

    for i in range(warmup):
        if i == warmup - 1:
            timer.clear()
        step()
    torch.cuda.synchronize()
    whole = list(timer.solves)
    per_step = timer.calls if warmup else 0
    timer.clear()
    if warmup:
        timer.whole = False
        timer.iters.reserve(per_step * steps)
        torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        out = step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    if warmup:
        timer.solves[:0] = whole
        timer.whole = True
    return elapsed, out


def base_line(metric, value, args, elapsed, dtype, data, config):
    return {
        "metric": metric, "value": value, "unit": "MPC solves/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": elapsed / args.steps * 1e3, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": dtype, "data": data, "config": config,
    }


def roofline(achieved, traffic, kernel, bytes_per_launch, avg_ms, **extra):
    r = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
         "traffic": traffic, "kernel": kernel, "algorithmic_bytes_per_launch": bytes_per_launch,
         "avg_launch_ms": avg_ms}
    r.update(extra)
    return r


# --------------------------------------------------------------- workloads ----
def run_sqp_workload(args, dev):
    """config3 (the metric) and config4: the SQP solve from the same guess."""
    import torch

    from turbompc_amd.problems import configs
    from turbompc_amd.problems.quadrotor import make_quadrotor_config

    c4 = args.workload == "config4"
    B = args.batch
    if c4:
        prob = configs.config4(B=B, seed=args.seed).to(dev, torch.float32)
    else:
        prob = make_quadrotor_config(B=B, seed=args.seed, dtype=torch.float32, device=dev)
    solver = make_solver(prob, args.sqp, args.admm_iters, args.linesearch)
    guess = solver.initial_guess()
    with SolveTimer(dev) as timer:
        elapsed, sol = timed_steps(lambda: solver.solve(guess), args.steps, args.warmup, timer)
    solve_avg_s, iter_avg_s = timer.averages_s()
    copy_calibration(args, dev)

    T = prob.horizon + 1
    if c4:  # n = 9, nx = n0 = 6, 3 box rows and 8 obstacle rows (data-carrying)
        per_qp, F, It = bytes_per_qp(T, 9, 6, 6, 11, args.admm_iters, 4, m_g=8)
        workload = (f"config 4: obstacle avoidance, double integrator nx=6 nu=3 N={prob.horizon}, 8 spheres "
                    f"(linearized rows), |u| <= 3, {args.sqp} SQP x {args.admm_iters} ADMM, ADMM state carried "
                    f"across SQP iterations, direct block-tridiagonal KKT backend")
        data = "synthetic (seeded obstacle fields: 8 spheres, start and goal on opposite faces of [-4,4]^3)"
    else:  # n = 17, nx = n0 = 13, 4 box rows
        per_qp, F, It = bytes_per_qp(T, 17, 13, 13, 4, args.admm_iters, 4)
        workload = ("config 3: quadrotor nonlinear SQP, nx=13 nu=4 N=40, RK4 dt=0.02, 5 SQP x 20 ADMM, "
                    "direct block-tridiagonal KKT backend")
        data = "synthetic (seeded quadrotor fleet: random goals, perturbed hover starts)"
    if args.linesearch:
        workload += ", merit line search (alphas 0.1 0.3 0.7 1.0) after every QP solve"
    iter_bytes = B * args.admm_iters * It  # algorithmic bytes of one iteration-kernel launch
    achieved = iter_bytes / iter_avg_s / 1e9
    qp_achieved = per_qp * B / solve_avg_s / 1e9
    finite = bool(torch.isfinite(sol.states).all() and torch.isfinite(sol.controls).all())
    label = (", config 4" if c4 else "") + (", merit line search" if args.linesearch else "")
    line = base_line(f"MPC solves/sec at B={B}{label} (1 MI355X)", B * args.steps / elapsed,
                     args, elapsed, "f32", data, {
                         "workload": workload, "batch": B, "horizon": prob.horizon, "sqp_iterations": args.sqp,
                         "admm_iterations": args.admm_iters, "parallelism": "single GPU, batch-parallel",
                         "solution_finite": finite, "kernel_only_solves_per_s": B / (args.sqp * solve_avg_s)})
    line["roofline"] = roofline(
        achieved, None if c4 else measured_traffic(B, args.admm_iters),
        f"admm_stream_kernel (one launch = {args.admm_iters} ADMM iterations of the batch)", iter_bytes,
        iter_avg_s * 1e3,
        qp_solve={"kernels": "stage_pack + factor_row + admm_stream + stage_unpack", "algorithmic_bytes": per_qp * B,
                  "avg_ms": solve_avg_s * 1e3, "achieved": qp_achieved, "frac": qp_achieved / HBM_PEAK_GBS})
    return line


def run_config5(args, dev):
    """Forward ADMM (K iterations) and the backward pass of sum |x_N|^2."""
    import torch

    from turbompc_amd.problems import configs
    from turbompc_amd.solvers.turbompc_solver import TurboMPCSolver

    B, K = args.batch, args.admm_iters
    prob = configs.config5(B=B, seed=args.seed).to(dev, torch.float64)
    solver = TurboMPCSolver(prob, sqp_params(1, K), forward_backend="admm_hip_direct",
                            backward_backend="direct_hip_kkt")
    fsolve = solver.get_differentiable_solve_function()
    guess = solver.initial_guess()
    keys = ("weights_penalization_reference_state_trajectory", "weights_penalization_control_squared")
    x0 = prob.x0.clone().requires_grad_(True)
    w = {k: v.clone().requires_grad_(True) for k, v in prob.weights_dict().items()}
    bwd_events = []
    orig_vjp = TurboMPCSolver.solve_vjp

    def timed_vjp(self, *a, **kw):
        s = torch.cuda.current_stream(dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        out = orig_vjp(self, *a, **kw)
        e1.record(s)
        bwd_events.append((e0, e1))
        return out

    def step():
        sol = fsolve(guess, {"initial_state": x0}, w)
        L = (sol.states[:, -1] ** 2).sum()
        return sol, torch.autograd.grad(L, [x0] + [w[k] for k in keys])

    TurboMPCSolver.solve_vjp = timed_vjp
    try:
        with SolveTimer(dev) as timer:
            bwd_events.clear()
            elapsed, (sol, grads) = timed_steps(step, args.steps, args.warmup, timer)
    finally:
        TurboMPCSolver.solve_vjp = orig_vjp
    solve_avg_s, iter_avg_s = timer.averages_s()
    bwd = [a.elapsed_time(b) for a, b in bwd_events[-args.steps:]]
    bwd_avg_ms = sum(bwd) / len(bwd)
    copy_calibration(args, dev)
    T = prob.horizon + 1
    per_qp, F, It = bytes_per_qp(T, 9, 6, 6, 3, K, 8)
    iter_bytes = B * K * It
    achieved = iter_bytes / iter_avg_s / 1e9
    finite = bool(all(torch.isfinite(g).all() for g in grads) and torch.isfinite(sol.states).all())
    line = base_line(f"MPC solves/sec at B={B}, config 5 forward + gradient (1 MI355X)", B * args.steps / elapsed,
                     args, elapsed, "f64",
                     "synthetic (seeded Clohessy-Wiltshire rendezvous: x0 ~ N(0, diag(100^2 I3, 0.1^2 I3)), "
                     "Q, R ~ U as learnable weights)", {
                         "workload": f"config 5: spacecraft rendezvous, Clohessy-Wiltshire nx=6 nu=3 N=100 dt=10 s "
                                     f"(exact ZOH), |u| <= 0.01, {K} ADMM iterations (direct block-tridiagonal "
                                     f"KKT), then the adjoint KKT solve and gradients of sum |x_N|^2 w.r.t. x0, Q "
                                     f"and R (direct_hip_kkt)",
                         "batch": B, "horizon": prob.horizon, "admm_iterations": K,
                         "parallelism": "single GPU, batch-parallel", "solution_finite": finite,
                         "forward_qp_solve_ms": solve_avg_s * 1e3, "backward_ms": bwd_avg_ms})
    line["roofline"] = roofline(
        achieved, None, f"admm_stream_kernel, fp64 (one launch = {K} ADMM iterations of the batch)", iter_bytes,
        iter_avg_s * 1e3,
        qp_solve={"kernels": "stage_pack + factor_row + admm_stream + stage_unpack", "algorithmic_bytes": per_qp * B,
                  "avg_ms": solve_avg_s * 1e3, "achieved": per_qp * B / solve_avg_s / 1e9,
                  "frac": per_qp * B / solve_avg_s / 1e9 / HBM_PEAK_GBS})
    return line


def run_config2(args, dev):
    """One QP solve of K ADMM iterations on the PCG Schur solve."""
    import torch

    from turbompc_amd import _lib
    from turbompc_amd.problems import configs
    from turbompc_amd.solvers.admm.admm import ADMMSolver
    from turbompc_amd.solvers.linear_systems_solvers.backends import AdmmBackend
    from turbompc_amd.solvers.qp_utils import ZShape

    B, K = args.batch, args.admm_iters
    dt = torch.float64 if args.dtype == "f64" else torch.float32
    prob = configs.config2(B=B, seed=args.seed).to(dev, dt)
    qp = prob.build_qp(*prob.initial_guess())
    _, T, n, nx, n0, m = qp.dims
    kflags = {"dpp": _lib.flag_pcg_kernel(_lib.PCG_KERNEL_DPP), "lds": _lib.flag_pcg_kernel(_lib.PCG_KERNEL_LDS),
              "chunk": _lib.FLAG_GENERIC_KERNEL}[args.pcg_kernel]
    one_launch = args.pcg_kernel != "chunk"
    solver = ADMMSolver(ZShape(T - 1, nx, n - nx), {"max_iter": 50, "tol_epsilon": 1e-6}, sigma=1e-6, max_iter=K,
                        eps_abs=1e-30, eps_rel=1e-30, check_termination_every=K + 1, adapt_rho_every=0,
                        rho_f_factor=1000.0, admm_backend=AdmmBackend.HIP_PCG, std_dynamics=True,
                        kernel_flags=kflags)
    st0 = solver.initial_state(qp, rho_bar=0.1)
    with SolveTimer(dev) as timer:
        elapsed, (_, stats, st) = timed_steps(lambda: solver.solve(qp, st0, alpha=1.0), args.steps, args.warmup,
                                              timer)
    solve_avg_s, iter_avg_s = timer.averages_s()
    copy_calibration(args, dev)
    w = 8 if dt == torch.float64 else 4
    pcg_total = int(stats.num_pcg_iters.sum())  # PCG iterations of the batch in one solve
    per_solve, phase = bytes_pcg(T, n, nx, n0, m, K, 0, w)
    _, pcg_bytes = bytes_pcg(T, n, nx, n0, m, 0, 1, w)
    phase_bytes = B * phase + pcg_total * pcg_bytes
    solve_bytes = B * (per_solve - phase) + phase_bytes
    # the one-launch kernel also builds S and Phiinv: its launch carries the
    # whole solve's algorithmic bytes; the chunk kernels carry the iteration phase
    kernel_bytes = solve_bytes if one_launch else phase_bytes
    achieved = kernel_bytes / iter_avg_s / 1e9
    # the one-launch kernels keep S, Phiinv and the PCG vectors on chip, so
    # they are bound by instruction issue, not by HBM: their roofline is the
    # algorithmic PCG flop rate against the VALU peak
    pcg_flops = pcg_total * flops_pcg_iteration(T, n)
    tflops = pcg_flops / iter_avg_s / 1e12
    finite = bool(torch.isfinite(st.x_blocks).all())
    line = base_line(f"MPC solves/sec at B={B}, config 2 PCG {args.dtype} (1 MI355X)", B * args.steps / elapsed,
                     args, elapsed, args.dtype,
                     "synthetic (seeded random stable LTI systems, spectral radius <= 1.05)", {
                         "workload": f"config 2: random stable LTI nx=12 nu=4 N=50, |x| <= 5, |u| <= 1, {K} ADMM "
                                     f"iterations on the block-tridiagonal Schur PCG (block-Jacobi preconditioner, "
                                     f"tol 1e-6, at most 50 iterations), one QP",
                         "batch": B, "horizon": T - 1, "admm_iterations": K,
                         "mean_pcg_iterations": pcg_total / (B * K),
                         "parallelism": "single GPU, batch-parallel", "solution_finite": finite})
    if one_launch:
        kernels = f"admm_pcg_{args.pcg_kernel}"
        kname = (f"{kernels}_kernel (one launch = the whole solve: S and Phiinv blocks built on chip, "
                 f"{K} ADMM iterations with their PCG solves; algorithmic bytes are the streaming model's, "
                 f"which this kernel does not move: S, Phiinv and the PCG vectors stay in LDS and registers)")
    else:
        kname = f"admm_pcg_chunk_kernel (one launch = {K} ADMM iterations with their PCG solves)"
        kernels = "schur_build + admm_pcg_chunk"
    line["config"]["pcg_kernel"] = args.pcg_kernel
    hbm = roofline(achieved, None, kname, kernel_bytes, iter_avg_s * 1e3,
                   qp_solve={"kernels": kernels, "algorithmic_bytes": solve_bytes, "avg_ms": solve_avg_s * 1e3})
    if one_launch:
        line["roofline"] = {
            "bound": "valu", "achieved": tflops, "peak": VALU_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": tflops / VALU_PEAK_TFLOPS, "traffic": None, "kernel": kname,
            "algorithmic_flops_per_launch": pcg_flops, "avg_launch_ms": iter_avg_s * 1e3,
            "flops_model": "per PCG iteration and problem 4 (3T-2) n^2 + 10 T n (S and Phiinv block products, "
                           "2 dots, 3 updates) x the PCG iterations the launch ran",
            "issue_counters": "VALU busy per SIMD 0.56, any instruction issuing 0.19 of wave cycles, 0.56 of wave "
                              "cycles waiting (barriers): profiles/admm_pcg_dpp_kernel_config2.txt (fp32)",
            "hbm_streaming_model": {"achieved": achieved, "frac": achieved / HBM_PEAK_GBS,
                                    "note": "S and Phiinv are not streamed by this kernel; a fraction above 1 "
                                            "is the on-chip reuse"},
        }
    else:
        line["roofline"] = hbm
    return line


def copy_calibration(args, dev):
    """A device-to-device copy of known size after the timed steps, for
    calibrating rocprofv3's FETCH_SIZE / WRITE_SIZE against known bytes."""
    if not args.copy_calibration:
        return
    import torch

    x = torch.ones(args.copy_calibration * (1 << 18), dtype=torch.float32, device=dev)
    y = torch.empty_like(x)
    y.copy_(x)
    torch.cuda.synchronize()


DEFAULTS = {  # batch, SQP iterations, ADMM iterations
    "config3": (4096, 5, 20),
    "config4": (16384, 8, 30),
    "config5": (2048, 1, 200),
    "config2": (1024, 1, 100),
}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", choices=tuple(DEFAULTS), default="config3",
                    help="config3 (the metric's workload) or a secondary line: config4, config5, config2")
    ap.add_argument("--batch", type=int, default=None)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--sqp", type=int, default=None, help="SQP iterations (config3 / config4)")
    ap.add_argument("--admm-iters", type=int, default=None)
    ap.add_argument("--dtype", choices=("f32", "f64"), default="f32", help="config2 only")
    ap.add_argument("--pcg-kernel", choices=("dpp", "lds", "chunk"), default="dpp",
                    help="config2 only: the one-launch kernels (dpp: a stage per 16-lane row, lds: LDS-resident) "
                         "or the chunk kernel that streams S and Phiinv")
    ap.add_argument("--linesearch", action="store_true",
                    help="config3 / config4: the merit line search after every QP solve (a secondary line)")
    ap.add_argument("--cpu-baseline", type=int, default=1)
    ap.add_argument("--cpu-budget", type=float, default=15.0, help="seconds of CPU work for the baseline sample")
    ap.add_argument("--copy-calibration", type=int, default=0,
                    help="after timing, copy this many MiB device-to-device (counter calibration under rocprofv3)")
    ap.add_argument("--secondary", type=int, default=1,
                    help="with the default workload: also run configs 4, 5 and 2 (fp32, fp64) and report them "
                         "under `secondary` (short runs, a few seconds of CPU baseline each)")
    ap.add_argument("--secondary-steps", type=int, default=5)
    ap.add_argument("--secondary-cpu-budget", type=float, default=3.0)
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build measures one GPU only (the batch of independent MPC problems would shard "
              "across GPUs with no communication in the forward solve); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    default_run = args.workload == "config3" and not args.linesearch and args.batch is None and \
        args.sqp is None and args.admm_iters is None
    B, n_sqp, K = DEFAULTS[args.workload]
    args.batch = args.batch or B
    args.sqp = args.sqp or n_sqp
    args.admm_iters = args.admm_iters or K

    import torch

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    line = run_workload(args, dev)
    if default_run and args.secondary:
        # the other configurations at their own sizes, one entry each (the
        # metric above stays config 3's)
        line["secondary"] = {}
        for name, workload, dtype in (("config4", "config4", "f32"), ("config5", "config5", "f64"),
                                      ("config2_f32", "config2", "f32"), ("config2_f64", "config2", "f64")):
            b, s_, k = DEFAULTS[workload]
            sub = argparse.Namespace(**{**vars(args), "workload": workload, "batch": b, "sqp": s_, "admm_iters": k,
                                        "dtype": dtype, "steps": args.secondary_steps, "warmup": 2,
                                        "cpu_budget": args.secondary_cpu_budget, "copy_calibration": 0})
            print(f"bench.py: secondary {name} ({b} problems, {args.secondary_steps} steps)", file=sys.stderr,
                  flush=True)
            line["secondary"][name] = run_workload(sub, dev)
    print(json.dumps(line), flush=True)


def run_workload(args, dev):
    """One bench line (with its CPU baseline) for args.workload."""
    print(f"bench.py: {args.workload} ({args.batch} problems, {args.steps} steps)", file=sys.stderr, flush=True)
    if args.workload in ("config3", "config4"):
        line = run_sqp_workload(args, dev)
    elif args.workload == "config5":
        line = run_config5(args, dev)
    else:
        line = run_config2(args, dev)
    if args.cpu_baseline and not args.linesearch:  # the CPU port times the workload without the line search
        line["cpu_baseline"] = cpu_baseline(args.workload, args.batch, args)
    return line


if __name__ == "__main__":
    main()
