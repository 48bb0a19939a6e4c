"""ADMM solver for box-constrained optimal-control QPs, HIP backends.

Mirrors turbompc/solvers/admm/admm.py: `ADMMState` (:27-34), `ADMMStats`
(:50-59), `ADMMSolver` (:584-1088) with `solve(qp_data, admm_state0, rho_bar,
alpha, *, slack_weight)` and `initial_state(...)`.  The reference solves one
problem and is batched with jax.vmap; here every tensor carries the batch axis
and one call solves the whole batch on the GPU with the semantics of the
reference's JAX loop (`_solve_jax_loop`, :795-1049), each problem terminating
independently.
"""
from __future__ import annotations

from typing import NamedTuple, Optional, Tuple

import torch

from ..linear_systems_solvers.backends import AdmmBackend
from ..linear_systems_solvers.schur_solver import SchurComplementMatrices
from ..qp_data import QPData, is_std_dynamics
from ..qp_utils import ZShape, pack_x, unpack_x
from . import admm_hip_backend as hip
from ... import _lib


class ADMMParams(NamedTuple):
    sigma: float
    max_iter: int
    eps_abs: float
    eps_rel: float
    rho_min: float
    rho_max: float
    check_termination_every: int
    adapt_rho_every: int
    adaptive_rho_tolerance: float
    rho_f_factor: float
    alpha: float


class ADMMState(NamedTuple):
    x_blocks: torch.Tensor  # (B, N+1, n)
    y_g: torch.Tensor  # (B, N+1, m)
    y_f_0: torch.Tensor  # (B, n0)
    y_f_dyn: torch.Tensor  # (B, N, nx)
    z_g: torch.Tensor  # (B, N+1, m)
    xi_g: torch.Tensor  # (B, N+1, m)
    rho_bar: torch.Tensor  # (B,)


class ADMMStats(NamedTuple):
    """Per-solve statistics.  The fused backends report iteration counts only,
    as the reference's fused path does (admm.py:778-792)."""

    num_iter: torch.Tensor  # (B,)
    num_pcg_iters: Optional[torch.Tensor]  # (B, max_iter) for the PCG backend
    nonfinite: Optional[torch.Tensor] = None  # (B,) bool: the output state holds NaN or infinity


def _split_iters(iters: torch.Tensor):
    """iters_out words -> (iteration counts, non-finite flags): bit 31 is
    TMPC_ITERS_NONFINITE, which makes the int32 view negative."""
    return iters & 0x7FFFFFFF, iters < 0


def compute_S_Phiinv(qp_data: QPData, rho_f, sigma: float, rho_ineq=0.0) -> SchurComplementMatrices:
    """Block-tridiagonal Schur matrix and block preconditioner (admm.py:71-154),
    evaluated on the device.  rho_ineq may be a scalar or (B,); rho_f must equal
    rho_ineq * rho_f_factor for a common factor (the reference's usage)."""
    B = qp_data.batch
    rho = torch.as_tensor(rho_ineq, dtype=qp_data.dtype, device=qp_data.device).expand(B)
    rho_f = torch.as_tensor(rho_f, dtype=qp_data.dtype, device=qp_data.device).expand(B)
    if bool(torch.all(rho == 0)):
        raise ValueError("compute_S_Phiinv on the device needs rho_ineq > 0 (rho_f is rho * rho_f_factor)")
    factor = rho_f / rho
    fac = float(factor.flatten()[0])
    if not bool(torch.allclose(factor, torch.full_like(factor, fac))):
        raise ValueError("rho_f / rho_ineq must be the same for every problem of the batch")
    S, P = hip.schur_build(qp_data, rho, sigma, fac)
    return SchurComplementMatrices(S=S, preconditioner_Phiinv=P)


class ADMMSolver:
    """ADMM loop over primal (state-control) variables (admm.py:584-1088)."""

    def __init__(
        self,
        zshape: ZShape,
        pcg_params: dict,
        *,
        schur_solver=None,
        sigma: float = 1.0e-6,
        max_iter: int = 50,
        eps_abs: float = 1.0e-5,
        eps_rel: float = 1.0e-4,
        rho_min: float = 1.0e-6,
        rho_max: float = 1.0e6,
        check_termination_every: int = 1,
        adapt_rho_every: int = 5,
        adaptive_rho_tolerance: float = 5.0,
        rho_f_factor: float = 1000.0,
        admm_backend: AdmmBackend = AdmmBackend.HIP_DIRECT,
        use_slack: bool = False,
        std_dynamics: Optional[bool] = None,
        kernel_flags: int = 0,
        diag_cost: bool = False,
        const_g: bool = False,
        invariant_a: Optional[bool] = None,
    ):
        admm_backend = AdmmBackend(admm_backend)
        if admm_backend not in (AdmmBackend.HIP_DIRECT, AdmmBackend.HIP_PCG):
            raise ValueError(
                f"ADMM backend {admm_backend.name} needs the reference's JAX/CUDA stack; use HIP_DIRECT or HIP_PCG"
            )
        self._schur_solver = schur_solver
        self._pcg_params = dict(pcg_params)
        self._sigma = float(sigma)
        self._max_iter = int(max_iter)
        self._eps_abs = float(eps_abs)
        self._eps_rel = float(eps_rel)
        self._rho_min = float(rho_min)
        self._rho_max = float(rho_max)
        self._check_termination_every = int(check_termination_every)
        self._adapt_rho_every = int(adapt_rho_every)
        self._adaptive_rho_tolerance = float(adaptive_rho_tolerance)
        self._rho_f_factor = float(rho_f_factor)
        self._admm_backend = admm_backend
        self._use_slack = bool(use_slack)
        self._zshape = zshape
        self._std_dynamics = std_dynamics
        self._kernel_flags = int(kernel_flags)  # _lib.FLAG_GENERIC_KERNEL / flag_stream_p (cross-checks)
        if diag_cost:  # the caller vouches that every D_t is diagonal
            self._kernel_flags |= _lib.FLAG_DIAG_COST
        if const_g:  # the caller vouches that G_t is the same for every stage and problem
            self._kernel_flags |= _lib.FLAG_CONST_G
        # the stage-invariant A_minus entries stay resident (found on the
        # device; exact, so on by default wherever the G rows are resident)
        if const_g if invariant_a is None else invariant_a:
            self._kernel_flags |= _lib.FLAG_INVARIANT_A

    # properties of the reference solver
    schur_solver = property(lambda self: self._schur_solver)
    sigma = property(lambda self: self._sigma)
    max_iter = property(lambda self: self._max_iter)
    eps_abs = property(lambda self: self._eps_abs)
    eps_rel = property(lambda self: self._eps_rel)
    rho_min = property(lambda self: self._rho_min)
    rho_max = property(lambda self: self._rho_max)
    check_termination_every = property(lambda self: self._check_termination_every)
    adapt_rho_every = property(lambda self: self._adapt_rho_every)
    adaptive_rho_tolerance = property(lambda self: self._adaptive_rho_tolerance)
    rho_f_factor = property(lambda self: self._rho_f_factor)
    admm_backend = property(lambda self: self._admm_backend)

    def _cfg(self, alpha: float, flags: int) -> _lib.AdmmCfg:
        return hip.cfg_struct(
            max_iter=self._max_iter,
            check_every=self._check_termination_every,
            adapt_rho_every=self._adapt_rho_every,
            pcg_max_iter=int(self._pcg_params.get("max_iter", 200)),
            use_slack=self._use_slack,
            flags=flags,
            sigma=self._sigma,
            eps_abs=self._eps_abs,
            eps_rel=self._eps_rel,
            rho_min=self._rho_min,
            rho_max=self._rho_max,
            adaptive_rho_tolerance=self._adaptive_rho_tolerance,
            rho_f_factor=self._rho_f_factor,
            alpha=alpha,
            pcg_eps=float(self._pcg_params.get("tol_epsilon", 1e-8)),
        )

    def solve(
        self,
        qp_data: QPData,
        admm_state0: Optional[ADMMState] = None,
        rho_bar: float = 1.0,
        alpha: float = 1.0,
        *,
        slack_weight=0.0,
        workspace: Optional[torch.Tensor] = None,
        donate_state: bool = False,
        iters_out: Optional[torch.Tensor] = None,
    ) -> Tuple[Tuple[torch.Tensor, torch.Tensor], ADMMStats, ADMMState]:
        """`workspace` (direct backend): a caller-owned workspace instead of the
        shared cached one (an SQP loop passes its own, see sqp_step).
        donate_state: admm_state0's buffers may be updated in place (the caller
        does not read admm_state0 again).  iters_out: a zero-filled (B,) int32
        device buffer for the raw iteration words (count | TMPC_ITERS_NONFINITE
        in bit 31); the caller then splits them (the returned stats carry
        num_iter and nonfinite None)."""
        if not qp_data.cost.D.is_cuda:
            raise ValueError("ADMMSolver (HIP backends) needs device tensors; there is no CPU path")
        state0 = self.initial_state(qp_data, rho_bar=rho_bar) if admm_state0 is None else admm_state0
        std = self._std_dynamics if self._std_dynamics is not None else is_std_dynamics(qp_data)
        cfg = self._cfg(alpha, (_lib.FLAG_STD_DYNAMICS if std else 0) | self._kernel_flags)
        sw = slack_weight if self._use_slack else None
        outs, iters, pcg_iters = hip.admm_hip_solve(
            qp_data,
            state0,
            schur="direct" if self._admm_backend == AdmmBackend.HIP_DIRECT else "pcg",
            cfg=cfg,
            slack_weight=sw,
            want_pcg_iters=self._admm_backend == AdmmBackend.HIP_PCG,
            workspace=workspace,
            donate=donate_state and admm_state0 is not None,
            iters_out=iters_out,
        )
        x, z, yg, y0, yf, xi, rho = outs
        state = ADMMState(x_blocks=x, y_g=yg, y_f_0=y0, y_f_dyn=yf, z_g=z, xi_g=xi, rho_bar=rho)
        states, controls = unpack_x(x, self._zshape)
        iters, bad = _split_iters(iters) if iters_out is None else (None, None)
        return (states, controls), ADMMStats(num_iter=iters, num_pcg_iters=pcg_iters, nonfinite=bad), state

    def sqp_step(self, qp_data: QPData, admm_state0: ADMMState, active: torch.Tensor, tol: Optional[float],
                 rho_bar: float = 1.0, alpha: float = 1.0, *, slack_weight=0.0,
                 workspace: Optional[torch.Tensor] = None, warm_records: bool = False,
                 warm_ineq: bool = False, donate_state: bool = False, iters_out: Optional[torch.Tensor] = None,
                 quadrotor=None, obstacles=None, same_dynamics: bool = False):
        """One device SQP step (tmpc_sqp_admm_step_*): the first-order check of
        admm_state0's iterate against qp_data, the activity test
        active & (conv > tol), and the solve of the problems that pass it (the
        others keep their state and report 0 iterations).  warm_records: the
        caller vouches that `workspace` holds the records of the previous call
        on it, whose output is admm_state0, and that qp_data differs from that
        call's QP only in A_minus and c (FLAG_WARM_RECORDS); with warm_ineq
        also in G, l and u (FLAG_WARM_INEQ); with same_dynamics A_minus and
        c are that call's too (FLAG_WARM_SAME_DYNAMICS: their rows are kept).
        donate_state:
        admm_state0's buffers may be updated in place.  tol None: the
        activity is given (no check; the problems where `active` is False keep
        their state, and the check outputs are None).  iters_out: as in
        solve (raw iteration words, stats num_iter and nonfinite None).
        quadrotor = (dt, params): qp_data's A_minus and c are outputs, built
        by the step as the quadrotor's linearization at admm_state0's x
        (QuadrotorOCP.qp_for_next_step; tmpc_sqp_admm_step_quadrotor_*).
        obstacles (admm_hip_backend.ObstacleRows): the obstacle rows of
        qp_data's G, l and u are outputs in the same way
        (ObstacleOCP.qp_for_next_step; tmpc_sqp_admm_step_obstacle_*).  Returns
        ((states, controls), stats, state, (conv, eq_err, ineq_err, g), active_out)."""
        if self._admm_backend != AdmmBackend.HIP_DIRECT:
            raise ValueError("sqp_step needs the direct Schur solve (HIP_DIRECT)")
        if warm_records and workspace is None:
            raise ValueError("warm_records needs the caller's workspace")
        std = self._std_dynamics if self._std_dynamics is not None else is_std_dynamics(qp_data)
        flags = (_lib.FLAG_STD_DYNAMICS if std else 0) | self._kernel_flags
        if warm_records:
            flags |= _lib.FLAG_WARM_RECORDS
            if warm_ineq:
                flags |= _lib.FLAG_WARM_INEQ
            if same_dynamics and quadrotor is None:
                flags |= _lib.FLAG_WARM_SAME_DYNAMICS
        cfg = self._cfg(alpha, flags)
        sw = slack_weight if self._use_slack else None
        outs, iters, _, (conv, eq, iq, g, act) = hip.admm_hip_solve(
            qp_data, admm_state0, schur="direct", cfg=cfg, slack_weight=sw, sqp=(active, tol), workspace=workspace,
            donate=donate_state, iters_out=iters_out, quadrotor=quadrotor, obstacles=obstacles)
        x, z, yg, y0, yf, xi, rho = outs
        state = ADMMState(x_blocks=x, y_g=yg, y_f_0=y0, y_f_dyn=yf, z_g=z, xi_g=xi, rho_bar=rho)
        states, controls = unpack_x(x, self._zshape)
        iters, bad = _split_iters(iters) if iters_out is None else (None, None)
        return ((states, controls), ADMMStats(num_iter=iters, num_pcg_iters=None, nonfinite=bad), state,
                (conv, eq, iq, g), act)

    def initial_state(
        self,
        qp_data: QPData,
        rho_bar=1.0,
        states0: Optional[torch.Tensor] = None,
        controls0: Optional[torch.Tensor] = None,
    ) -> ADMMState:
        """x = (states0, controls0) (zeros by default), z = clip(G x, l, u), duals 0
        (admm.py:1051-1088)."""
        B, T, n, nx, n0, m = qp_data.dims
        dt, dev = qp_data.dtype, qp_data.device
        zs = self._zshape
        x_zero = states0 is None and controls0 is None  # then G x = 0 needs no product
        if x_zero:
            x0 = torch.zeros((B, T, n), dtype=dt, device=dev)
        else:
            if states0 is None:
                states0 = torch.zeros((B, T, zs.num_states), dtype=dt, device=dev)
            if controls0 is None:
                controls0 = torch.zeros((B, T, zs.num_controls), dtype=dt, device=dev)
            x0 = pack_x(states0.to(dt), controls0.to(dt)).contiguous()
        if m == 0:
            z0 = torch.zeros((B, T, 0), dtype=dt, device=dev)
        elif x_zero:
            z0 = torch.minimum(qp_data.ineq.l.to(dt).clamp(min=0.0), qp_data.ineq.u.to(dt))
        else:
            gx = (qp_data.ineq.G * x0.unsqueeze(-2)).sum(-1)
            z0 = torch.minimum(torch.maximum(gx, qp_data.ineq.l), qp_data.ineq.u)
        return ADMMState(
            x_blocks=x0,
            y_g=torch.zeros_like(z0),
            y_f_0=torch.zeros((B, n0), dtype=dt, device=dev),
            y_f_dyn=torch.zeros((B, T - 1, nx), dtype=dt, device=dev),
            z_g=z0.contiguous(),
            xi_g=torch.zeros_like(z0),
            rho_bar=torch.full((B,), float(rho_bar), dtype=dt, device=dev)
            if not torch.is_tensor(rho_bar)
            else rho_bar.to(dt).expand(B).contiguous(),
        )
