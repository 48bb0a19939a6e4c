"""TurboMPC SQP solver with the gfx950 HIP backends.

Mirrors turbompc/solvers/turbompc_solver.py: backend enums and name maps
(:56-191, with the new members ADMM_HIP_DIRECT / ADMM_HIP_PCG /
DIRECT_HIP_KKT), `TurboMPCSolution` (:225-237), `TurboMPCSolver(program,
params, forward_backend=, backward_backend=)` (:303-438), `initial_guess`
(:476-509), the SQP loop `_solve_impl` (:1519-1760) with the first-order
convergence check (:1158-1225) and KKT state (:1387-1439), and the backward
pass (`_build_backward_qp` :544-618, `_solve_backward_qp_direct` :706-779,
weight and initial-state gradients :781-1018).

Differences of form, not of semantics: every tensor has a leading batch axis
(the reference vmaps one problem), problems stop independently exactly as a
vmapped `lax.while_loop` does, and differentiation is exposed through
`solve_vjp` / `DifferentiableSolve` instead of `jax.custom_vjp`.
"""
from __future__ import annotations

import copy
import enum
from pathlib import Path
from typing import Any, Dict, NamedTuple, Optional, Union

import torch
import yaml

from .admm.admm import ADMMSolver, ADMMState
from .admm.admm_hip_backend import direct_workspace as admm_direct_workspace
from .linear_systems_solvers.backends import AdmmBackend, SchurSolverBackend
from .linesearch import backtracking_linesearch
from .qp_data import QPData
from .qp_ops import apply_C_parts, apply_Ct, apply_G, apply_Gt, apply_P, inf_norm
from .qp_utils import ZShape, pack_x, pack_z
from .backward.backward_kkt_hip import solve_backward_kkt_hip
from .qp_data import QPCostBlocks, QPEqualityBlocks, QPInequalityBlocks
from .sqp_hip import first_order_check, kkt_active_sets

_PARAMS_DIR = Path(__file__).resolve().parent / "params"


def load_solver_params(name: str = "turbompc.yaml") -> Dict[str, Any]:
    with open(_PARAMS_DIR / name) as f:
        return yaml.safe_load(f)


DEFAULT_SOLVER_PARAMS = load_solver_params("turbompc.yaml")


class ForwardBackend(enum.IntEnum):
    ADMM_JAX_LOOP_PCG = 0
    ADMM_JAX_LOOP_PCG_FFI = 1
    ADMM_JAX_LOOP_CUDSS_FFI = 2
    ADMM_JAX_LOOP_JAX_DENSE = 3
    ADMM_FUSED_PCG = 4
    ADMM_FUSED_CUDSS = 5
    ADMM_HIP_DIRECT = 6  # fused ADMM + block-tridiagonal factorize/solve (gfx950)
    ADMM_HIP_PCG = 7  # fused ADMM + Schur PCG (gfx950)


class BackwardBackend(enum.IntEnum):
    ADMM_JAX_LOOP_PCG = 0
    ADMM_JAX_LOOP_PCG_FFI = 1
    ADMM_JAX_LOOP_CUDSS_FFI = 2
    ADMM_JAX_LOOP_JAX_DENSE = 3
    ADMM_FUSED_PCG = 4
    ADMM_FUSED_CUDSS = 5
    DIRECT_JAX_DENSE = 6
    DIRECT_CUDSS_FFI = 7
    DIRECT_HIP_KKT = 8  # stage-block adjoint KKT factorize/solve (gfx950)


_FORWARD_BACKEND_COMPONENTS = {
    ForwardBackend.ADMM_HIP_DIRECT: (AdmmBackend.HIP_DIRECT, SchurSolverBackend.IGNORED),
    ForwardBackend.ADMM_HIP_PCG: (AdmmBackend.HIP_PCG, SchurSolverBackend.IGNORED),
}

_NAME_TO_FORWARD_BACKEND = {
    "admm_jax_loop_pcg": ForwardBackend.ADMM_JAX_LOOP_PCG,
    "admm_jax_loop_pcg_ffi": ForwardBackend.ADMM_JAX_LOOP_PCG_FFI,
    "admm_jax_loop_cudss_ffi": ForwardBackend.ADMM_JAX_LOOP_CUDSS_FFI,
    "admm_jax_loop_jax_dense": ForwardBackend.ADMM_JAX_LOOP_JAX_DENSE,
    "admm_fused_pcg": ForwardBackend.ADMM_FUSED_PCG,
    "admm_fused_cudss": ForwardBackend.ADMM_FUSED_CUDSS,
    "admm_hip_direct": ForwardBackend.ADMM_HIP_DIRECT,
    "admm_hip_pcg": ForwardBackend.ADMM_HIP_PCG,
}
_NAME_TO_BACKWARD_BACKEND = {
    "admm_jax_loop_pcg": BackwardBackend.ADMM_JAX_LOOP_PCG,
    "admm_jax_loop_pcg_ffi": BackwardBackend.ADMM_JAX_LOOP_PCG_FFI,
    "admm_jax_loop_cudss_ffi": BackwardBackend.ADMM_JAX_LOOP_CUDSS_FFI,
    "admm_jax_loop_jax_dense": BackwardBackend.ADMM_JAX_LOOP_JAX_DENSE,
    "admm_fused_pcg": BackwardBackend.ADMM_FUSED_PCG,
    "admm_fused_cudss": BackwardBackend.ADMM_FUSED_CUDSS,
    "direct_jax_dense": BackwardBackend.DIRECT_JAX_DENSE,
    "direct_cudss_ffi": BackwardBackend.DIRECT_CUDSS_FFI,
    "direct_hip_kkt": BackwardBackend.DIRECT_HIP_KKT,
}
FORWARD_BACKEND_CHOICES = tuple(sorted(_NAME_TO_FORWARD_BACKEND))
BACKWARD_BACKEND_CHOICES = tuple(sorted(_NAME_TO_BACKWARD_BACKEND))
CONVERGENCE_CRITERION_CHOICES = ("first_order", "step")


def parse_forward_backend(value: Union[str, ForwardBackend]) -> ForwardBackend:
    if isinstance(value, ForwardBackend):
        return value
    if not isinstance(value, str):
        raise TypeError(f"Expected str or ForwardBackend, got {type(value)}")
    try:
        return _NAME_TO_FORWARD_BACKEND[value.lower()]
    except KeyError as exc:
        raise ValueError(f"Unknown forward backend: {value!r}. Options: {sorted(_NAME_TO_FORWARD_BACKEND)}") from exc


def parse_backward_backend(value: Union[str, BackwardBackend]) -> BackwardBackend:
    if isinstance(value, BackwardBackend):
        return value
    if not isinstance(value, str):
        raise TypeError(f"Expected str or BackwardBackend, got {type(value)}")
    try:
        return _NAME_TO_BACKWARD_BACKEND[value.lower()]
    except KeyError as exc:
        raise ValueError(f"Unknown backward backend: {value!r}. Options: {sorted(_NAME_TO_BACKWARD_BACKEND)}") from exc


def parse_convergence_criterion(value: str) -> str:
    if not isinstance(value, str):
        raise TypeError(f"Expected str convergence criterion, got {type(value)}")
    if value.lower() not in CONVERGENCE_CRITERION_CHOICES:
        raise ValueError(f"Unknown convergence criterion: {value!r}. Options: {CONVERGENCE_CRITERION_CHOICES}")
    return value.lower()


class KKTState(NamedTuple):
    states: torch.Tensor
    controls: torch.Tensor
    slack: torch.Tensor
    y_f: torch.Tensor  # (B, T, nx)
    y_ineq: torch.Tensor
    ineq_active_lower_idx: torch.Tensor
    ineq_active_upper_idx: torch.Tensor


class SolverStats(NamedTuple):
    admm_num_iters: torch.Tensor  # (B, max_iter)
    eq_constraints_violations: torch.Tensor
    ineq_constraints_violations: torch.Tensor
    convergence_errors: torch.Tensor


class TurboMPCSolution(NamedTuple):
    states: torch.Tensor
    controls: torch.Tensor
    slack: torch.Tensor
    status: int
    num_iter: torch.Tensor  # (B,)
    convergence_error: torch.Tensor  # (B,)
    admm_iters: torch.Tensor  # (B, max_iter)
    linesearch_alphas: Optional[torch.Tensor] = None
    admm_state: Optional[ADMMState] = None
    solver_stats: Optional[SolverStats] = None
    dual_backward_guess: Optional[torch.Tensor] = None
    kkt_state: Optional[KKTState] = None
    nonfinite: Optional[torch.Tensor] = None  # (B,) bool: the returned iterate or ADMM state holds NaN or infinity


def _nonfinite(*tensors) -> torch.Tensor:
    """(B,) True where any of the batched tensors holds a NaN or an infinity."""
    bad = None
    for t in tensors:
        if t is None or t.numel() == 0:
            continue
        b = ~torch.isfinite(t).reshape(t.shape[0], -1).all(dim=1)
        bad = b if bad is None else bad | b
    return bad


def identify_active_inequalities(g, l, u, eps_abs: float, eps_rel: float):
    """min(g - l, u - g) <= eps_abs + eps_rel |bound| (turbompc_solver.py:269-292).
    The elementwise torch form; the solver runs tmpc_kkt_active_sets_*, whose
    tests hold it to active_sets_torch value for value."""
    dl, du = g - l, u - g
    use_upper = du < dl
    tol = eps_abs + eps_rel * torch.where(use_upper, u.abs(), l.abs())
    active = torch.minimum(dl, du) <= tol
    return active & ~use_upper, active & use_upper


def active_sets_torch(g, l, u, y, eps_abs: float, eps_rel: float, dual_tol: float):
    """The KKT state's active sets in torch: proximity, then the dual's sign
    where |y| > dual_tol (turbompc_solver.py:1387-1439)."""
    lo, up = identify_active_inequalities(g, l, u, eps_abs, eps_rel)
    if y is not None and y.shape[-1] > 0:
        dl, du = y < -dual_tol, y > dual_tol
        und = ~(dl | du)
        lo, up = dl | (und & lo), du | (und & up)
    return lo, up


def _where(mask: torch.Tensor, a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    return torch.where(mask.view(-1, *([1] * (a.dim() - 1))), a, b)


class TurboMPCSolver:
    """SQP solver that uses ADMM (on the GPU) for the QP subproblems."""

    STATUS_SUCCESS = 0
    STATUS_FAILED = -1

    def __init__(
        self,
        program,
        params: Optional[Dict[str, Any]] = None,
        name: str = "TurboMPCSolver",
        *,
        forward_backend: Union[str, ForwardBackend] = ForwardBackend.ADMM_HIP_DIRECT,
        backward_backend: Union[str, BackwardBackend] = BackwardBackend.DIRECT_HIP_KKT,
        use_full_hessian: bool = True,
    ):
        self._program = program
        self._name = name
        self._params = copy.deepcopy(DEFAULT_SOLVER_PARAMS if params is None else params)
        self._use_full_hessian = use_full_hessian
        self._forward_backend = parse_forward_backend(forward_backend)
        self._backward_backend = parse_backward_backend(backward_backend)
        self._convergence_criterion = parse_convergence_criterion(
            self._params.get("convergence_criterion", "first_order"))
        if self._forward_backend not in _FORWARD_BACKEND_COMPONENTS:
            raise ValueError(
                f"forward backend {self._forward_backend.name} needs the reference's JAX/CUDA stack; "
                "use 'admm_hip_direct' or 'admm_hip_pcg'")
        if self._backward_backend != BackwardBackend.DIRECT_HIP_KKT:
            raise ValueError(
                f"backward backend {self._backward_backend.name} needs the reference's JAX/CUDA stack; "
                "use 'direct_hip_kkt'")
        self._forward_admm_backend, self._forward_schur_backend = _FORWARD_BACKEND_COMPONENTS[self._forward_backend]
        # "device": the SQP loops on the device SQP step where they apply;
        # "masked": the host-masked loop everywhere (kept for cross-checks)
        self._sqp_loop = "device"
        self._zshape = ZShape(program.horizon, program.num_state_variables, program.num_control_variables)
        ap = self._params["admm"]
        self._admm_solver_fwd = ADMMSolver(
            zshape=self._zshape,
            pcg_params=ap["pcg"],
            sigma=ap["sigma"],
            max_iter=ap["max_iter"],
            eps_abs=ap.get("eps_abs", 1.0e-4),
            eps_rel=ap.get("eps_rel", 1.0e-3),
            rho_min=ap.get("rho_min", 1.0e-6),
            rho_max=ap.get("rho_max", 1.0e6),
            check_termination_every=ap.get("check_termination_every", 1),
            adapt_rho_every=ap.get("adapt_rho_every", 5),
            adaptive_rho_tolerance=ap.get("adaptive_rho_tolerance", 5.0),
            rho_f_factor=ap.get("rho_f_factor", ap.get("active_constraint_rho_factor", 1000.0)),
            admm_backend=self._forward_admm_backend,
            use_slack=bool(getattr(program, "use_slack_variables", False)),
            std_dynamics=getattr(program, "std_dynamics", None),
            diag_cost=bool(getattr(program, "diag_cost", False)),
            const_g=bool(getattr(program, "const_g", False)),
        )

    program = property(lambda self: self._program)
    params = property(lambda self: self._params)
    name = property(lambda self: self._name)
    forward_backend = property(lambda self: self._forward_backend)
    backward_backend = property(lambda self: self._backward_backend)
    # the direct adjoint solve runs no ADMM; direct backward backends report
    # these values in the reference too (turbompc_solver.py:329-334)
    backward_admm_backend = property(lambda self: AdmmBackend.JAX_LOOP)
    backward_schur_backend = property(lambda self: SchurSolverBackend.IGNORED)
    forward_admm_backend = property(lambda self: self._forward_admm_backend)
    forward_schur_backend = property(lambda self: self._forward_schur_backend)

    # ------------------------------------------------------------------ API ----
    def initial_guess(self, params=None) -> TurboMPCSolution:
        """SQP-ADMM initial guess (turbompc_solver.py:476-509)."""
        states, controls = self._program.initial_guess()
        B, max_iter = states.shape[0], self._params["num_sqp_iteration_max"]
        m = self._program.num_inequality_constraints
        z = lambda *s: torch.zeros(s, dtype=states.dtype, device=states.device)  # noqa: E731
        zi = lambda *s: torch.zeros(s, dtype=torch.int32, device=states.device)  # noqa: E731
        return TurboMPCSolution(
            states=states, controls=controls, slack=z(B, states.shape[1], m), status=self.STATUS_SUCCESS,
            num_iter=zi(B), convergence_error=z(B), admm_iters=zi(B, max_iter),
            linesearch_alphas=z(B, max_iter) if self._params.get("linesearch") else None,
            admm_state=None,
            solver_stats=SolverStats(zi(B, max_iter), z(B, max_iter), z(B, max_iter), z(B, max_iter)),
            dual_backward_guess=None, kkt_state=None,
        )

    def solve(self, initial_guess: TurboMPCSolution, problem_params=None, weights=None) -> TurboMPCSolution:
        program = self._program_for(problem_params, weights)
        return self._solve_impl(program, initial_guess.states, initial_guess.controls, initial_guess.admm_state)

    def solve_vjp(self, solution: TurboMPCSolution, dl_dstates: torch.Tensor, dl_dcontrols: torch.Tensor,
                  dl_dslack: Optional[torch.Tensor] = None, problem_params=None, weights=None):
        """Backward pass of the differentiable solve (`_solve_bwd` of
        get_differentiable_solve_function, turbompc_solver.py:1052-1084): returns
        (problem_params cotangent {"initial_state": dL/dx0 (B, nx)}, plus
        "initial_control": dL/du0 (B, nu) with constrain_initial_control
        (_build_problem_params_cotangent, :990-1018), dL/dweights {key: (B, ...)})
        for the cotangents of the solution's states and controls."""
        problem_params, weights = self._split_params(problem_params, weights)
        program = self._program_for(problem_params, weights)
        if solution.kkt_state is None:
            raise ValueError("the solution carries no KKT state (no SQP iteration ran)")
        if dl_dslack is None:
            dl_dslack = torch.zeros_like(solution.kkt_state.slack)
        ctx = self._build_backward_qp(program, solution, dl_dstates, dl_dcontrols, dl_dslack)
        res = self._solve_backward_qp_direct(program, ctx, solution, dl_dslack)
        kkt = solution.kkt_state
        dL_dw = program.weight_gradient(kkt.states, kkt.controls, res.dx_states, res.dx_controls)
        if weights and "slack_penalization_weight" in weights:
            dL_dw["slack_penalization_weight"] = res.dL_dgamma
        cot = {"initial_state": res.dL_dx_init}
        if res.dL_du_init is not None:
            cot["initial_control"] = res.dL_du_init
        return cot, dL_dw

    def get_differentiable_solve_function(self):
        """A solve(initial_guess, problem_params=None, weights=None) whose states
        and controls carry torch autograd with respect to
        problem_params["initial_state"] and the weight tensors (the custom_vjp
        of turbompc_solver.py:1020-1090)."""
        return DifferentiableSolve(self)

    def make_params_with_weights(self, weights, problem_params=None) -> Dict[str, Any]:
        """A deep copy of problem_params (of the program's own params when
        None) with the entries of `weights` merged in, nested dictionaries key
        by key (make_params_with_weights, turbompc_solver.py:511-526); the
        caller's dictionaries are not changed.  solve and solve_vjp take the
        weight keys from problem_params as from `weights`."""
        def merge(dst, src):
            for k, v in src.items():
                if isinstance(v, dict) and isinstance(dst.get(k), dict):
                    merge(dst[k], v)
                else:
                    dst[k] = v

        base = problem_params if problem_params is not None else getattr(self._program, "problem_params", {})
        out = copy.deepcopy(dict(base))
        merge(out, copy.deepcopy(dict(weights)) if weights else {})
        return out

    def linesearch(self, states, controls, slacks, states_new, controls_new, slacks_new, problem_params=None):
        """The merit line search along the SQP step (turbompc_solver.py:1480-1501):
        ((states, controls, slacks) at the accepted step, alpha (B,))."""
        program = self._program_for(problem_params, None)
        return backtracking_linesearch(program, None, self._params, states, controls, slacks, states_new,
                                       controls_new, slacks_new)

    def _split_params(self, problem_params, weights):
        """(problem_params, weights) with weight keys merged into problem_params
        (make_params_with_weights) moved to the weights."""
        if problem_params:
            wkeys = set(getattr(self._program, "WEIGHT_KEYS", ())) | {"slack_penalization_weight"}
            inline = {k: v for k, v in problem_params.items() if k in wkeys}
            if inline:
                weights = {**inline, **(weights or {})}
                problem_params = {k: v for k, v in problem_params.items() if k not in wkeys}
        return problem_params, weights

    def _program_for(self, problem_params, weights):
        problem_params, weights = self._split_params(problem_params, weights)
        program = self._program
        if weights:
            program = program.with_weights(weights)
        if problem_params:
            program = program.with_params(problem_params)
        return program

    # ---------------------------------------------------------- backward ----
    def _build_backward_qp(self, program, solution: TurboMPCSolution, dl_dstates, dl_dcontrols, dl_dslack):
        """The adjoint QP (`_build_backward_qp`, turbompc_solver.py:544-618): the QP
        at the solution with c0 = c = 0, q = -dL/dz, the active rows of G signed
        (+1 lower, -1 upper, 0 inactive) and, with use_full_hessian, the
        dynamics and inequality Lagrangian Hessians added to D (:1323-1385)."""
        kkt = solution.kkt_state
        qp = program.build_qp(kkt.states, kkt.controls)
        D = qp.cost.D
        # with rescaling the adjoint is solved in the forward QP's scaled
        # variables: the same KKT system as the reference's (unscaled variables,
        # scaled rows, turbompc_solver.py:1347-1349) with its columns scaled by
        # S, so its multipliers are the reference's and its step is S^-1 dz
        resc = self._rescaled(program)
        if resc:
            s = torch.cat([program.state_diff, program.control_diff]).to(D)
            colsym = lambda H: H * s[:, None] * s  # noqa: E731
        if self._use_full_hessian:
            lambdas = solution.admm_state.y_f_dyn if solution.admm_state is not None else kkt.y_f[:, 1:]
            if resc:  # multipliers of rows scaled by 1 / state_diff (:1372-1378)
                lambdas = lambdas / program.state_diff.to(lambdas)
            H = program.dynamics_lagrangian_hessian(kkt.states, kkt.controls, lambdas)
            if H is not None:
                D = D + (colsym(H) if resc else H)
            # mu = active * y_g (:1357-1385); None when every row is linear (bounds)
            y_g = solution.admm_state.y_g if solution.admm_state is not None else kkt.y_ineq
            active = (kkt.ineq_active_lower_idx | kkt.ineq_active_upper_idx).to(y_g.dtype)
            mus = active * y_g
            if resc:
                mus = mus * program.inequality_row_scale().to(mus)
            Hg = program.inequality_lagrangian_hessian(kkt.states, kkt.controls, mus)
            if Hg is not None:
                D = D + (colsym(Hg) if resc else Hg)
        base = QPData(cost=QPCostBlocks(D, qp.cost.E, qp.cost.q), eq=qp.eq, ineq=qp.ineq)
        eq = QPEqualityBlocks(qp.eq.A0, qp.eq.A_minus, qp.eq.A_plus, torch.zeros_like(qp.eq.c0),
                              torch.zeros_like(qp.eq.c))
        G = qp.ineq.G
        if G.shape[2] == 0:
            G_active = G
        else:
            sign = kkt.ineq_active_lower_idx.to(G.dtype) - kkt.ineq_active_upper_idx.to(G.dtype)
            G_active = G * sign.unsqueeze(-1)
        dl = pack_x(dl_dstates.to(D.dtype), dl_dcontrols.to(D.dtype))
        if resc:  # the cost's linear term in the scaled variables
            dl = dl * s
        if qp.ineq.use_slack_variables and G.shape[2] > 0:
            gamma = qp.ineq.slack_penalization_weight
            Gt = G_active.transpose(-1, -2)
            D2 = D + gamma * torch.matmul(Gt, G_active)
            shift = torch.matmul(Gt, dl_dslack.to(D.dtype).unsqueeze(-1)).squeeze(-1)
            cost = QPCostBlocks(D2, qp.cost.E, -(dl - shift))
            empty = torch.zeros(G.shape[:2] + (0,), dtype=G.dtype, device=G.device)
            ineq = QPInequalityBlocks(torch.zeros(G.shape[:2] + (0, G.shape[-1]), dtype=G.dtype, device=G.device),
                                      empty, empty, gamma, False)
        else:
            cost = QPCostBlocks(D, qp.cost.E, -dl)
            ineq = QPInequalityBlocks(G_active, torch.zeros_like(qp.ineq.l), torch.zeros_like(qp.ineq.u),
                                      qp.ineq.slack_penalization_weight, qp.ineq.use_slack_variables)
        return _BackwardQPContext(base, QPData(cost=cost, eq=eq, ineq=ineq), G_active)

    def _solve_backward_qp_direct(self, program, ctx: "_BackwardQPContext", solution: TurboMPCSolution,
                                  dl_dslack) -> "_BackwardSolveResult":
        """`_solve_backward_qp_direct` (turbompc_solver.py:706-779): one batched
        adjoint KKT solve (tmpc_adjoint_kkt_*) and the multiplier unpacking."""
        (dxs, dus), mult = solve_backward_kkt_hip(ctx.solve_qp, self._zshape,
                                                  std_dynamics=getattr(program, "std_dynamics", None))
        B, T, n, nx, n0, m = ctx.solve_qp.dims
        m_eq = n0 + (T - 1) * nx
        y_f0 = mult[:, :n0]
        y_eq_lin = mult[:, :m_eq]
        if n0 > nx:
            # constrain_initial_control: the u_0 rows' multipliers go last, as
            # in the reference's equality-constraint vector (:739-744)
            y_eq_lin = torch.cat([y_f0[:, :nx], mult[:, n0:m_eq], y_f0[:, nx:]], dim=1)
        kkt = solution.kkt_state
        dL_dgamma = torch.zeros((), dtype=mult.dtype, device=mult.device)
        base = ctx.base_qp
        if base.ineq.use_slack_variables and base.ineq.G.shape[2] > 0:
            # _recover_slack_active_ineq_gradient (:620-643)
            active = (kkt.ineq_active_lower_idx | kkt.ineq_active_upper_idx).to(mult.dtype)
            dls = dl_dslack.to(mult.dtype) * active
            dz = pack_x(dxs, dus)
            g_dz = torch.matmul(ctx.G_active, dz.unsqueeze(-1)).squeeze(-1)
            gamma = base.ineq.slack_penalization_weight
            y_ineq_lin = (dls + gamma * g_dz).flatten(1)
            sign = kkt.ineq_active_lower_idx.to(mult.dtype) - kkt.ineq_active_upper_idx.to(mult.dtype)
            dL_dgamma = (sign * kkt.slack * active * g_dz).flatten(1).sum(dim=1)
        else:
            y_ineq_lin = mult[:, m_eq:]
        # dL/dx0 and, with constrain_initial_control, dL/du0 (:765-770); with
        # rescaling the initial rows are x_0 / state_diff = x0 / state_diff
        # (and u_0 / control_diff), so the cotangents are divided by the
        # scales (:1007-1016), and the step returns to true units
        dx0, du0 = y_f0[:, :nx], (y_f0[:, nx:] if n0 > nx else None)
        if self._rescaled(program):
            dxs, dus = program.unscale_states_controls(dxs, dus)
            dx0 = dx0 / program.state_diff.to(dx0)
            if du0 is not None:
                du0 = du0 / program.control_diff.to(du0)
        return _BackwardSolveResult(dxs, dus, y_eq_lin, y_ineq_lin, dL_dgamma, dx0, du0)

    # ------------------------------------------------------------ internals ----
    def _first_order_check(self, qp: QPData, states, controls, slacks, admm_state: ADMMState):
        """_compute_first_order_convergence_error (turbompc_solver.py:1158-1225), one HIP kernel."""
        x = pack_x(states, controls)
        use_slack = bool(qp.ineq.use_slack_variables) and qp.dims[5] > 0
        return first_order_check(qp, x, admm_state.y_f_0, admm_state.y_f_dyn, admm_state.y_g,
                                 slacks if use_slack else None, float(qp.ineq.slack_penalization_weight),
                                 std_dynamics=getattr(self._program, "std_dynamics", None),
                                 diag_cost=bool(getattr(self._program, "diag_cost", False)))

    def _first_order_check_torch(self, qp: QPData, states, controls, slacks, admm_state: ADMMState):
        """Same check with torch operators; kept for validating the kernel."""
        x = pack_x(states, controls)
        stat = apply_P(qp, x) + qp.cost.q + apply_Ct(qp, admm_state.y_f_0, admm_state.y_f_dyn)
        m = qp.dims[5]
        if m:
            stat = stat + apply_Gt(qp, admm_state.y_g)
        stat_err = inf_norm(stat)
        c0x, cx = apply_C_parts(qp, x)
        eq_err = torch.maximum(inf_norm(c0x - qp.eq.c0), inf_norm(cx - qp.eq.c))
        g = apply_G(qp, x) if m else torch.zeros_like(qp.ineq.l)
        if qp.ineq.use_slack_variables:
            g = g + slacks
        if m:
            viol = torch.maximum(torch.clamp(qp.ineq.l - g, min=0.0), torch.clamp(g - qp.ineq.u, min=0.0))
            ineq_err = inf_norm(viol)
        else:
            ineq_err = torch.zeros_like(stat_err)
        conv = torch.maximum(stat_err, torch.maximum(eq_err, ineq_err))
        if qp.ineq.use_slack_variables and m:
            # slack stationarity |gamma xi + y_g| (turbompc_solver.py:1207-1212)
            slack_err = inf_norm(qp.ineq.slack_penalization_weight * slacks + admm_state.y_g)
            conv = torch.maximum(conv, slack_err)
        return conv, eq_err, ineq_err, g

    def _build_kkt_state(self, states, controls, admm_state: ADMMState, g, l, u) -> KKTState:
        """Active sets from proximity, disambiguated by the dual sign (turbompc_solver.py:1387-1439)."""
        ap = self._params["admm"]
        y_f = torch.cat([admm_state.y_f_0[:, None, : self._zshape.num_states], admm_state.y_f_dyn], dim=1)
        y_ineq = admm_state.y_g
        if getattr(self._program, "use_slack_variables", False):
            # soft constraints: the slack's sign marks the active side (:1413-1415)
            slack = admm_state.xi_g
            return KKTState(states, controls, slack, y_f, y_ineq, slack > 1.0e-12, slack < -1.0e-12)
        # proximity, then the dual's sign beyond eps_abs, in one kernel
        lo, up = kkt_active_sets(g, l, u, y_ineq if y_ineq.shape[-1] > 0 else None, ap["eps_abs"], ap["eps_rel"],
                                 ap["eps_abs"])
        return KKTState(states, controls, admm_state.xi_g, y_f, y_ineq, lo, up)

    @staticmethod
    def _rescaled(program) -> bool:
        return bool(getattr(program, "rescale_optimization_variables", False))

    @staticmethod
    def _to_qp(program, states, controls):
        """An iterate in the QP's variables (scaled with rescaling, as
        _first_order_check and _inequality_values_from_qp scale it,
        turbompc_solver.py:1174, :1235)."""
        if TurboMPCSolver._rescaled(program):
            return program.scale_states_controls(states, controls)
        return states, controls

    @staticmethod
    def _qp_x(program, states, controls):
        return pack_x(*TurboMPCSolver._to_qp(program, states, controls))

    def _g_of(self, program, qp: QPData, x_qp: Optional[torch.Tensor], states, controls) -> torch.Tensor:
        """G x (B, T, m) at the iterate (states, controls), in the QP's
        variables.  x_qp: the ADMM state's x when the iterate is that state's
        own solution (without rescaling it is the packed iterate bit for bit),
        else None.  Where G_t is one block for every stage and problem (the
        OCP box selectors) the product is one GEMM with it: exact for selector
        rows, like the batched form apply_G (a product per entry and a sum)."""
        x = x_qp if x_qp is not None and not self._rescaled(program) else self._qp_x(program, states, controls)
        G = qp.ineq.G
        if getattr(program, "const_g", False) and G.shape[2] > 0:
            B, T, n = x.shape
            return (x.reshape(B * T, n) @ G[0, 0].t()).view(B, T, G.shape[2])
        return apply_G(qp, x)

    @staticmethod
    def _from_qp(program, states, controls):
        """A QP solution's states and controls in true units (the unscaling
        after ADMMSolver.solve, turbompc_solver.py:1582-1585)."""
        if TurboMPCSolver._rescaled(program):
            return program.unscale_states_controls(states, controls)
        return states, controls

    def _solve_impl(self, program, states, controls, admm_state0: Optional[ADMMState] = None) -> TurboMPCSolution:
        """The SQP loop of turbompc_solver.py:1519-1760, batched with per-problem termination."""
        if (int(self._params["num_sqp_iteration_max"]) > 1 and self._forward_admm_backend == AdmmBackend.HIP_DIRECT
                and self._sqp_loop != "masked"):
            if self._convergence_criterion == "first_order" and not self._params.get("linesearch"):
                return self._solve_impl_device(program, states, controls, admm_state0)
            return self._solve_impl_device_ls(program, states, controls, admm_state0)
        return self._solve_impl_masked(program, states, controls, admm_state0)

    def _solve_impl_device(self, program, states, controls, admm_state0: Optional[ADMMState] = None) -> TurboMPCSolution:
        """The SQP loop with the per-problem bookkeeping on the device: from the
        second iteration on, each step is one tmpc_sqp_admm_step call that
        evaluates the first-order check of the committed iterate (the check
        the reference runs at the end of the previous iteration), applies the
        activity test conv > tol_convergence and solves the QP of the problems
        that pass it.  Stopped problems keep their iterate (zero ADMM
        iterations), so no masked commit and no host synchronisation is needed
        (one per iteration only when tol_convergence > 0, to stop early)."""
        P, ap = self._params, self._params["admm"]
        max_iter, tol = int(P["num_sqp_iteration_max"]), float(P["tol_convergence"])
        alpha = float(ap.get("relaxation_parameter", 1.0))
        admm = self._admm_solver_fwd
        B, dev, dt = states.shape[0], states.device, states.dtype
        qp = program.build_qp(states, controls)
        own_state = admm_state0 is None  # the loop may update its own state in place
        if admm_state0 is None:
            admm_state0 = admm.initial_state(qp, rho_bar=ap["rho"])  # x = 0 (turbompc_solver.py:1545-1551)
        admm_state = admm_state0
        # per-iteration records, iteration-major so that one iteration's entries
        # are one contiguous (3, B) block, written in place:
        # [:, 0] eq violation, [:, 1] ineq violation, [:, 2] convergence error
        hist = torch.zeros((max_iter, 3, B), dtype=dt, device=dev)
        # each step's iteration words (count | TMPC_ITERS_NONFINITE), written
        # by the library into its row; split once after the loop
        words = torch.zeros((max_iter, B), dtype=torch.int32, device=dev)
        ran = []  # the activity of each step that ran
        active = torch.ones(B, dtype=torch.bool, device=dev)
        conv = g_c = None
        last = 0
        step_words = words[0]
        # a workspace of the solve's own: its stage records stay valid between
        # steps, so a step whose QP differs from the previous one only in the
        # relinearized dynamics (A_minus, c) rewrites just those records
        ws = admm_direct_workspace(qp)
        # a problem whose SQP step can build its own relinearized rows (the
        # quadrotor's dynamics rows, the obstacle rows): each later QP leaves
        # them to the step, which linearizes at its input iterate -- the
        # iterate build_qp would get -- straight into the stage records as
        # well; lin holds the step's keywords
        lin = getattr(program, "step_linearization", None)
        lin = lin() if lin is not None else None
        prev = None
        for it in range(max_iter):
            sw = qp.ineq.slack_penalization_weight
            if it == 0:  # cond_fun runs the first iteration unconditionally
                (states, controls), _, admm_state = admm.solve(qp, admm_state, rho_bar=ap["rho"], alpha=alpha,
                                                                slack_weight=sw, workspace=ws,
                                                                donate_state=own_state, iters_out=words[0])
                states, controls = self._from_qp(program, states, controls)
            else:
                # the state is the loop's own from here on: updated in place
                warm = _warm_level(qp, prev)
                (states, controls), _, admm_state, (cv, e, i, g), act = admm.sqp_step(
                    qp, admm_state, active, tol, rho_bar=ap["rho"], alpha=alpha, slack_weight=sw, workspace=ws,
                    warm_records=warm is not None, warm_ineq=warm == "constraints", donate_state=True,
                    iters_out=words[it], same_dynamics=_same_dynamics(qp, prev), **(lin or {}))
                states, controls = self._from_qp(program, states, controls)
                # the check belongs to the iterate committed at it - 1 (the
                # records of a stopped problem stay zero, as in the reference)
                if it == 1:
                    torch.stack([e, i, cv], out=hist[0])
                else:
                    torch.where(active, torch.stack([e, i, cv]), hist[it - 1], out=hist[it - 1])
                # a stopped problem keeps its iterate, state and QP, so this
                # check of it repeats, value for value, the one recorded when
                # it stopped: conv and G x need no masked merge
                conv, g_c = cv, g
                active = act
                step_words = words[it]
                if tol > 0 and not bool(active.any()):
                    break  # no problem iterated in this step
            ran.append(active)
            last = it
            prev = qp
            if it + 1 < max_iter:
                qp = program.qp_for_next_step(qp) if lin is not None else program.build_qp(states, controls)
        if conv is None:
            conv = torch.full((B,), float("inf"), dtype=dt, device=dev)
        # the last committed iterate is not checked (the reference evaluates no
        # check after its final iteration): its record keeps the previous error
        # and G x at the QP it was solved on
        torch.where(active, conv, hist[last, 2], out=hist[last, 2])
        g_last = self._g_of(program, qp, admm_state.x_blocks, states, controls)
        g_c = g_last if g_c is None else torch.where(active[:, None, None], g_last, g_c)
        kkt = self._build_kkt_state(states, controls, admm_state, g_c, qp.ineq.l, qp.ineq.u)
        num_iter = torch.stack(ran).sum(dim=0, dtype=torch.int32)
        admm_iters = (words & 0x7FFFFFFF).t()
        return TurboMPCSolution(
            states=states, controls=controls, slack=admm_state.xi_g, status=self.STATUS_SUCCESS, num_iter=num_iter,
            convergence_error=conv, admm_iters=admm_iters, linesearch_alphas=None, admm_state=admm_state,
            solver_stats=SolverStats(admm_iters, hist[:, 0].t(), hist[:, 1].t(), hist[:, 2].t()), kkt_state=kkt,
            # the last step scanned every problem's state (stopped ones keep theirs)
            nonfinite=step_words < 0,
        )

    def _solve_impl_device_ls(self, program, states, controls, admm_state0: Optional[ADMMState] = None
                              ) -> TurboMPCSolution:
        """The SQP loop on the device SQP step for the merit line search and
        the `step` criterion, where the step's fused check (of the ADMM
        state's x) is not the convergence error.  With the line search the
        iterate is the blend z + alpha (z_QP - z) of the previous iterate and
        the QP solution, while the ADMM state, its own x included, is carried
        unblended (turbompc_solver.py:1591-1604); the first-order check then
        runs on the committed iterate (tmpc_sqp_first_order_*).  The `step`
        criterion takes max |z_new - z| (+ the slack step) instead.  The step
        takes the activity as given (tol None: no fused check runs): stopped
        problems are skipped (their ADMM state stays as it was) and keep their
        iterate by masked selects, and relinearizing at the committed iterate
        rebuilds a stopped problem's QP unchanged.  Same records as
        _solve_impl_masked, without its host synchronisations."""
        P, ap = self._params, self._params["admm"]
        use_ls, by_step = bool(P.get("linesearch", False)), self._convergence_criterion == "step"
        max_iter, tol = int(P["num_sqp_iteration_max"]), float(P["tol_convergence"])
        alpha = float(ap.get("relaxation_parameter", 1.0))
        admm = self._admm_solver_fwd
        B, dev, dt = states.shape[0], states.device, states.dtype
        qp = program.build_qp(states, controls)
        own_state = admm_state0 is None
        if admm_state0 is None:
            admm_state0 = admm.initial_state(qp, rho_bar=ap["rho"])  # x = 0 (turbompc_solver.py:1545-1551)
        admm_state = admm_state0
        slacks = admm_state0.xi_g.clone()  # the iterate's slack (the state's own is updated in place)
        conv = torch.full((B,), float("inf"), dtype=dt, device=dev)
        admm_iters = torch.zeros((B, max_iter), dtype=torch.int32, device=dev)
        eq_v = torch.zeros((B, max_iter), dtype=dt, device=dev)
        in_v, conv_h = torch.zeros_like(eq_v), torch.zeros_like(eq_v)
        ls_alphas = torch.zeros((B, max_iter), dtype=dt, device=dev) if use_ls else None
        num_iter = torch.zeros(B, dtype=torch.int32, device=dev)
        active = torch.ones(B, dtype=torch.bool, device=dev)
        g_c = None
        z_prev = pack_z(states, controls) if by_step else None
        ws = admm_direct_workspace(qp)
        prev = None
        for it in range(max_iter):
            sw = qp.ineq.slack_penalization_weight
            if it == 0:
                (s_new, c_new), stats, adm_new = admm.solve(qp, admm_state, rho_bar=ap["rho"], alpha=alpha,
                                                            slack_weight=sw, workspace=ws, donate_state=own_state)
                s_new, c_new = self._from_qp(program, s_new, c_new)
            else:
                active = active & (conv > tol)
                if tol > 0 and not bool(active.any()):
                    break
                warm = _warm_level(qp, prev)
                (s_new, c_new), stats, adm_new, _, _ = admm.sqp_step(
                    qp, admm_state, active, None, rho_bar=ap["rho"], alpha=alpha, slack_weight=sw, workspace=ws,
                    warm_records=warm is not None, warm_ineq=warm == "constraints", donate_state=True,
                    same_dynamics=_same_dynamics(qp, prev))
                s_new, c_new = self._from_qp(program, s_new, c_new)
            sl_new = adm_new.xi_g
            if use_ls:
                # the step (s_new, c_new, xi) - (states, controls, slacks) is
                # scaled per problem; the ADMM state is not
                (s_new, c_new, sl_new), ls_a = backtracking_linesearch(program, None, P, states, controls, slacks,
                                                                     s_new, c_new, sl_new)
            sel = lambda a, b: torch.where(active.view(-1, *([1] * (a.dim() - 1))), a, b)  # noqa: E731
            if by_step:
                z_new = pack_z(s_new, c_new)
                c_err = (z_new - z_prev).abs().amax(dim=1)
                if sl_new.shape[-1] > 0:
                    c_err = c_err + (sl_new - slacks).abs().flatten(1).amax(dim=1)
                e_err = i_err = torch.zeros_like(c_err)
                z_prev = sel(z_new, z_prev)
            if it + 1 < max_iter:
                states, controls, slacks = sel(s_new, states), sel(c_new, controls), sel(sl_new, slacks)
                prev = qp
                qp = program.build_qp(states, controls)
                if by_step:
                    g = self._g_of(program, qp, None, states, controls)
                else:
                    c_err, e_err, i_err, g = self._first_order_check(
                        qp, *self._to_qp(program, states, controls), slacks, adm_new)
            elif by_step:
                g = self._g_of(program, qp, None, s_new, c_new)
                states, controls, slacks = sel(s_new, states), sel(c_new, controls), sel(sl_new, slacks)
            else:
                # the last iterate is not checked: its record keeps the previous
                # error, and G x at the QP it was solved on
                c_err, e_err, i_err = conv, torch.zeros_like(conv), torch.zeros_like(conv)
                g = self._g_of(program, qp, None, s_new, c_new)
                states, controls, slacks = sel(s_new, states), sel(c_new, controls), sel(sl_new, slacks)
            admm_state = adm_new
            if use_ls:
                ls_alphas[:, it] = sel(ls_a, ls_alphas[:, it])
            g_c = g if g_c is None else sel(g, g_c)
            conv = sel(c_err, conv)
            admm_iters[:, it] = sel(stats.num_iter, admm_iters[:, it])
            eq_v[:, it] = sel(e_err, eq_v[:, it])
            in_v[:, it] = sel(i_err, in_v[:, it])
            conv_h[:, it] = sel(c_err, conv_h[:, it])
            num_iter = num_iter + active.to(torch.int32)
        kkt = self._build_kkt_state(states, controls, admm_state, g_c, qp.ineq.l, qp.ineq.u)
        return TurboMPCSolution(
            states=states, controls=controls, slack=admm_state.xi_g, status=self.STATUS_SUCCESS, num_iter=num_iter,
            convergence_error=conv, admm_iters=admm_iters, linesearch_alphas=ls_alphas, admm_state=admm_state,
            solver_stats=SolverStats(admm_iters, eq_v, in_v, conv_h), kkt_state=kkt,
            nonfinite=_nonfinite(states, controls, *admm_state),
        )

    def _solve_impl_masked(self, program, states, controls, admm_state0: Optional[ADMMState] = None) -> TurboMPCSolution:
        """The SQP loop with host-side commits (masked selects once a problem
        has stopped); used for the `step` criterion, single iterations, the
        PCG backend and the merit line search, whose iterate (a blend of the
        previous iterate and the QP solution, linesearch.py:54-178) differs
        from the ADMM state's primal variable."""
        P, ap = self._params, self._params["admm"]
        max_iter, tol = int(P["num_sqp_iteration_max"]), float(P["tol_convergence"])
        alpha = float(ap.get("relaxation_parameter", 1.0))
        admm = self._admm_solver_fwd
        B, dev, dt = states.shape[0], states.device, states.dtype
        qp = program.build_qp(states, controls)
        if admm_state0 is None:
            admm_state0 = admm.initial_state(qp, rho_bar=ap["rho"])  # x = 0 (turbompc_solver.py:1545-1551)
        admm_state = admm_state0
        slacks = admm_state0.xi_g
        # the SQP step is read only by the "step" criterion (and by a single
        # iteration's convergence error)
        need_step = self._convergence_criterion == "step" or max_iter == 1
        z_prev = pack_z(states, controls) if need_step else None
        conv = torch.full((B,), float("inf"), dtype=dt, device=dev)
        admm_iters = torch.zeros((B, max_iter), dtype=torch.int32, device=dev)
        eq_v = torch.zeros((B, max_iter), dtype=dt, device=dev)
        in_v = torch.zeros_like(eq_v)
        conv_h = torch.zeros_like(eq_v)
        num_iter = torch.zeros(B, dtype=torch.int32, device=dev)
        active = torch.ones(B, dtype=torch.bool, device=dev)
        g_c = None  # G x (+ slack) at each problem's last committed iterate
        use_ls = bool(P.get("linesearch", False))
        ls_alphas = torch.zeros((B, max_iter), dtype=dt, device=dev) if use_ls else None
        for it in range(max_iter):
            if it >= 1:
                active = active & (conv > tol)
                if tol > 0 and not bool(active.any()):
                    break
            # while no problem has stopped, committing is plain assignment (one
            # host sync per SQP iteration instead of a masked select per tensor)
            all_active = it == 0 or bool(active.all())
            (s_new, c_new), stats, adm_new = admm.solve(qp, admm_state, rho_bar=ap["rho"], alpha=alpha,
                                                        slack_weight=qp.ineq.slack_penalization_weight)
            s_new, c_new = self._from_qp(program, s_new, c_new)
            sl_new = adm_new.xi_g
            if use_ls:
                # the step (s_new, c_new, sl_new) - (states, controls, slacks) is
                # scaled per problem; the ADMM state (multipliers, x blocks) is not
                (s_new, c_new, sl_new), ls_a = backtracking_linesearch(program, None, P, states, controls, slacks,
                                                                     s_new, c_new, sl_new)
                ls_alphas[:, it] = ls_a if all_active else torch.where(active, ls_a, ls_alphas[:, it])
            if need_step:
                z_new = pack_z(s_new, c_new)
                step = (z_new - z_prev).abs().amax(dim=1)
                if sl_new.shape[-1] > 0:
                    step = step + (sl_new - slacks).abs().flatten(1).amax(dim=1)
            if self._convergence_criterion == "first_order" and it + 1 < max_iter:
                qp_next = program.build_qp(s_new, c_new)
                c_new_err, e_err, i_err, g = self._first_order_check(
                    qp_next, *self._to_qp(program, s_new, c_new), sl_new, adm_new)
            else:
                rebuild = self._convergence_criterion == "step" and it + 1 < max_iter
                qp_next = program.build_qp(s_new, c_new) if rebuild else qp
                c_new_err = step if (it == 0 or self._convergence_criterion == "step") else conv
                e_err = torch.zeros_like(c_new_err)
                i_err = torch.zeros_like(c_new_err)
                g = self._g_of(program, qp_next, None, s_new, c_new)
            # commit where active (vmapped while_loop semantics)
            if all_active:
                sel = lambda a, b: a  # noqa: E731
                qp = qp_next
            else:
                sel = lambda a, b: _where(active, a, b)  # noqa: E731
                qp = _select_qp(active, qp_next, qp)
            states, controls, slacks = sel(s_new, states), sel(c_new, controls), sel(sl_new, slacks)
            if need_step:
                z_prev = sel(z_new, z_prev)
            admm_state = ADMMState(*[sel(a, b) for a, b in zip(adm_new, admm_state)])
            g_c = g if g_c is None else sel(g, g_c)
            conv = sel(c_new_err, conv)
            if all_active:
                admm_iters[:, it] = stats.num_iter
                eq_v[:, it] = e_err
                in_v[:, it] = i_err
                conv_h[:, it] = c_new_err
                num_iter = num_iter + 1
            else:
                admm_iters[:, it] = torch.where(active, stats.num_iter, admm_iters[:, it])
                eq_v[:, it] = torch.where(active, e_err, eq_v[:, it])
                in_v[:, it] = torch.where(active, i_err, in_v[:, it])
                conv_h[:, it] = torch.where(active, c_new_err, conv_h[:, it])
                num_iter = num_iter + active.to(torch.int32)
        # the KKT state of each problem's last committed iterate (a per-problem
        # function of committed values, so it is formed once, after the loop)
        kkt = None
        if g_c is not None:
            kkt = self._build_kkt_state(states, controls, admm_state, g_c, qp.ineq.l, qp.ineq.u)
        return TurboMPCSolution(
            states=states, controls=controls, slack=admm_state.xi_g, status=self.STATUS_SUCCESS, num_iter=num_iter,
            convergence_error=conv, admm_iters=admm_iters, linesearch_alphas=ls_alphas, admm_state=admm_state,
            solver_stats=SolverStats(admm_iters, eq_v, in_v, conv_h), kkt_state=kkt,
            nonfinite=_nonfinite(states, controls, *admm_state),
        )


class _BackwardQPContext(NamedTuple):
    base_qp: QPData
    solve_qp: QPData
    G_active: torch.Tensor


class _BackwardSolveResult(NamedTuple):
    dx_states: torch.Tensor
    dx_controls: torch.Tensor
    y_eq_lin: torch.Tensor
    y_ineq_lin: torch.Tensor
    dL_dgamma: torch.Tensor
    dL_dx_init: torch.Tensor
    dL_du_init: Optional[torch.Tensor]


class _AttachSolution(torch.autograd.Function):
    """Attaches a computed solution's states and controls to the autograd graph
    of (x0, weights...); the backward pass is TurboMPCSolver.solve_vjp."""

    @staticmethod
    def forward(ctx, solver, sol, params, weights, keys, pkeys, *inputs):
        ctx.solver, ctx.sol, ctx.params, ctx.weights, ctx.keys, ctx.pkeys = solver, sol, params, weights, keys, pkeys
        ctx.metas = [(t.shape, t.device, t.dtype) for t in inputs]
        return sol.states.clone(), sol.controls.clone()

    @staticmethod
    def backward(ctx, g_states, g_controls):
        cot, dw = ctx.solver.solve_vjp(ctx.sol, g_states, g_controls, None, ctx.params, ctx.weights)
        grads = [cot[k] for k in ctx.pkeys] + [dw[k] for k in ctx.keys]
        # inputs shared across the batch get the batch sum of their per-problem gradients
        grads = [g.sum_to_size(shape).to(device=dev, dtype=dt) for g, (shape, dev, dt) in zip(grads, ctx.metas)]
        return (None, None, None, None, None, None, *grads)


class DifferentiableSolve:
    """Callable returned by TurboMPCSolver.get_differentiable_solve_function."""

    def __init__(self, solver: "TurboMPCSolver"):
        self._solver = solver

    def __call__(self, initial_guess: TurboMPCSolution, problem_params=None, weights=None) -> TurboMPCSolution:
        keys = tuple(weights.keys()) if weights else ()
        # differentiable problem parameters: the initial state, and the initial
        # control where the problem constrains it
        constrained_u0 = getattr(self._solver.program, "constrain_initial_control", False)
        pkeys = ("initial_state",) + (("initial_control",) if constrained_u0 else ())
        pkeys = tuple(k for k in pkeys if problem_params and problem_params.get(k) is not None)
        inputs = [torch.as_tensor(problem_params[k]) for k in pkeys] + [torch.as_tensor(weights[k]) for k in keys]
        det = lambda d: {k: (v.detach() if torch.is_tensor(v) else v) for k, v in d.items()} if d else d  # noqa: E731
        params_d, weights_d = det(problem_params), det(weights)
        with torch.no_grad():
            sol = self._solver.solve(initial_guess, params_d, weights_d)
        if not any(t.requires_grad for t in inputs):
            return sol
        states, controls = _AttachSolution.apply(self._solver, sol, params_d, weights_d, keys, pkeys, *inputs)
        return sol._replace(states=states, controls=controls)


def _warm_level(qp: QPData, prev: Optional[QPData]) -> Optional[str]:
    """How qp differs from prev, for the warm stage records of an SQP step:
    "dynamics" (at most in A_minus and c), "constraints" (also in G, l, u) or
    None (in other blocks too).  The blocks that do not depend on the
    linearization point are the same tensors (the OCP classes build them once
    per problem) and the slack weight is unchanged."""
    if prev is None:
        return None
    same = lambda a, b: a is b  # noqa: E731
    fixed = (same(qp.cost.D, prev.cost.D) and same(qp.cost.E, prev.cost.E) and same(qp.cost.q, prev.cost.q)
             and same(qp.eq.A0, prev.eq.A0) and same(qp.eq.c0, prev.eq.c0) and same(qp.eq.A_plus, prev.eq.A_plus)
             and qp.ineq.use_slack_variables == prev.ineq.use_slack_variables
             and float(qp.ineq.slack_penalization_weight) == float(prev.ineq.slack_penalization_weight))
    if not fixed:
        return None
    if same(qp.ineq.G, prev.ineq.G) and same(qp.ineq.l, prev.ineq.l) and same(qp.ineq.u, prev.ineq.u):
        return "dynamics"
    return "constraints"


def _same_dynamics(qp: QPData, prev: Optional[QPData]) -> bool:
    """Whether qp's dynamics rows (A_minus, c) are prev's tensors: linear
    dynamics, whose blocks the problem builds once (LinearOCP.dynamics_blocks)."""
    return prev is not None and qp.eq.A_minus is prev.eq.A_minus and qp.eq.c is prev.eq.c


def _same_static_blocks(qp: QPData, prev: Optional[QPData]) -> bool:
    """Whether qp differs from prev at most in A_minus and c."""
    return _warm_level(qp, prev) == "dynamics"


def _select_qp(mask: torch.Tensor, a: QPData, b: QPData) -> QPData:
    if a is b:
        return a
    pick = lambda x, y: x if x is y else _where(mask, x, y)  # noqa: E731
    return QPData(
        cost=type(a.cost)(pick(a.cost.D, b.cost.D), pick(a.cost.E, b.cost.E), pick(a.cost.q, b.cost.q)),
        eq=type(a.eq)(pick(a.eq.A0, b.eq.A0), pick(a.eq.A_minus, b.eq.A_minus), pick(a.eq.A_plus, b.eq.A_plus),
                      pick(a.eq.c0, b.eq.c0), pick(a.eq.c, b.eq.c)),
        ineq=type(a.ineq)(pick(a.ineq.G, b.ineq.G), pick(a.ineq.l, b.ineq.l), pick(a.ineq.u, b.ineq.u),
                          a.ineq.slack_penalization_weight, a.ineq.use_slack_variables),
    )
