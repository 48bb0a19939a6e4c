"""Batched quadratic-tracking optimal control problems (host side, torch tensors).

Follows OptimalControlProblem (turbompc/problems/optimal_control_problem.py:123-1480)
for explicit integrators and diagonal tracking weights, where the QP blocks
have closed forms:
  * cost (get_cost_linearized_blocks, :1068-1174, stage cost :982-1009, terminal
    cost :1011-1032):  D_t = 2 diag(w_x, w_u) for t < N, D_N = 2 diag(w_x + w_f, w_u),
    E = 0, q_t = -2 diag(w) z_ref_t (control reference only when
    penalize_control_reference, else 0);
  * initial condition (:914-980): A0 = [I 0], c0 = x0; with
    constrain_initial_control also the control rows [0 I], u0 (n0 = nx + nu);
  * dynamics (explicit branch, :1217-1272): A_minus_t = [df/dx, df/du],
    A_plus_t = [-I 0], c_t = -f(xbar, ubar) + A xbar + B ubar;
  * box bounds (:413-471): one G row per state/control coordinate with a finite
    bound (|b| < 1e6 on either side), l/u the bounds;
  * soft constraints (SlackProblemAdapter, :1483-1544): with
    use_slack_variables the QP carries the slack weight gamma, and the
    inequality rows are softened to l <= G z + xi <= u with cost gamma/2 |xi|^2.
Every tensor has a leading batch axis B.  Subclasses provide the dynamics.
"""
from __future__ import annotations

import ctypes
from typing import Dict, Optional, Tuple

import torch

from ..solvers.qp_data import QPCostBlocks, QPData, QPEqualityBlocks, QPInequalityBlocks, scale_qp_data

BOUND_INF = 1.0e6


def as_tensor(t, dtype, device) -> torch.Tensor:
    """t as a `dtype` tensor on `device`; Python and numpy numbers are converted
    straight to `dtype` (no detour through torch's default float32)."""
    if torch.is_tensor(t):
        return t.to(device=device, dtype=dtype)
    return torch.as_tensor(t, dtype=dtype, device=device)


class QuadraticTrackingOCP:
    """Base class: tracking cost, initial-state equality, box bounds."""

    def __init__(
        self,
        *,
        horizon: int,
        num_states: int,
        num_controls: int,
        initial_state: torch.Tensor,  # (B, nx)
        weights_state: torch.Tensor,  # (B, nx)
        weights_control: torch.Tensor,  # (B, nu)
        weights_final: torch.Tensor,  # (B, nx)
        reference_state: Optional[torch.Tensor] = None,  # (B, T, nx)
        reference_control: Optional[torch.Tensor] = None,  # (B, T, nu)
        penalize_control_reference: bool = False,
        state_bounds: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,  # (nx,), (nx,)
        control_bounds: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,  # (nu,), (nu,)
        initial_guess_final_state: Optional[torch.Tensor] = None,  # (B, nx)
        use_slack_variables: bool = False,
        slack_penalization_weight: float = 0.0,
        constrain_initial_control: bool = False,
        initial_control: Optional[torch.Tensor] = None,  # (B, nu), with constrain_initial_control
        rescale_optimization_variables: bool = False,
        state_rescaling_min: Optional[torch.Tensor] = None,  # (nx,), with rescale_optimization_variables
        state_rescaling_max: Optional[torch.Tensor] = None,
        control_rescaling_min: Optional[torch.Tensor] = None,  # (nu,)
        control_rescaling_max: Optional[torch.Tensor] = None,
        dtype: torch.dtype = torch.float64,
        device="cpu",
    ):
        self.horizon = int(horizon)
        self.num_state_variables = int(num_states)
        self.num_control_variables = int(num_controls)
        self.dtype, self.device = dtype, torch.device(device)
        cv = lambda t: as_tensor(t, dtype, self.device).contiguous()  # noqa: E731
        self.x0 = cv(initial_state)
        self.B = int(self.x0.shape[0])
        T, nx, nu = self.horizon + 1, num_states, num_controls
        self.wx, self.wu, self.wf = cv(weights_state), cv(weights_control), cv(weights_final)
        self.x_ref = cv(reference_state) if reference_state is not None else torch.zeros(
            (self.B, T, nx), dtype=dtype, device=self.device)
        self.u_ref = cv(reference_control) if reference_control is not None else torch.zeros(
            (self.B, T, nu), dtype=dtype, device=self.device)
        self.penalize_control_reference = bool(penalize_control_reference)
        inf = torch.full((nx,), BOUND_INF, dtype=dtype)
        infu = torch.full((nu,), BOUND_INF, dtype=dtype)
        xl, xu = (cv(b) for b in state_bounds) if state_bounds is not None else (-inf.to(self.device), inf.to(self.device))
        ul, uu = (cv(b) for b in control_bounds) if control_bounds is not None else (-infu.to(self.device), infu.to(self.device))
        self.x_bounds, self.u_bounds = (xl, xu), (ul, uu)
        # active rows: a finite bound on either side (optimal_control_problem.py:191-199)
        self.state_mask = (xl > -BOUND_INF) | (xu < BOUND_INF)
        self.control_mask = (ul > -BOUND_INF) | (uu < BOUND_INF)
        self.num_inequality_constraints = int(self.state_mask.sum() + self.control_mask.sum())
        self.x_final_guess = cv(initial_guess_final_state) if initial_guess_final_state is not None else self.x0
        self.use_slack_variables = bool(use_slack_variables)
        self.slack_penalization_weight = float(slack_penalization_weight)
        # u_0 = initial_control as equality rows of A0 (optimal_control_problem.py:958-978)
        self.constrain_initial_control = bool(constrain_initial_control)
        if self.constrain_initial_control and initial_control is None:
            raise ValueError("initial_control must be provided when constrain_initial_control is True.")
        self.u0 = (self._per_problem_vector("initial_control", initial_control, nu) if initial_control is not None
                   else torch.zeros((self.B, nu), dtype=dtype, device=self.device))
        if self.use_slack_variables and not self.slack_penalization_weight > 0.0:
            raise ValueError("use_slack_variables needs a positive slack_penalization_weight")
        # variable rescaling (optimal_control_problem.py:170-171, :284-349): the
        # QP is solved in x / state_diff, u / control_diff with its constraint
        # rows scaled to match; state_diff = (max - min) / 2
        self.rescale_optimization_variables = bool(rescale_optimization_variables)
        if self.rescale_optimization_variables:
            lims = {"state_rescaling_min": (state_rescaling_min, nx), "state_rescaling_max": (state_rescaling_max, nx),
                    "control_rescaling_min": (control_rescaling_min, nu),
                    "control_rescaling_max": (control_rescaling_max, nu)}
            for name, (v, k) in lims.items():
                if v is None:
                    raise ValueError(f"{name} must be provided when rescale_optimization_variables is True")
                if tuple(torch.as_tensor(v).shape) != (k,):
                    raise ValueError(f"{name} must have shape ({k},), got {tuple(torch.as_tensor(v).shape)}")
            self.state_diff = (cv(state_rescaling_max) - cv(state_rescaling_min)) / 2.0
            self.control_diff = (cv(control_rescaling_max) - cv(control_rescaling_min)) / 2.0
            if not (bool(torch.all(self.state_diff > 0)) and bool(torch.all(self.control_diff > 0))):
                raise ValueError("the rescaling ranges must satisfy max > min")
        else:
            self.state_diff = torch.ones(nx, dtype=dtype, device=self.device)
            self.control_diff = torch.ones(nu, dtype=dtype, device=self.device)
        self.std_dynamics = True  # explicit integrators: A_plus = [-I 0], E = 0
        self.diag_cost = True  # D_t = diag(2 w): per-variable tracking weights (cost_blocks)
        # the inequality rows are the box rows: the same G_t for every stage and
        # problem (inequality_blocks; subclasses with other rows clear it)
        self.const_g = True
        self._static = None
        # values derived from the problem's tensors, built on first use (copies
        # made by with_weights, with_params, to and tile start empty); like the
        # static QP blocks they assume the tensors are not changed in place
        self._memo: Dict[str, object] = {}

    def _per_problem_vector(self, name, t, k):
        """t as a (B, k) tensor: a (k,) vector is shared by the batch."""
        t = as_tensor(t, self.dtype, self.device)
        if t.shape[-1:] != (k,) or t.dim() > 2 or (t.dim() == 2 and t.shape[0] not in (1, self.B)):
            raise ValueError(f"{name} has shape {tuple(t.shape)}, expected ({k},) or ({self.B}, {k})")
        return t.expand(self.B, k).contiguous()

    def _memoized(self, key, make):
        v = self._memo.get(key)
        if v is None:
            v = self._memo[key] = make()
        return v

    def _box_rows(self):
        """(rows, idx, lo, hi): the z coordinates with a finite bound (state
        rows, then control rows) as a list and as an index tensor, and their
        bounds (m,)."""
        def make():
            nx = self.num_state_variables
            rows = [i for i in range(nx) if bool(self.state_mask[i])] + \
                [nx + j for j in range(self.num_control_variables) if bool(self.control_mask[j])]
            lo = torch.cat([self.x_bounds[0][self.state_mask], self.u_bounds[0][self.control_mask]])
            hi = torch.cat([self.x_bounds[1][self.state_mask], self.u_bounds[1][self.control_mask]])
            return rows, torch.tensor(rows, dtype=torch.long, device=self.device), lo, hi
        return self._memoized("box_rows", make)

    # ------------------------------------------------------------ blocks ----
    def cost_blocks(self):
        B, N, nx, nu = self.B, self.horizon, self.num_state_variables, self.num_control_variables
        T, n = N + 1, nx + nu
        w = torch.cat([self.wx, self.wu], dim=-1)  # (B, n)
        wN = torch.cat([self.wx + self.wf, self.wu], dim=-1)
        wt = w.unsqueeze(1).expand(B, T, n).clone()
        wt[:, N] = wN
        D = torch.diag_embed(2.0 * wt)
        E = torch.zeros((B, N, n, n), dtype=self.dtype, device=self.device)
        uref = self.u_ref if self.penalize_control_reference else torch.zeros_like(self.u_ref)
        zref = torch.cat([self.x_ref, uref], dim=-1)
        q = -2.0 * wt * zref
        return D.contiguous(), E, q.contiguous()

    def initial_equality(self):
        """(A0 (B, n0, n), c0 (B, n0)): x_0 = x0, and with
        constrain_initial_control also u_0 = u0 (n0 = nx + nu)
        (get_initial_equality_linearized_matrices, :914-980)."""
        nx, nu = self.num_state_variables, self.num_control_variables
        n0 = nx + nu if self.constrain_initial_control else nx
        A0 = torch.zeros((self.B, n0, nx + nu), dtype=self.dtype, device=self.device)
        A0[:, :, :n0] = torch.eye(n0, dtype=self.dtype, device=self.device)
        c0 = torch.cat([self.x0, self.u0], dim=1) if self.constrain_initial_control else self.x0.clone()
        return A0, c0.contiguous()

    def a_plus(self):
        nx, nu = self.num_state_variables, self.num_control_variables
        Ap = torch.zeros((self.B, self.horizon, nx, nx + nu), dtype=self.dtype, device=self.device)
        Ap[..., :nx] = -torch.eye(nx, dtype=self.dtype, device=self.device)
        return Ap

    def inequality_blocks(self):
        nx, nu = self.num_state_variables, self.num_control_variables
        rows, _, lo, hi = self._box_rows()
        T, n, m = self.horizon + 1, nx + nu, len(rows)
        G1 = torch.zeros((m, n), dtype=self.dtype, device=self.device)
        for r, col in enumerate(rows):
            G1[r, col] = 1.0
        G = G1.expand(self.B, T, m, n).contiguous()
        return G, lo.expand(self.B, T, m).contiguous(), hi.expand(self.B, T, m).contiguous()

    def dynamics_blocks(self, states: torch.Tensor, controls: torch.Tensor):
        """A_minus (B,N,nx,n), c (B,N,nx) linearized at (states, controls)."""
        raise NotImplementedError

    def dynamics_lagrangian_hessian(self, states: torch.Tensor, controls: torch.Tensor, lambdas: torch.Tensor):
        """(B,T,n,n) blocks d^2/dz_t^2 [lambda_t . f(z_t)] (zero at t = N), or None
        when the dynamics are linear (get_dynamics_lagrangian_hessian,
        optimal_control_problem.py:1334-1441)."""
        raise NotImplementedError

    def inequality_lagrangian_hessian(self, states: torch.Tensor, controls: torch.Tensor, mus: torch.Tensor):
        """(B,T,n,n) blocks sum_i mu_i d^2 g_i/dz_t^2, or None when every
        inequality row is linear, as the box rows are
        (get_inequality_lagrangian_hessian, optimal_control_problem.py:1443-1480)."""
        return None

    # ------------------------------------------------ merit-function terms ----
    def tracking_weights(self):
        """(w, zref), each (B, T, n): the per-stage weights of the tracking
        cost (w_x + w_f on the final state) and the reference (the control
        reference only with penalize_control_reference)."""
        def make():
            B, N = self.B, self.horizon
            T, n = N + 1, self.num_state_variables + self.num_control_variables
            w = torch.cat([self.wx, self.wu], dim=-1).unsqueeze(1).expand(B, T, n).clone()
            w[:, N, : self.num_state_variables] += self.wf
            uref = self.u_ref if self.penalize_control_reference else torch.zeros_like(self.u_ref)
            return w, torch.cat([self.x_ref, uref], dim=-1)
        return self._memoized("tracking_weights", make)

    def cost(self, states, controls, slacks=None):
        """(B,) cost of each problem (cost, optimal_control_problem.py:982-1066:
        sum_t w (z_t - zref_t)^2 with the final-state weight w_x + w_f), plus
        gamma/2 |slack|^2 for soft constraints (cost_with_slack, :1504-1515)."""
        w, zref = self.tracking_weights()
        e = torch.cat([states, controls], dim=-1) - zref
        c = (w * e * e).flatten(1).sum(dim=1)
        if self.use_slack_variables and slacks is not None and slacks.numel():
            c = c + 0.5 * self.slack_penalization_weight * (slacks * slacks).flatten(1).sum(dim=1)
        return c

    def cost_directional_derivative(self, states, controls, slacks, dstates, dcontrols, dslacks):
        """(B,) gradient of `cost` along the direction (dstates, dcontrols, dslacks)."""
        w, zref = self.tracking_weights()
        z = torch.cat([states, controls], dim=-1)
        d = (2.0 * w * (z - zref) * torch.cat([dstates, dcontrols], dim=-1)).flatten(1).sum(dim=1)
        if self.use_slack_variables and slacks is not None and slacks.numel():
            d = d + self.slack_penalization_weight * (slacks * dslacks).flatten(1).sum(dim=1)
        return d

    def next_states(self, states: torch.Tensor, controls: torch.Tensor) -> torch.Tensor:
        """(B, N, nx): the discrete dynamics x_{t+1} = f(x_t, u_t) for t < N."""
        raise NotImplementedError

    def equality_residuals(self, states, controls):
        """(B, T nx [+ nu]) flattened as the reference's equality_constraints
        (optimal_control_problem.py:841-912): x_0 - x0, then f(x_t, u_t) -
        x_{t+1}, then u_0 - u0 with constrain_initial_control; with rescaling
        the rows are divided by state_diff (control_diff for u_0)."""
        x0 = (states[:, 0] - self.x0).unsqueeze(1)
        h = torch.cat([x0, self.next_states(states, controls) - states[:, 1:]], dim=1)
        if self.rescale_optimization_variables:
            h = h / self.state_diff
        h = h.flatten(1)
        if self.constrain_initial_control:
            hu = controls[:, 0] - self.u0
            h = torch.cat([h, hu / self.control_diff if self.rescale_optimization_variables else hu], dim=1)
        return h

    def inequality_values(self, states, controls):
        """(g, l, u), each (B, T, m): the inequality rows g(x, u) and their
        bounds (step_inequality_constraints, :413-471)."""
        _, idx, lo, hi = self._box_rows()
        g = torch.cat([states, controls], dim=-1).index_select(-1, idx)
        lo, hi = lo.expand_as(g), hi.expand_as(g)
        if self.rescale_optimization_variables:  # rows divided by their variable's scale (:460-469)
            r = self.box_row_scale()
            g, lo, hi = g * r, lo * r, hi * r
        return g, lo, hi

    # the inequality_values form the fused merit terms reproduce (a subclass
    # that defines its own rows and has no fused form falls back to torch)
    _merit_rows_form = inequality_values

    def _merit_host_constants(self):
        """The per-row constants of tmpc_ocp_merit_terms_* as host ctypes
        arrays (read back once per problem object)."""
        def make():
            rows, _, lo, hi = self._box_rows()
            m = len(rows)
            dbl = lambda v: (ctypes.c_double * max(len(v), 1))(*[float(x) for x in v])  # noqa: E731
            out = {"mbox": m, "box_idx": (ctypes.c_int32 * max(m, 1))(*rows),
                   "box_lo": dbl(lo.tolist()), "box_hi": dbl(hi.tolist())}
            if self.rescale_optimization_variables:
                out.update(box_scale=dbl(self.box_row_scale().tolist()),
                           state_scale=dbl(self.state_diff.tolist()), control_scale=dbl(self.control_diff.tolist()))
            return out
        return self._memoized("merit_host", make)

    def _merit_linear_dynamics(self):
        """(A, Bm, b), per problem, when the merit kernel may form the
        dynamics step itself (linear dynamics); None: it reads next_states."""
        return None

    def _merit_obstacle_rows(self):
        """The obstacle rows that follow the box rows in the fused merit terms
        (dict nobs, dim, centers, radii, scale), or None: none here."""
        return None

    def merit_terms(self, states, controls, slacks=None, dstates=None, dcontrols=None, dslacks=None,
                    copies: int = 1):
        """(cost, |h|_1, |viol|_1, dcost or None), each (copies B,), for
        `copies` stacked batches (copy j at rows j B .. j B + B - 1) in one
        kernel (tmpc_ocp_merit_terms_*): the terms the merit line search
        takes from cost, cost_directional_derivative and
        evaluate_constraints_with_bounds (linesearch.py:14-178), the
        dynamics residuals from next_states.  None where this problem
        defines those terms otherwise (a subclass with inequality rows
        beyond the box rows, or its own cost or residuals), where the
        shapes exceed the kernel's limits, or off the GPU: the caller then
        evaluates the torch forms."""
        base, cls = QuadraticTrackingOCP, type(self)
        if not (states.is_cuda and cls.inequality_values is cls._merit_rows_form
                and cls.cost is base.cost and cls.equality_residuals is base.equality_residuals
                and cls.cost_directional_derivative is base.cost_directional_derivative):
            return None
        nx, nu = self.num_state_variables, self.num_control_variables
        hc = self._merit_host_constants()
        obs = self._merit_obstacle_rows()
        if (nx > 64 or nu > 64 or hc["mbox"] > 32 or states.shape[0] != copies * self.B
                or (obs is not None and obs["nobs"] > 32)):
            return None
        from .. import _lib

        dt, dev = self.dtype, states.device
        P, T = states.shape[0], states.shape[1]
        c = lambda t: t.to(device=dev, dtype=dt).contiguous() if t is not None else None  # noqa: E731
        states, controls = c(states), c(controls)
        lin = self._merit_linear_dynamics()
        if lin is None:
            nxt = (self.tile(copies) if copies > 1 else self).next_states(states, controls).to(dt).contiguous()
        else:  # the kernel forms the linear step itself
            nxt = None
            lin = tuple(c(t) for t in lin)
        w, zref = (c(t) for t in self.tracking_weights())
        soft = self.use_slack_variables and slacks is not None and slacks.numel() > 0
        slacks = c(slacks) if soft else None
        dstates, dcontrols = c(dstates), c(dcontrols)
        dslacks = c(dslacks) if soft and dslacks is not None else None
        x0 = c(self.x0)
        u0 = c(self.u0) if self.constrain_initial_control else None
        cost, eq, iq = (torch.empty(P, dtype=dt, device=dev) for _ in range(3))
        dcost = torch.empty(P, dtype=dt, device=dev) if dstates is not None else None
        args = _lib.MeritTerms(P=P, B0=self.B, T=T, nx=nx, nu=nu, mbox=hc["mbox"], states=_lib.ptr(states),
                               controls=_lib.ptr(controls), next=_lib.ptr(nxt), x0=_lib.ptr(x0), u0=_lib.ptr(u0),
                               w=_lib.ptr(w), zref=_lib.ptr(zref),
                               scaled=1 if self.rescale_optimization_variables else 0,
                               state_scale=hc.get("state_scale"), control_scale=hc.get("control_scale"),
                               box_idx=hc["box_idx"], box_lo=hc["box_lo"], box_hi=hc["box_hi"],
                               box_scale=hc.get("box_scale"), slacks=_lib.ptr(slacks),
                               gamma=float(self.slack_penalization_weight), dstates=_lib.ptr(dstates),
                               dcontrols=_lib.ptr(dcontrols), dslacks=_lib.ptr(dslacks), cost=_lib.ptr(cost),
                               dcost=_lib.ptr(dcost), eq=_lib.ptr(eq), iq=_lib.ptr(iq))
        if lin is not None:
            args.lin_A, args.lin_B, args.lin_b = (_lib.ptr(t) for t in lin)
        if obs is not None:
            centers, radii = c(obs["centers"]), c(obs["radii"])  # held until the launch
            args.nobs, args.dim, args.obs_scale = obs["nobs"], obs["dim"], obs["scale"]
            args.centers, args.radii = _lib.ptr(centers), _lib.ptr(radii)
        fn = f"tmpc_ocp_merit_terms_{_lib.suffix(dt)}"
        _lib.check(fn, getattr(_lib.load(), fn)(_lib.stream_handle(dev), ctypes.byref(args)))
        return cost, eq, iq, dcost

    # -------------------------------------------------------- parameters ----
    WEIGHT_KEYS = (
        "weights_penalization_reference_state_trajectory",
        "weights_penalization_control_squared",
        "weights_penalization_final_state",
    )

    def with_weights(self, weights: Optional[Dict[str, torch.Tensor]]) -> "QuadraticTrackingOCP":
        """Copy with the tracking weights of `weights` (keys of weights_dict; missing
        keys keep their value), as make_params_with_weights does for the
        reference's solve(..., weights)."""
        import copy

        if not weights:
            return self
        unknown = set(weights) - set(self.WEIGHT_KEYS) - {"slack_penalization_weight"}
        if unknown:
            raise KeyError(f"unknown weight keys {sorted(unknown)}; expected {self.WEIGHT_KEYS}")
        other = copy.copy(self)
        if "slack_penalization_weight" in weights:
            gamma = weights["slack_penalization_weight"]
            if torch.is_tensor(gamma) and gamma.numel() != 1:
                raise ValueError("slack_penalization_weight is one scalar shared by the batch")
            other.slack_penalization_weight = float(gamma)
        cv = lambda t, ref: as_tensor(t, self.dtype, self.device).expand_as(ref).contiguous()  # noqa: E731
        k = self.WEIGHT_KEYS
        if k[0] in weights:
            other.wx = cv(weights[k[0]], self.wx)
        if k[1] in weights:
            other.wu = cv(weights[k[1]], self.wu)
        if k[2] in weights:
            other.wf = cv(weights[k[2]], self.wf)
        other._static, other._memo = None, {}
        return other

    def with_params(self, problem_params: Optional[Dict[str, torch.Tensor]]) -> "QuadraticTrackingOCP":
        """Copy with the entries of problem_params that this problem carries
        ("initial_state": (B, nx), "initial_control": (B, nu)); others are
        ignored."""
        import copy

        if not problem_params or not ({"initial_state", "initial_control"} & set(problem_params)):
            return self
        other = copy.copy(self)
        if "initial_state" in problem_params:
            other.x0 = self._per_problem_vector("initial_state", problem_params["initial_state"],
                                                self.num_state_variables)
        if "initial_control" in problem_params:
            other.u0 = self._per_problem_vector("initial_control", problem_params["initial_control"],
                                                self.num_control_variables)
        other._static, other._memo = None, {}
        return other

    def weight_gradient(self, states, controls, dx_states, dx_controls) -> Dict[str, torch.Tensor]:
        """dL/dtheta for the tracking weights given the adjoint step dz
        (_assemble_parameter_gradient, turbompc_solver.py:930-966): the cost
        gradient sum_t 2 w (z_t - zref_t) gives d/dw grad = 2 (z_t - zref_t) per
        variable, and neither the dynamics nor the bounds depend on the
        weights, so dL/dw = -sum_t 2 (z_t - zref_t) dz_t (the final-state weight
        only at t = N)."""
        uref = self.u_ref if self.penalize_control_reference else torch.zeros_like(self.u_ref)
        ex = states - self.x_ref
        eu = controls - uref
        return {
            self.WEIGHT_KEYS[0]: -2.0 * (ex * dx_states).sum(dim=1),
            self.WEIGHT_KEYS[1]: -2.0 * (eu * dx_controls).sum(dim=1),
            self.WEIGHT_KEYS[2]: -2.0 * ex[:, -1] * dx_states[:, -1],
        }

    # ------------------------------------------------------------ rescaling ----
    def scale_states_controls(self, states, controls):
        """x / state_diff, u / control_diff with rescaling, else unchanged
        (scale_states_controls, optimal_control_problem.py:327-336)."""
        if not self.rescale_optimization_variables:
            return states, controls
        return states / self.state_diff, controls / self.control_diff

    def unscale_states_controls(self, states, controls):
        """The inverse of scale_states_controls (:338-349)."""
        if not self.rescale_optimization_variables:
            return states, controls
        return states * self.state_diff, controls * self.control_diff

    def box_row_scale(self):
        """(m_box,) 1 / the scale of the variable each box row bounds."""
        _, idx, _, _ = self._box_rows()
        return 1.0 / torch.cat([self.state_diff, self.control_diff]).index_select(0, idx)

    def inequality_row_scale(self):
        """(m,) the factors the inequality rows are multiplied by with rescaling."""
        return self.box_row_scale()

    def _rescale_qp(self, qp: QPData, num_selector_rows: int) -> QPData:
        """The QP in scaled variables: its rows scaled as the problem scales
        its constraints (initial rows by 1 / state_diff and 1 / control_diff,
        dynamics rows by 1 / state_diff, :944-956, :1324-1332; inequality rows
        by inequality_row_scale), then its columns by scale_qp_data
        (turbompc_solver.py:1151-1155).  A0 = [I 0], A_plus = [-I 0] and the box
        selector rows come out of the two scalings as they went in (r_i s_i = 1
        for the variable they select), so they are kept exact."""
        sd, cd = self.state_diff, self.control_diff
        r0 = 1.0 / torch.cat([sd, cd]) if self.constrain_initial_control else 1.0 / sd
        rd, rg = 1.0 / sd, self.inequality_row_scale()
        eq = QPEqualityBlocks(qp.eq.A0 * r0[:, None], qp.eq.A_minus * rd[:, None], qp.eq.A_plus * rd[:, None],
                              qp.eq.c0 * r0, qp.eq.c * rd)
        ineq = QPInequalityBlocks(qp.ineq.G * rg[:, None], qp.ineq.l * rg, qp.ineq.u * rg,
                                  qp.ineq.slack_penalization_weight, qp.ineq.use_slack_variables)
        out = scale_qp_data(QPData(cost=qp.cost, eq=eq, ineq=ineq), sd, cd)
        G = out.ineq.G
        if num_selector_rows:
            G = G.clone()
            G[..., :num_selector_rows, :] = qp.ineq.G[..., :num_selector_rows, :]
        return QPData(
            cost=out.cost,
            eq=QPEqualityBlocks(qp.eq.A0, out.eq.A_minus, qp.eq.A_plus, out.eq.c0, out.eq.c),
            ineq=QPInequalityBlocks(G, out.ineq.l, out.ineq.u, out.ineq.slack_penalization_weight,
                                    out.ineq.use_slack_variables),
        )

    def build_qp(self, states: torch.Tensor, controls: torch.Tensor) -> QPData:
        """QP of one SQP iteration (TurboMPCSolver._build_qp_data, turbompc_solver.py:1098-1156),
        in the scaled variables with rescaling."""
        return self._qp_with_dynamics(*self.dynamics_blocks(states, controls))

    def _qp_with_dynamics(self, Am: torch.Tensor, c: torch.Tensor) -> QPData:
        """The QP of this problem's blocks (built once) with the dynamics rows
        (A_minus, c), rescaled with rescaling."""
        if self._static is None:
            D, E, q = self.cost_blocks()
            A0, c0 = self.initial_equality()
            G, l, u = self.inequality_blocks()
            self._static = (D, E, q, A0, c0, self.a_plus(), G, l, u)
        D, E, q, A0, c0, Ap, G, l, u = self._static
        qp = QPData(
            cost=QPCostBlocks(D, E, q),
            eq=QPEqualityBlocks(A0, Am, Ap, c0, c),
            ineq=QPInequalityBlocks(G, l, u, torch.tensor(self.slack_penalization_weight, dtype=self.dtype),
                                    self.use_slack_variables),
        )
        return self._rescale_qp(qp, G.shape[2]) if self.rescale_optimization_variables else qp

    def initial_guess(self) -> Tuple[torch.Tensor, torch.Tensor]:
        """Straight line from x0 to the final guess, +1e-6; controls 1e-6
        (optimal_control_problem.py:819-839)."""
        N = self.horizon
        t = torch.arange(N + 1, dtype=self.dtype, device=self.device).view(1, N + 1, 1)
        a1, a2 = (N - t) / N, t / N
        states = self.x0.unsqueeze(1) * a1 + self.x_final_guess.unsqueeze(1) * a2 + 1e-6
        controls = torch.zeros((self.B, N + 1, self.num_control_variables), dtype=self.dtype, device=self.device) + 1e-6
        return states.contiguous(), controls.contiguous()

    def to(self, device=None, dtype=None):
        """Copy of the problem with every tensor moved/cast."""
        import copy

        other = copy.copy(self)
        dtype = dtype or self.dtype
        device = torch.device(device) if device is not None else self.device
        for k, v in list(vars(self).items()):
            if torch.is_tensor(v):
                setattr(other, k, v.to(device=device, dtype=dtype if v.is_floating_point() else v.dtype))
            elif isinstance(v, tuple) and v and torch.is_tensor(v[0]):
                setattr(other, k, tuple(t.to(device=device, dtype=dtype) for t in v))
        other.dtype, other.device, other._static, other._memo = dtype, device, None, {}
        return other

    # per-problem tensors (leading axis B); subclasses add theirs
    PER_PROBLEM = ("x0", "u0", "wx", "wu", "wf", "x_ref", "u_ref", "x_final_guess")

    def tile(self, k: int) -> "QuadraticTrackingOCP":
        """Copy holding k copies of the batch, problem b of copy j at index
        j B + b: the merit line search evaluates every step candidate of every
        problem in one pass over the k B problems."""
        import copy

        tiles = self._memoized("tiles", dict)
        if k in tiles:
            return tiles[k]
        other = copy.copy(self)
        for name in self.PER_PROBLEM:
            v = getattr(self, name)
            setattr(other, name, v.repeat(k, *([1] * (v.dim() - 1))))
        other.B, other._static, other._memo = self.B * k, None, {}
        tiles[k] = other
        return other

    @property
    def problem_params(self) -> Dict[str, torch.Tensor]:
        """The problem parameters with_params and with_weights accept, at
        their current values (the entries of the reference program's `params`
        that a solve takes, optimal_control_problem.py:123-240)."""
        out = {"initial_state": self.x0, **self.weights_dict()}
        if self.constrain_initial_control:
            out["initial_control"] = self.u0
        return out

    def weights_dict(self) -> Dict[str, torch.Tensor]:
        return {
            "weights_penalization_reference_state_trajectory": self.wx,
            "weights_penalization_control_squared": self.wu,
            "weights_penalization_final_state": self.wf,
        }


class LinearOCP(QuadraticTrackingOCP):
    """x_{t+1} = A x_t + B u_t (+ b): constant dynamics blocks, c_t = -b."""

    PER_PROBLEM = QuadraticTrackingOCP.PER_PROBLEM + ("A", "Bm", "b")

    def __init__(self, *, A: torch.Tensor, Bm: torch.Tensor, b: Optional[torch.Tensor] = None, **kw):
        super().__init__(**kw)
        B, nx, nu = self.B, self.num_state_variables, self.num_control_variables

        def per_problem(name, t, shape):
            # blocks shared by the batch ((nx, nx), (1, nx), ...) are expanded to
            # one copy per problem: the device kernels index them per problem
            t = as_tensor(t, self.dtype, self.device)
            try:
                return t.expand(shape).contiguous()
            except RuntimeError:
                raise ValueError(f"{name} of shape {tuple(t.shape)} does not broadcast to {shape}") from None

        self.A = per_problem("A", A, (B, nx, nx))
        self.Bm = per_problem("Bm", Bm, (B, nx, nu))
        self.b = per_problem("b", b if b is not None else torch.zeros(nx, dtype=self.dtype), (B, nx))

    def dynamics_lagrangian_hessian(self, states, controls, lambdas):
        return None  # linear dynamics

    def _merit_linear_dynamics(self):
        # the step of next_states, unless a subclass defines its own
        return (self.A, self.Bm, self.b) if type(self).next_states is LinearOCP.next_states else None

    def next_states(self, states, controls):
        """(B, N, nx): A x_t + B u_t + b (tmpc_linear_dynamics_* on the device: a
        batched GEMM of these tiny blocks takes milliseconds).  Every block is
        per problem and the trajectories have N + 1 stages (ValueError
        otherwise): the kernel indexes them so."""
        B, N, nx, nu = states.shape[0], self.horizon, self.num_state_variables, self.num_control_variables
        want = {"A": (self.A, (B, nx, nx)), "Bm": (self.Bm, (B, nx, nu)), "b": (self.b, (B, nx)),
                "states": (states, (B, N + 1, nx)), "controls": (controls, (B, N + 1, nu))}
        for name, (t, shape) in want.items():
            if tuple(t.shape) != shape:
                raise ValueError(f"next_states: {name} has shape {tuple(t.shape)}, expected {shape}")
        if not states.is_cuda:
            xn = torch.einsum("bij,btj->bti", self.A, states[:, :-1]) + torch.einsum("bij,btj->bti", self.Bm,
                                                                                    controls[:, :-1])
            return xn + self.b.unsqueeze(1)
        from .. import _lib

        lib = _lib.load()
        c = lambda t: t.to(self.dtype).contiguous()  # noqa: E731
        states, controls, A, Bm, b = c(states), c(controls), c(self.A), c(self.Bm), c(self.b)
        nxt = torch.empty((B, N, nx), dtype=self.dtype, device=states.device)
        fn = f"tmpc_linear_dynamics_{_lib.suffix(self.dtype)}"
        _lib.check(fn, getattr(lib, fn)(_lib.stream_handle(states.device), B, N, nx, nu, _lib.ptr(states),
                                        _lib.ptr(controls), _lib.ptr(A), _lib.ptr(Bm), _lib.ptr(b), _lib.ptr(nxt)))
        return nxt

    def dynamics_blocks(self, states, controls):
        """The constant blocks, built once: every SQP step's QP holds the same
        A_minus and c tensors, so a warm step keeps their stage records."""
        def make():
            N = self.horizon
            AB = torch.cat([self.A, self.Bm], dim=-1)  # (B, nx, n)
            Am = AB.unsqueeze(1).expand(self.B, N, *AB.shape[1:]).contiguous()
            c = (-self.b).unsqueeze(1).expand(self.B, N, self.num_state_variables).contiguous()
            return Am, c

        return self._memoized("dynamics_blocks", make)
