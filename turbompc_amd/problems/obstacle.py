"""Linear-dynamics tracking OCP with spherical obstacle-avoidance constraints.

Follows OptimalControlProblemObstacle (turbompc/problems/obstacle_avoidance.py:13-52)
and its slack variant OptimalControlProblemObstacleSlack (:55, through
make_slack_problem, optimal_control_problem.py:1539-1544): every stage carries
the box rows of the base problem followed by one row per obstacle,
    g_k(x) = 1 - |p - c_k| / (r_k + 0.001) <= 0      (l = -1e9, u = 0),
with p the first `obstacles_dimension` state coordinates.  The obstacle rows
are linearized at each SQP iterate on the device (tmpc_obstacle_linearize_*);
the backward pass adds their Lagrangian Hessian (tmpc_obstacle_lagrangian_hessian_*).
"""
from __future__ import annotations

import torch

from .. import _lib
from ..solvers.qp_data import QPCostBlocks, QPData, QPEqualityBlocks, QPInequalityBlocks
from .ocp import LinearOCP, as_tensor


class ObstacleOCP(LinearOCP):
    PER_PROBLEM = LinearOCP.PER_PROBLEM + ("centers", "radii")

    def __init__(self, *, obstacles_centers: torch.Tensor, obstacles_radii: torch.Tensor,
                 obstacles_dimension: int = 3, **kw):
        """obstacles_centers (B, K, dim) or (K, dim); obstacles_radii (B, K) or (K,)."""
        super().__init__(**kw)
        self.const_g = False  # the obstacle rows are relinearized per problem and stage
        c = as_tensor(obstacles_centers, self.dtype, self.device)
        r = as_tensor(obstacles_radii, self.dtype, self.device)
        self.obstacles_dimension = int(obstacles_dimension)
        if c.dim() == 2:
            c = c.unsqueeze(0).expand(self.B, *c.shape)
        if r.dim() == 1:
            r = r.unsqueeze(0).expand(self.B, r.shape[0])
        if c.shape[0] != self.B or c.shape[-1] != self.obstacles_dimension or r.shape != c.shape[:2]:
            raise ValueError(f"obstacle shapes {tuple(c.shape)}, {tuple(r.shape)} do not match B={self.B}, "
                             f"dim={self.obstacles_dimension}")
        if not 1 <= self.obstacles_dimension <= self.num_state_variables:
            raise ValueError("obstacles_dimension must lie in [1, nx]")
        self.centers, self.radii = c.contiguous(), r.contiguous()
        self.num_obstacles = int(c.shape[1])
        self.num_box_constraints = self.num_inequality_constraints
        self.num_inequality_constraints = self.num_box_constraints + self.num_obstacles

    def _call(self, name: str, states: torch.Tensor, *tensors: torch.Tensor):
        if not states.is_cuda:
            raise ValueError("ObstacleOCP linearization runs on the GPU; pass device tensors")
        lib = _lib.load()
        sfx = _lib.suffix(self.dtype)
        fn = f"{name}_{sfx}"
        st = getattr(lib, fn)(
            _lib.stream_handle(states.device), self.B, self.horizon, self.num_state_variables,
            self.num_control_variables, self.obstacles_dimension, self.num_obstacles, _lib.ptr(states),
            _lib.ptr(self.centers), _lib.ptr(self.radii), self.num_inequality_constraints, self.num_box_constraints,
            *[_lib.ptr(t) for t in tensors],
        )
        _lib.check(fn, st)

    def inequality_blocks_at(self, states: torch.Tensor, controls: torch.Tensor, box=None):
        """G (B,T,m,n), l, u (B,T,m): the box rows, then the obstacle rows
        linearized at (states, controls)."""
        nx, nu = self.num_state_variables, self.num_control_variables
        T, n, m, mb = self.horizon + 1, nx + nu, self.num_inequality_constraints, self.num_box_constraints
        if box is None:
            box = super().inequality_blocks()
        Gb, lb, ub = box
        states = states.to(self.dtype).contiguous()
        G = torch.empty((self.B, T, m, n), dtype=self.dtype, device=states.device)
        l = torch.empty((self.B, T, m), dtype=self.dtype, device=states.device)
        u = torch.empty_like(l)
        if mb:
            G[:, :, :mb] = Gb
            l[:, :, :mb] = lb
            u[:, :, :mb] = ub
        self._call("tmpc_obstacle_linearize", states, G, l, u)
        return G, l, u

    def inequality_blocks(self):
        raise NotImplementedError("obstacle rows depend on the iterate; use inequality_blocks_at(states, controls)")

    def step_linearization(self):
        """The keywords of an SQP step that builds the obstacle rows itself
        (ADMMSolver.sqp_step(obstacles=...), tmpc_sqp_admm_step_obstacle_*), or
        None with rescaling (the step writes the unscaled rows) or without
        obstacles."""
        if self.rescale_optimization_variables or self.num_obstacles == 0:
            return None
        from ..solvers.admm.admm_hip_backend import ObstacleRows

        return {"obstacles": ObstacleRows(self.obstacles_dimension, self.num_obstacles, self.centers, self.radii,
                                          self.num_box_constraints)}

    def qp_for_next_step(self, prev: QPData) -> QPData:
        """The QP of the next SQP iteration with its obstacle rows left to the
        step that solves it: prev itself, the previous step's QP (from
        build_qp or from here).  Its other blocks do not depend on the
        iterate (the dynamics blocks are built once), and the step overwrites
        the obstacle rows of its G, l and u with the linearization at the
        step's input iterate, the ADMM state's x (the iterate build_qp would
        be given); their box rows stay."""
        return prev

    def inequality_values(self, states, controls):
        """(g, l, u): the box rows, then g_k = 1 - |p - c_k| / (r_k + 0.001) with
        bounds (-1e9, 0) (obstacle_avoidance.py:16-52)."""
        g, lo, hi = super().inequality_values(states, controls)
        d = states[..., None, : self.obstacles_dimension] - self.centers[:, None]
        go = 1.0 - torch.linalg.norm(d, dim=-1) / (self.radii[:, None] + 0.001)
        glo, ghi = torch.full_like(go, -1.0e9), torch.zeros_like(go)
        if self.rescale_optimization_variables:
            ro = 1.0 / self.state_diff[: self.obstacles_dimension].mean()
            go, glo, ghi = go * ro, glo * ro, ghi * ro
        return torch.cat([g, go], dim=-1), torch.cat([lo, glo], dim=-1), torch.cat([hi, ghi], dim=-1)

    _merit_rows_form = inequality_values  # the fused merit terms' obstacle rows reproduce it

    def _merit_obstacle_rows(self):
        """The obstacle rows of inequality_values for the fused merit terms; the
        row scale 1 / mean(state_diff[:dim]) read back once per problem."""
        def make():
            if not self.rescale_optimization_variables:
                return 1.0
            return float(1.0 / self.state_diff[: self.obstacles_dimension].mean())
        return {"nobs": self.num_obstacles, "dim": self.obstacles_dimension, "centers": self.centers,
                "radii": self.radii, "scale": self._memoized("merit_obs_scale", make)}

    def inequality_lagrangian_hessian(self, states, controls, mus):
        """(B, T, n, n): sum_k mu_k d^2 g_k/dz^2 of the obstacle rows (box rows are linear)."""
        states = states.to(self.dtype).contiguous()
        mus = mus.to(self.dtype).contiguous()
        n = self.num_state_variables + self.num_control_variables
        H = torch.empty((self.B, self.horizon + 1, n, n), dtype=self.dtype, device=states.device)
        self._call("tmpc_obstacle_lagrangian_hessian", states, mus, H)
        return H

    def build_qp(self, states: torch.Tensor, controls: torch.Tensor) -> QPData:
        if self._static is None:
            D, E, q = self.cost_blocks()
            A0, c0 = self.initial_equality()
            box = super().inequality_blocks()
            self._static = (D, E, q, A0, c0, self.a_plus(), box)
        D, E, q, A0, c0, Ap, box = self._static
        Am, c = self.dynamics_blocks(states, controls)
        G, l, u = self.inequality_blocks_at(states, controls, box)
        qp = QPData(
            cost=QPCostBlocks(D, E, q),
            eq=QPEqualityBlocks(A0, Am, Ap, c0, c),
            ineq=QPInequalityBlocks(G, l, u, torch.tensor(self.slack_penalization_weight, dtype=self.dtype),
                                    self.use_slack_variables),
        )
        return self._rescale_qp(qp, self.num_box_constraints) if self.rescale_optimization_variables else qp

    def inequality_row_scale(self):
        """Box rows as the base class; each obstacle row by 1 / the mean scale of
        the position coordinates (obstacle_avoidance.py:42-47)."""
        ro = 1.0 / self.state_diff[: self.obstacles_dimension].mean()
        return torch.cat([self.box_row_scale(), ro.expand(self.num_obstacles)])


__all__ = ["ObstacleOCP"]
