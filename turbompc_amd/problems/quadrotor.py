"""Rotor-thrust quadrotor OCP whose SQP linearization runs on the GPU.

Model (fixed here; the reference's own quadrotor, turbompc/dynamics/quadrotor_dynamics.py,
takes thrust/torque inputs): state x = [p (3), q = (w, x, y, z) (4), v (3),
omega (3)], input f = four rotor thrusts of an x-configuration with rotors at
(+-arm/sqrt2, +-arm/sqrt2), spin directions (-, +, -, +):
  p' = v,  q' = 1/2 q (x) (0, omega),
  v' = R(q) e_z (sum f) / mass - g e_z,
  omega' = J^{-1} (tau - omega x J omega),
  tau = (d (f0 + f1 - f2 - f3), d (f1 + f2 - f0 - f3), k (f1 + f3 - f0 - f2)),  d = arm/sqrt2,
discretized by RK4 (turbompc/dynamics/integrators.py:67-76) with the control
held over the step.  Jacobians come from tmpc_quadrotor_linearize_* (forward-mode
dual numbers on the device).
"""
from __future__ import annotations

import ctypes
import math
from typing import Optional

import torch

from .. import _lib
from ..solvers.qp_data import QPData
from .ocp import QuadraticTrackingOCP

# mass [kg], Jxx, Jyy, Jzz [kg m^2], arm [m], yaw-moment coefficient [m], g [m/s^2]
QUAD_PARAMS = (1.0, 0.01, 0.01, 0.02, 0.15, 0.016, 9.81)


def hover_thrust(params=QUAD_PARAMS) -> float:
    return params[0] * params[6] / 4.0


class QuadrotorOCP(QuadraticTrackingOCP):
    def __init__(self, *, dt: float = 0.02, params=QUAD_PARAMS, **kw):
        super().__init__(num_states=13, num_controls=4, **kw)
        self.dt = float(dt)
        self.params = tuple(float(p) for p in params)
        self._cparams = (ctypes.c_double * 7)(*self.params)

    @staticmethod
    def _rows(t: torch.Tensor, width: int):
        """(t, row stride): t itself where its (b, t) rows are evenly strided
        with unit column stride (column slices of a packed iterate, such as
        the ADMM state's z rows), else a contiguous copy."""
        if t.stride(-1) == 1 and t.stride(1) >= width and t.stride(0) == t.shape[1] * t.stride(1):
            return t, t.stride(1)
        return t.contiguous(), width

    def dynamics_blocks(self, states, controls):
        if not states.is_cuda:
            raise ValueError("QuadrotorOCP linearization runs on the GPU; pass device tensors")
        lib = _lib.load()
        B, N = self.B, self.horizon
        if tuple(states.shape) != (B, N + 1, 13) or tuple(controls.shape) != (B, N + 1, 4):
            raise ValueError(f"states {tuple(states.shape)} / controls {tuple(controls.shape)}: expected "
                             f"({B}, {N + 1}, 13) / ({B}, {N + 1}, 4)")
        # read in place where the rows are evenly strided (no copy of a packed iterate)
        states, ls = self._rows(states.to(self.dtype), 13)
        controls, lu = self._rows(controls.to(self.dtype), 4)
        Am = torch.empty((B, N, 13, 17), dtype=self.dtype, device=states.device)
        c = torch.empty((B, N, 13), dtype=self.dtype, device=states.device)
        sfx = _lib.suffix(self.dtype)
        st = getattr(lib, f"tmpc_quadrotor_linearize_strided_{sfx}")(
            _lib.stream_handle(states.device), B, N, states.data_ptr(), ls, controls.data_ptr(), lu, self.dt,
            self._cparams, _lib.ptr(Am), _lib.ptr(c),
        )
        _lib.check(f"tmpc_quadrotor_linearize_strided_{sfx}", st)
        return Am, c

    def step_linearization(self):
        """The keywords of an SQP step that builds this problem's dynamics
        rows itself (ADMMSolver.sqp_step(quadrotor=(dt, params))), or None
        with rescaling (the step writes the unscaled rows)."""
        return None if self.rescale_optimization_variables else {"quadrotor": (self.dt, self._cparams)}

    def qp_for_next_step(self, prev: Optional[QPData] = None) -> QPData:
        """The QP of the next SQP iteration with its dynamics rows left to the
        step that solves it: A_minus and c are empty buffers that
        tmpc_sqp_admm_step_quadrotor_* fills with the linearization at the
        step's input iterate, the ADMM state's x (the iterate build_qp would
        be given).  The other blocks are this problem's, as in build_qp
        (prev, the previous step's QP, is not needed)."""
        B, N = self.B, self.horizon
        Am = torch.empty((B, N, 13, 17), dtype=self.dtype, device=self.device)
        c = torch.empty((B, N, 13), dtype=self.dtype, device=self.device)
        return self._qp_with_dynamics(Am, c)

    def next_states(self, states, controls):
        """(B, N, 13): the RK4 step at every stage (tmpc_quadrotor_dynamics_*)."""
        if not states.is_cuda:
            raise ValueError("QuadrotorOCP dynamics run on the GPU; pass device tensors")
        lib = _lib.load()
        B, N = self.B, self.horizon
        states = states.to(self.dtype).contiguous()
        controls = controls.to(self.dtype).contiguous()
        nxt = torch.empty((B, N, 13), dtype=self.dtype, device=states.device)
        sfx = _lib.suffix(self.dtype)
        st = getattr(lib, f"tmpc_quadrotor_dynamics_{sfx}")(
            _lib.stream_handle(states.device), B, N, _lib.ptr(states), _lib.ptr(controls), self.dt,
            self._cparams, _lib.ptr(nxt))
        _lib.check(f"tmpc_quadrotor_dynamics_{sfx}", st)
        return nxt

    def dynamics_lagrangian_hessian(self, states, controls, lambdas):
        """(B, N+1, 17, 17): d^2/dz_t^2 [lambda_t . f(z_t)] for t < N, zero at N
        (tmpc_quadrotor_lagrangian_hessian_*, hyper-dual numbers on the device)."""
        if not states.is_cuda:
            raise ValueError("QuadrotorOCP Hessians run on the GPU; pass device tensors")
        lib = _lib.load()
        B, N = self.B, self.horizon
        states = states.to(self.dtype).contiguous()
        controls = controls.to(self.dtype).contiguous()
        lambdas = lambdas.to(self.dtype).contiguous()
        H = torch.empty((B, N + 1, 17, 17), dtype=self.dtype, device=states.device)
        sfx = _lib.suffix(self.dtype)
        st = getattr(lib, f"tmpc_quadrotor_lagrangian_hessian_{sfx}")(
            _lib.stream_handle(states.device), B, N, _lib.ptr(states), _lib.ptr(controls), self.dt,
            self._cparams, _lib.ptr(lambdas), _lib.ptr(H),
        )
        _lib.check(f"tmpc_quadrotor_lagrangian_hessian_{sfx}", st)
        return H


def quaternion_from_rotvec(r: torch.Tensor) -> torch.Tensor:
    """(..., 3) rotation vectors -> (..., 4) unit quaternions (w, x, y, z)."""
    ang = torch.linalg.norm(r, dim=-1, keepdim=True)
    half = 0.5 * ang
    s = torch.where(ang > 1e-12, torch.sin(half) / torch.clamp(ang, min=1e-300), 0.5 - ang * ang / 48.0)
    return torch.cat([torch.cos(half), s * r], dim=-1)


def make_quadrotor_config(B: int = 4096, seed: int = 0, *, N: int = 40, dt: float = 0.02,
                          dtype=torch.float32, device="cpu", **kw) -> QuadrotorOCP:
    """Config 3 of the benchmark: goal ~ U[-2,2]^3, x0 = hover + N(0, 0.3) on p and v
    plus a small random rotation; Q = diag(10 I3, I4, I3, 0.1 I3), R = 0.01 I4
    toward hover thrust, thrusts in [0, 2 hover].  Other keyword arguments go
    to the problem (for example constrain_initial_control, initial_control)."""
    g = torch.Generator().manual_seed(int(seed))
    hov = hover_thrust()
    goal = torch.rand((B, 3), generator=g, dtype=torch.float64) * 4.0 - 2.0
    p0 = torch.randn((B, 3), generator=g, dtype=torch.float64) * 0.3
    v0 = torch.randn((B, 3), generator=g, dtype=torch.float64) * 0.3
    rv = torch.randn((B, 3), generator=g, dtype=torch.float64) * 0.1
    q0 = quaternion_from_rotvec(rv)
    x0 = torch.cat([p0, q0, v0, torch.zeros((B, 3), dtype=torch.float64)], dim=-1)
    xg = torch.zeros((B, 13), dtype=torch.float64)
    xg[:, :3] = goal
    xg[:, 3] = 1.0
    T = N + 1
    wx = torch.tensor([10.0] * 3 + [1.0] * 4 + [1.0] * 3 + [0.1] * 3, dtype=torch.float64).expand(B, 13)
    wu = torch.full((B, 4), 0.01, dtype=torch.float64)
    return QuadrotorOCP(
        horizon=N,
        dt=dt,
        initial_state=x0,
        weights_state=wx,
        weights_control=wu,
        weights_final=torch.zeros((B, 13), dtype=torch.float64),
        reference_state=xg.unsqueeze(1).expand(B, T, 13),
        reference_control=torch.full((B, T, 4), hov, dtype=torch.float64),
        penalize_control_reference=True,
        control_bounds=(torch.zeros(4, dtype=torch.float64), torch.full((4,), 2.0 * hov, dtype=torch.float64)),
        initial_guess_final_state=xg,
        dtype=dtype,
        device=device,
        **kw,
    )


__all__ = ["QuadrotorOCP", "QUAD_PARAMS", "hover_thrust", "make_quadrotor_config", "quaternion_from_rotvec"]
_ = math
