"""Seeded synthetic workloads of the benchmark configurations (numpy RNG).

config1  2D point-mass double integrator, nx=4, nu=2, N=20, dt=0.1, |u|<=1
config2  random stable LTI, nx=12, nu=4, N=50, |x|<=5, |u|<=1
config3  quadrotor SQP (problems/quadrotor.py: make_quadrotor_config)
config4  3D double integrator among 8 spherical obstacles, nx=6, nu=3, N=60,
         dt=0.05, |u|<=3, obstacle rows linearized per SQP iteration
config5  Clohessy-Wiltshire rendezvous, nx=6, nu=3, N=100, dt=10 s (exact
         zero-order-hold discretization), |u|<=0.01
Each returns a LinearOCP with float64 tensors on the CPU; move it with .to().
Keyword arguments of config1/2/5 go to the problem (for example
constrain_initial_control=True, initial_control=u0).
"""
from __future__ import annotations

import numpy as np
import scipy.linalg
import torch

from .obstacle import ObstacleOCP
from .ocp import LinearOCP


def config1(B: int = 64, seed: int = 0, **kw) -> LinearOCP:
    rng = np.random.default_rng(seed)
    dt, N, nx, nu = 0.1, 20, 4, 2
    I2 = np.eye(2)
    A = np.block([[I2, dt * I2], [np.zeros((2, 2)), I2]])
    Bm = np.vstack([0.5 * dt * dt * I2, dt * I2])
    x0 = rng.uniform(-1.0, 1.0, size=(B, nx))
    return LinearOCP(
        A=torch.tensor(np.broadcast_to(A, (B, nx, nx)).copy()),
        Bm=torch.tensor(np.broadcast_to(Bm, (B, nx, nu)).copy()),
        horizon=N, num_states=nx, num_controls=nu,
        initial_state=torch.tensor(x0),
        weights_state=torch.ones((B, nx), dtype=torch.float64),
        weights_control=torch.full((B, nu), 0.1, dtype=torch.float64),
        weights_final=torch.full((B, nx), 9.0, dtype=torch.float64),  # Qf = 10 I = Q + 9 I
        control_bounds=(torch.full((nu,), -1.0, dtype=torch.float64), torch.full((nu,), 1.0, dtype=torch.float64)),
        **kw,
    )


def config2(B: int = 1024, seed: int = 0, **kw) -> LinearOCP:
    rng = np.random.default_rng(seed)
    N, nx, nu = 50, 12, 4
    A = np.empty((B, nx, nx))
    for b in range(B):
        G = rng.standard_normal((nx, nx))
        Ab = np.eye(nx) + 0.1 * G / np.sqrt(nx)
        rad = np.max(np.abs(np.linalg.eigvals(Ab)))
        if rad > 1.05:
            Ab *= 1.05 / rad
        A[b] = Ab
    Bm = rng.normal(0.0, 0.1, size=(B, nx, nu))
    wq = rng.uniform(0.1, 10.0, size=(B, nx))
    wr = rng.uniform(0.01, 1.0, size=(B, nu))
    x0 = rng.standard_normal((B, nx))
    return LinearOCP(
        A=torch.tensor(A), Bm=torch.tensor(Bm), horizon=N, num_states=nx, num_controls=nu,
        initial_state=torch.tensor(x0), weights_state=torch.tensor(wq), weights_control=torch.tensor(wr),
        weights_final=torch.zeros((B, nx), dtype=torch.float64),
        state_bounds=(torch.full((nx,), -5.0, dtype=torch.float64), torch.full((nx,), 5.0, dtype=torch.float64)),
        control_bounds=(torch.full((nu,), -1.0, dtype=torch.float64), torch.full((nu,), 1.0, dtype=torch.float64)),
        **kw,
    )


def config4(B: int = 16384, seed: int = 0, *, use_slack_variables: bool = False,
            slack_penalization_weight: float = 100.0, **kw) -> ObstacleOCP:
    """Start and goal on opposite faces of [-4, 4]^3 (random axis and side, the
    other coordinates uniform), at rest; 8 spheres per problem with centers
    U[-3, 3]^3 and radii U[0.3, 0.8], so the start and goal lie outside every
    sphere.  Tracking weights diag(1,1,1, .1,.1,.1) on the state, 0.01 on the
    controls, terminal weights diag(10,10,10, 1,1,1); the reference trajectory
    is the goal at rest, which is also the final state of the initial guess."""
    rng = np.random.default_rng(seed)
    dt, N, nx, nu, K = 0.05, 60, 6, 3, 8
    I3 = np.eye(3)
    A = np.block([[I3, dt * I3], [np.zeros((3, 3)), I3]])
    Bm = np.vstack([0.5 * dt * dt * I3, dt * I3])
    centers = rng.uniform(-3.0, 3.0, size=(B, K, 3))
    radii = rng.uniform(0.3, 0.8, size=(B, K))
    axis = rng.integers(0, 3, size=B)
    side = rng.choice([-1.0, 1.0], size=B)
    start = rng.uniform(-4.0, 4.0, size=(B, 3))
    goal = rng.uniform(-4.0, 4.0, size=(B, 3))
    start[np.arange(B), axis] = -4.0 * side
    goal[np.arange(B), axis] = 4.0 * side
    x0 = np.concatenate([start, np.zeros((B, 3))], axis=1)
    xg = np.concatenate([goal, np.zeros((B, 3))], axis=1)
    wx = np.array([1.0, 1.0, 1.0, 0.1, 0.1, 0.1])
    wf = np.array([10.0, 10.0, 10.0, 1.0, 1.0, 1.0])
    f64 = lambda a: torch.tensor(np.ascontiguousarray(a), dtype=torch.float64)  # noqa: E731
    return ObstacleOCP(
        A=f64(np.broadcast_to(A, (B, nx, nx))), Bm=f64(np.broadcast_to(Bm, (B, nx, nu))),
        horizon=N, num_states=nx, num_controls=nu,
        initial_state=f64(x0), weights_state=f64(np.broadcast_to(wx, (B, nx))),
        weights_control=torch.full((B, nu), 0.01, dtype=torch.float64),
        weights_final=f64(np.broadcast_to(wf, (B, nx))),
        reference_state=f64(np.broadcast_to(xg[:, None], (B, N + 1, nx))),
        control_bounds=(torch.full((nu,), -3.0, dtype=torch.float64), torch.full((nu,), 3.0, dtype=torch.float64)),
        initial_guess_final_state=f64(xg),
        obstacles_centers=f64(centers), obstacles_radii=f64(radii), obstacles_dimension=3,
        use_slack_variables=use_slack_variables, slack_penalization_weight=slack_penalization_weight, **kw,
    )


def cw_discrete(mean_motion: float = 0.0011, dt: float = 10.0):
    """Exact ZOH discretization of the Clohessy-Wiltshire equations
    (x radial, y along-track, z cross-track)."""
    n = mean_motion
    Ac = np.zeros((6, 6))
    Ac[0:3, 3:6] = np.eye(3)
    Ac[3, 0] = 3 * n * n
    Ac[3, 4] = 2 * n
    Ac[4, 3] = -2 * n
    Ac[5, 2] = -n * n
    Bc = np.zeros((6, 3))
    Bc[3:6, :] = np.eye(3)
    M = np.zeros((9, 9))
    M[:6, :6] = Ac
    M[:6, 6:] = Bc
    E = scipy.linalg.expm(M * dt)
    return E[:6, :6], E[:6, 6:]


def config5(B: int = 2048, seed: int = 0, **kw) -> LinearOCP:
    rng = np.random.default_rng(seed)
    N, nx, nu = 100, 6, 3
    Ad, Bd = cw_discrete()
    wq = rng.uniform(1.0, 10.0, size=(B, nx))
    wr = rng.uniform(0.1, 1.0, size=(B, nu))
    x0 = rng.standard_normal((B, nx)) * np.array([100.0] * 3 + [0.1] * 3)
    return LinearOCP(
        A=torch.tensor(np.broadcast_to(Ad, (B, nx, nx)).copy()),
        Bm=torch.tensor(np.broadcast_to(Bd, (B, nx, nu)).copy()),
        horizon=N, num_states=nx, num_controls=nu,
        initial_state=torch.tensor(x0), weights_state=torch.tensor(wq), weights_control=torch.tensor(wr),
        weights_final=torch.zeros((B, nx), dtype=torch.float64),
        control_bounds=(torch.full((nu,), -0.01, dtype=torch.float64), torch.full((nu,), 0.01, dtype=torch.float64)),
        **kw,
    )
