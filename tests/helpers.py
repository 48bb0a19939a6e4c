"""Shared test helpers: tolerances, relative errors, dense reference assembly."""
from __future__ import annotations

import numpy as np
import torch

# Parity bars at fixed iteration counts (normwise relative error).
TOL = {torch.float64: 1e-9, torch.float32: 1e-4, np.float64: 1e-9, np.float32: 1e-4}


def rel_err(a, b) -> float:
    a = np.asarray(a.detach().cpu() if torch.is_tensor(a) else a, dtype=np.float64)
    b = np.asarray(b.detach().cpu() if torch.is_tensor(b) else b, dtype=np.float64)
    scale = max(float(np.max(np.abs(b))) if b.size else 0.0, 1e-12)
    return float(np.max(np.abs(a - b))) / scale if a.size else 0.0


def np_qp(qp):
    """Dict of float64 numpy arrays of a QPData (torch tensors)."""
    f = lambda t: np.asarray(t.detach().cpu(), dtype=np.float64)  # noqa: E731
    return dict(
        D=f(qp.cost.D), E=f(qp.cost.E), q=f(qp.cost.q), A0=f(qp.eq.A0), Am=f(qp.eq.A_minus), Ap=f(qp.eq.A_plus),
        c0=f(qp.eq.c0), c=f(qp.eq.c), G=f(qp.ineq.G), l=f(qp.ineq.l), u=f(qp.ineq.u),
    )


def dense_P(D, E):
    """Dense P of one problem: P[t,t]=D_t, P[t+1,t]=E_t, P[t,t+1]=E_t^T
    (backward_kkt_jax.py:109-138)."""
    T, n, _ = D.shape
    P = np.zeros((T * n, T * n))
    for t in range(T):
        P[t * n:(t + 1) * n, t * n:(t + 1) * n] = D[t]
        if t < T - 1:
            P[(t + 1) * n:(t + 2) * n, t * n:(t + 1) * n] = E[t]
            P[t * n:(t + 1) * n, (t + 1) * n:(t + 2) * n] = E[t].T
    return P


def dense_C(A0, Am, Ap):
    n0, n = A0.shape
    N, nx, _ = Am.shape
    T = N + 1
    C = np.zeros((n0 + N * nx, T * n))
    C[:n0, :n] = A0
    for t in range(N):
        C[n0 + t * nx:n0 + (t + 1) * nx, t * n:(t + 1) * n] = Am[t]
        C[n0 + t * nx:n0 + (t + 1) * nx, (t + 1) * n:(t + 2) * n] = Ap[t]
    return C


def dense_G(G):
    T, m, n = G.shape
    out = np.zeros((T * m, T * n))
    for t in range(T):
        out[t * m:(t + 1) * m, t * n:(t + 1) * n] = G[t]
    return out


def blocks_to_dense(S):
    """(T, n, 3n) block rows [prev | diag | next] -> dense (T n, T n)."""
    T, n, _ = S.shape
    A = np.zeros((T * n, T * n))
    for t in range(T):
        A[t * n:(t + 1) * n, t * n:(t + 1) * n] = S[t, :, n:2 * n]
        if t > 0:
            A[t * n:(t + 1) * n, (t - 1) * n:t * n] = S[t, :, :n]
        if t < T - 1:
            A[t * n:(t + 1) * n, (t + 1) * n:(t + 2) * n] = S[t, :, 2 * n:]
    return A


def random_qp(B, T, n, nx, m, *, seed=0, std=False, dtype=torch.float64, n0=None, diag=False):
    """Random well-posed QP batch: SPD-ish D (diagonal with diag=True), small
    E, random dynamics rows, random G, boxes around zero."""
    from turbompc_amd.solvers.qp_data import QPCostBlocks, QPData, QPEqualityBlocks, QPInequalityBlocks

    rng = np.random.default_rng(seed)
    N = T - 1
    n0 = nx if n0 is None else n0
    L = rng.standard_normal((B, T, n, n)) * 0.3
    D = np.einsum("btij,btkj->btik", L, L) + np.eye(n) * rng.uniform(0.5, 2.0, size=(B, T, 1, 1))
    E = np.zeros((B, N, n, n)) if std else rng.standard_normal((B, N, n, n)) * 0.05
    q = rng.standard_normal((B, T, n))
    A0 = np.zeros((B, n0, n))
    A0[:, :, :n0] = np.eye(n0)
    Am = np.concatenate([np.eye(nx) + 0.1 * rng.standard_normal((B, N, nx, nx)),
                         0.3 * rng.standard_normal((B, N, nx, n - nx))], axis=-1)
    Ap = np.zeros((B, N, nx, n))
    Ap[..., :nx] = -np.eye(nx)
    if not std:
        Ap += 0.05 * rng.standard_normal((B, N, nx, n))
    # constraints built around a random trajectory zf so the QP is feasible
    zf = rng.standard_normal((B, T, n))
    c0 = np.einsum("bij,bj->bi", A0, zf[:, 0])
    c = np.einsum("btij,btj->bti", Am, zf[:, :-1]) + np.einsum("btij,btj->bti", Ap, zf[:, 1:])
    if diag:
        D = np.einsum("btij,ij->btij", D, np.eye(n))
    G = rng.standard_normal((B, T, m, n))
    gz = np.einsum("btij,btj->bti", G, zf)
    l = gz - rng.uniform(0.2, 1.0, size=(B, T, m))
    u = gz + rng.uniform(0.2, 1.0, size=(B, T, m))
    t = lambda a: torch.tensor(a, dtype=dtype)  # noqa: E731
    return QPData(
        cost=QPCostBlocks(t(D), t(E), t(q)),
        eq=QPEqualityBlocks(t(A0), t(Am), t(Ap), t(c0), t(c)),
        ineq=QPInequalityBlocks(t(G), t(l), t(u), torch.tensor(0.0, dtype=dtype), False),
    )


def zero_state(qp, rho):
    """ADMMState-like namespace of the reference initial state (x = 0)."""
    from collections import namedtuple

    B, T, n, nx, n0, m = qp.dims
    St = namedtuple("St", ["x_blocks", "y_g", "y_f_0", "y_f_dyn", "z_g", "xi_g", "rho_bar"])
    z0 = np.clip(np.zeros((B, T, m)), np.asarray(qp.ineq.l, dtype=np.float64), np.asarray(qp.ineq.u, dtype=np.float64))
    return St(np.zeros((B, T, n)), np.zeros((B, T, m)), np.zeros((B, n0)), np.zeros((B, T - 1, nx)), z0,
              np.zeros((B, T, m)), np.full((B,), float(rho)))


def soften(qp, gamma, shrink=1.0):
    """The QP with soft inequality rows (slack weight gamma), each box shrunk
    about its midpoint by `shrink` so that some rows end up violated."""
    from turbompc_amd.solvers.qp_data import QPData, QPInequalityBlocks

    l, u = qp.ineq.l, qp.ineq.u
    mid, half = 0.5 * (l + u), 0.5 * shrink * (u - l)
    return QPData(cost=qp.cost, eq=qp.eq,
                  ineq=QPInequalityBlocks(qp.ineq.G, mid - half, mid + half,
                                          torch.tensor(float(gamma), dtype=l.dtype), True))


def polish(a, b, lower, upper):
    """Exact solution of QP problem b (dict of np_qp arrays) on a fixed active
    set: the equality-constrained KKT [[P, C^T, Ga^T], [C, 0, 0], [Ga, 0, 0]]
    with the active rows of G held at their bounds, solved densely.  lower /
    upper (T*m,) mark the rows held at l / u.  Returns (x (T,n), y_f0, y_f
    (N,nx), y_g (T,m), bound violation of the other rows, sign margin): the
    active set is the QP's own when the violation is ~0 and the margin
    positive (y_g >= 0 at upper rows, <= 0 at lower rows, the sign convention
    P x + q + C^T y_f + G^T y_g = 0)."""
    T, n, _ = a["D"][b].shape
    N, nx, _ = a["Am"][b].shape
    m = a["G"][b].shape[1]
    n0 = a["A0"][b].shape[0]
    P = dense_P(a["D"][b], a["E"][b])
    C = dense_C(a["A0"][b], a["Am"][b], a["Ap"][b])
    G = dense_G(a["G"][b])
    l, u = a["l"][b].reshape(-1), a["u"][b].reshape(-1)
    act = lower | upper
    Ga, ba = G[act], np.where(lower, l, u)[act]
    c = np.concatenate([a["c0"][b], a["c"][b].reshape(-1)])
    nz, ne, na = P.shape[0], C.shape[0], Ga.shape[0]
    K = np.zeros((nz + ne + na, nz + ne + na))
    K[:nz, :nz] = P
    K[:nz, nz:nz + ne] = C.T
    K[nz:nz + ne, :nz] = C
    K[:nz, nz + ne:] = Ga.T
    K[nz + ne:, :nz] = Ga
    sol = np.linalg.solve(K, np.concatenate([-a["q"][b].reshape(-1), c, ba]))
    x, y = sol[:nz], sol[nz:nz + ne]
    yg = np.zeros(T * m)
    yg[act] = sol[nz + ne:]
    gx = G @ x
    viol = float(np.max(np.maximum(l - gx, 0) + np.maximum(gx - u, 0))) if T * m else 0.0
    margin = min(np.min(yg[upper], initial=np.inf), -np.max(yg[lower], initial=-np.inf))
    return x.reshape(T, n), y[:n0], y[n0:].reshape(N, nx), yg.reshape(T, m), viol, margin
