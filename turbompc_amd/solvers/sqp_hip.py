"""Device-side SQP helpers (tmpc_sqp_first_order_*).

first_order_check: _compute_first_order_convergence_error
(turbompc/solvers/turbompc_solver.py:1158-1225) for the whole batch in one
kernel launch over every (problem, stage) pair, returning
(conv, eq_err, ineq_err, g) with g = G x (+ slack).  std_dynamics=True asserts
A_plus_t = [-I 0] and E_t = 0 (explicit integrators), which the kernel then
does not read; None or False evaluates the general blocks.  diag_cost=True
asserts diagonal D_t (only the diagonal is read).
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from .. import _lib
from .admm.admm_hip_backend import qp_struct
from .qp_data import QPData


def first_order_check(qp: QPData, x: torch.Tensor, y_f0: torch.Tensor, y_f: torch.Tensor, y_g: torch.Tensor,
                      slack: Optional[torch.Tensor] = None, slack_weight: float = 0.0,
                      std_dynamics: Optional[bool] = None, diag_cost: bool = False):
    lib = _lib.load()
    B, T, n, nx, n0, m = qp.dims
    dt, dev = qp.dtype, qp.device
    dims = _lib.Dims(B, T, n, nx, n0, m)
    cq, keep = qp_struct(qp, None)
    x, y_f0, y_f, y_g = (t.to(dt).contiguous() for t in (x, y_f0, y_f, y_g))
    slack = slack.to(dt).contiguous() if slack is not None else None
    conv = torch.empty(B, dtype=dt, device=dev)
    eq = torch.empty(B, dtype=dt, device=dev)
    iq = torch.empty(B, dtype=dt, device=dev)
    g = torch.empty((B, T, m), dtype=dt, device=dev)
    sfx = _lib.suffix(dt)
    st = getattr(lib, f"tmpc_sqp_first_order_{sfx}")(
        _lib.stream_handle(dev), ctypes.byref(dims), ctypes.byref(cq), _lib.ptr(x), _lib.ptr(y_f0), _lib.ptr(y_f),
        _lib.ptr(y_g), _lib.ptr(slack), float(slack_weight),
        (_lib.FLAG_STD_DYNAMICS if std_dynamics else 0) | (_lib.FLAG_DIAG_COST if diag_cost else 0), _lib.ptr(conv), _lib.ptr(eq), _lib.ptr(iq), _lib.ptr(g),
    )
    _lib.check(f"tmpc_sqp_first_order_{sfx}", st)
    del keep
    return conv, eq, iq, g


def kkt_active_sets(g: torch.Tensor, l: torch.Tensor, u: torch.Tensor, y: Optional[torch.Tensor], eps_abs: float,
                    eps_rel: float, dual_tol: float):
    """(lower, upper) bool tensors of g's shape: the active sets of the KKT
    state (tmpc_kkt_active_sets_*; identify_active_inequalities and the dual
    sign test of _build_kkt_state, turbompc_solver.py:269-292, :1387-1439),
    one kernel instead of the elementwise chain; y None: proximity only."""
    if not g.is_cuda:
        raise ValueError("kkt_active_sets runs on the GPU; pass device tensors")
    lib = _lib.load()
    dt, dev = g.dtype, g.device
    g, l, u = (t.to(device=dev, dtype=dt).expand(g.shape).contiguous() for t in (g, l, u))
    y = y.to(device=dev, dtype=dt).expand(g.shape).contiguous() if y is not None else None
    lower = torch.empty(g.shape, dtype=torch.uint8, device=dev)
    upper = torch.empty(g.shape, dtype=torch.uint8, device=dev)
    sfx = _lib.suffix(dt)
    st = getattr(lib, f"tmpc_kkt_active_sets_{sfx}")(
        _lib.stream_handle(dev), g.numel(), _lib.ptr(g), _lib.ptr(l), _lib.ptr(u), _lib.ptr(y), float(eps_abs),
        float(eps_rel), float(dual_tol), _lib.ptr(lower), _lib.ptr(upper))
    _lib.check(f"tmpc_kkt_active_sets_{sfx}", st)
    return lower.view(torch.bool), upper.view(torch.bool)  # the kernel writes 0 / 1
