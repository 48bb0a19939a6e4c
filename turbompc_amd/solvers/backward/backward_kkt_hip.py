"""Batched adjoint KKT solve on the GPU (tmpc_adjoint_kkt_*).

Drop-in for solve_backward_kkt / solve_backward_kkt_cudss_ffi
(turbompc/solvers/backward/backward_kkt_jax.py:177-211,
turbompc/solvers/backward/backward_kkt_cudss_ffi.py:232-277): the backward QP
(`_build_backward_qp`, turbompc/solvers/turbompc_solver.py:544-618) carries the
signed active rows G_act in ineq.G and -dL/dz in cost.q; the result is
dz = (dx_states, dx_controls) and the multipliers [y_f0 | y_f_dyn | y_ineq]
(turbompc_solver.py:727-763), one row per problem.  The batch is native: no
block-diagonal merge and no chunking by memory probe are needed.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from ... import _lib
from ..admm.admm_hip_backend import qp_struct
from ..qp_data import QPData, is_std_dynamics
from ..qp_utils import ZShape, unpack_x


def solve_backward_kkt_hip(qp_data: QPData, zshape: Optional[ZShape] = None, *, reg: float = 0.0,
                           refine_steps: int = -1, std_dynamics: Optional[bool] = None, kernel_flags: int = 0):
    """Returns (dz, mult); with a ZShape, ((dx_states, dx_controls), mult) as the reference.

    reg: relative quasi-definite shift (<= 0: library default 1e-12);
    refine_steps: iterative-refinement rounds (< 0: library default);
    kernel_flags: _lib.FLAG_GENERIC_KERNEL runs the generic factorization and
    solve instead of the rows-in-lanes kernels (cross-checks)."""
    lib = _lib.load()
    if not qp_data.cost.D.is_cuda:
        raise ValueError("solve_backward_kkt_hip needs device tensors")
    B, T, n, nx, n0, m = qp_data.dims
    dims = _lib.Dims(B, T, n, nx, n0, m)
    if m == 0:
        # the backward QP keeps the inequality arrays even when empty
        qp_data = qp_data.replace_ineq(l=qp_data.ineq.l, u=qp_data.ineq.u)
    cq, keep = qp_struct(qp_data, None)
    dz = torch.empty((B, T, n), dtype=qp_data.dtype, device=qp_data.device)
    mult = torch.empty((B, n0 + (T - 1) * nx + T * m), dtype=qp_data.dtype, device=qp_data.device)
    es = 8 if qp_data.dtype == torch.float64 else 4
    nbytes = lib.tmpc_adjoint_kkt_workspace_bytes(es, ctypes.byref(dims))
    ws = _lib.workspace(nbytes, qp_data.device)
    std = is_std_dynamics(qp_data) if std_dynamics is None else bool(std_dynamics)
    sfx = _lib.suffix(qp_data.dtype)
    st = getattr(lib, f"tmpc_adjoint_kkt_{sfx}")(
        _lib.stream_handle(qp_data.device), ctypes.byref(dims), ctypes.byref(cq), _lib.ptr(dz), _lib.ptr(mult),
        float(reg), int(refine_steps), (_lib.FLAG_STD_DYNAMICS if std else 0) | int(kernel_flags), _lib.ptr(ws),
        nbytes,
    )
    _lib.check(f"tmpc_adjoint_kkt_{sfx}", st)
    del keep
    if zshape is not None:
        return unpack_x(dz, zshape), mult
    return dz, mult
