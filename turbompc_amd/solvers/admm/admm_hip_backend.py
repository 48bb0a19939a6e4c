"""ctypes marshalling of the fused ADMM entry points (tmpc_admm_direct_*, tmpc_admm_pcg_*).

Counterparts of the reference's FFI wrappers
  admm_cudss_ffi_solve  (turbompc/solvers/admm/admm_cudss_ffi_backend.py:62-258)
  admm_ffi_solve        (turbompc/solvers/admm/admm_ffi_backend.py:55-268)
with the same inputs (QP blocks, warm-start state, solver attributes) and
outputs (final state, iteration counts).  The Schur matrix is factorized (or S
and Phiinv are built) on the device, so no precomputed `schur` argument is
needed.
"""
from __future__ import annotations

import ctypes
from typing import NamedTuple, Optional, Tuple

import torch

from ... import _lib
from ..qp_data import QPData

# Workspaces of the calls that do not bring their own, one per (kind, device,
# stream): calls issued on different streams never share one, and the calls of
# one stream run in order.  A grown workspace replaces the old one only after
# the stream has finished with it (the caching allocator's stream semantics).
_WS_CACHE = {}


def _ws(kind: str, nbytes: int, device: torch.device) -> torch.Tensor:
    stream = torch.cuda.current_stream(device)
    key = (kind, device, stream.cuda_stream)
    t = _WS_CACHE.get(key)
    if t is None or t.numel() < nbytes:
        with torch.cuda.stream(stream):
            t = _lib.workspace(nbytes, device)
        _WS_CACHE[key] = t
    return t


def qp_struct(qp: QPData, slack_weight: Optional[torch.Tensor]):
    """Pointers of the QP blocks for the C ABI.  Every block must carry the
    solve's dtype: the library reads the buffers as that type."""
    B, T, n, nx, n0, m = qp.dims
    keep = []
    dt = qp.dtype

    def p(t):
        if t is None:
            return None
        if t.dtype != dt:
            raise TypeError(f"QP block of dtype {t.dtype} in a {dt} solve; convert the QP with QPData.to()")
        t = t.contiguous()
        keep.append(t)
        return _lib.ptr(t)

    s = _lib.QP(
        p(qp.cost.D), p(qp.cost.E), p(qp.cost.q), p(qp.eq.A0), p(qp.eq.A_minus), p(qp.eq.A_plus),
        p(qp.ineq.G) if m else None, p(qp.ineq.l) if m else None, p(qp.ineq.u) if m else None,
        p(qp.eq.c0), p(qp.eq.c), p(slack_weight),
    )
    return s, keep


def state_struct(x, z_g, y_g, y_f0, y_f, xi_g, rho):
    return _lib.State(*[_lib.ptr(t) for t in (x, z_g, y_g, y_f0, y_f, xi_g, rho)])


def cfg_struct(*, max_iter, check_every, adapt_rho_every, pcg_max_iter, use_slack, flags, sigma, eps_abs, eps_rel,
               rho_min, rho_max, adaptive_rho_tolerance, rho_f_factor, alpha, pcg_eps) -> _lib.AdmmCfg:
    return _lib.AdmmCfg(
        int(max_iter), int(check_every), int(adapt_rho_every), int(pcg_max_iter), int(bool(use_slack)), int(flags),
        float(sigma), float(eps_abs), float(eps_rel), float(rho_min), float(rho_max),
        float(adaptive_rho_tolerance), float(rho_f_factor), float(alpha), float(pcg_eps),
    )


def direct_workspace(qp: QPData) -> torch.Tensor:
    """A workspace of its own for tmpc_admm_direct_* / tmpc_sqp_admm_step_* (an
    SQP loop keeps one per solve so that its stage records stay valid between
    steps, see FLAG_WARM_RECORDS)."""
    lib = _lib.load()
    B, T, n, nx, n0, m = qp.dims
    nbytes = lib.tmpc_admm_direct_workspace_bytes(8 if qp.dtype == torch.float64 else 4,
                                                  ctypes.byref(_lib.Dims(B, T, n, nx, n0, m)))
    return _lib.workspace(nbytes, qp.device)


class ObstacleRows(NamedTuple):
    """Obstacle rows that an SQP step linearizes itself
    (tmpc_sqp_admm_step_obstacle_*): K spheres (centers (B, K, dim), radii
    (B, K)) in the first dim state coordinates, rows row0 .. row0 + K - 1 of
    every stage."""
    dim: int
    K: int
    centers: torch.Tensor
    radii: torch.Tensor
    row0: int


def admm_hip_solve(qp: QPData, state0, *, schur: str, cfg: _lib.AdmmCfg,
                   slack_weight: Optional[torch.Tensor] = None, want_pcg_iters: bool = False, sqp=None,
                   workspace: Optional[torch.Tensor] = None, donate: bool = False,
                   iters_out: Optional[torch.Tensor] = None, quadrotor=None,
                   obstacles: Optional["ObstacleRows"] = None):
    """Run the fused ADMM on the device.  `state0` is an ADMMState of batched
    tensors; returns (state fields tuple, iters (B,), pcg_iters or None).

    sqp = (active (B,) bool, tol) makes the call one SQP step
    (tmpc_sqp_admm_step_*, direct Schur solve only): the first-order check of
    state0 against qp, the activity test active & (conv > tol), and the solve of
    the problems that pass it; the call then also returns (conv, eq_err,
    ineq_err, g, active_out).  With tol None the activity is given: no check
    runs, the problems where `active` is False keep their state, and conv,
    eq_err, ineq_err and g are None.

    donate: the caller gives up state0: fields that already have the output's
    shape, dtype and layout are updated in place instead of copied (the
    library reads and writes the same buffers).

    iters_out: a zero-filled contiguous (B,) int32 device buffer that receives
    the iteration words (returned as `iters`) instead of a new one, e.g. a
    row of an SQP loop's per-iteration record.

    quadrotor = (dt, params as a ctypes double[7]) with sqp: the step builds
    the QP's dynamics rows itself (tmpc_sqp_admm_step_quadrotor_*):
    qp.eq.A_minus and qp.eq.c are outputs, the linearization at state0's x.
    obstacles (ObstacleRows) with sqp: the same for the obstacle rows of
    qp.ineq.G, l and u (tmpc_sqp_admm_step_obstacle_*; their other rows are
    inputs)."""
    if quadrotor is not None and obstacles is not None:
        raise ValueError("a step builds either the quadrotor's or the obstacle rows")
    if sqp is not None and schur != "direct":
        raise ValueError("an SQP step (sqp=...) needs the direct Schur solve")
    lib = _lib.load()
    B, T, n, nx, n0, m = qp.dims
    dev, dt = qp.device, qp.dtype
    sfx = _lib.suffix(dt)
    dims = _lib.Dims(B, T, n, nx, n0, m)
    if slack_weight is not None:
        slack_weight = torch.as_tensor(slack_weight, dtype=dt, device=dev).expand(B).contiguous()
    cq, keep = qp_struct(qp, slack_weight)

    def prep(t, shape):
        if donate and torch.is_tensor(t) and t.dtype == dt and t.device == dev and t.shape == shape \
                and t.is_contiguous():
            return t
        t = torch.as_tensor(t, dtype=dt, device=dev)
        return t.expand(shape).contiguous().clone() if t.shape != shape else t.contiguous().clone()

    outs = [
        prep(state0.x_blocks, (B, T, n)),
        prep(state0.z_g, (B, T, m)),
        prep(state0.y_g, (B, T, m)),
        prep(state0.y_f_0, (B, n0)),
        prep(state0.y_f_dyn, (B, T - 1, nx)),
        prep(state0.xi_g, (B, T, m)),
        prep(state0.rho_bar, (B,)),
    ]
    sv = state_struct(*outs)
    if iters_out is None:
        iters = torch.zeros(B, dtype=torch.int32, device=dev)
    elif (iters_out.dtype == torch.int32 and iters_out.shape == (B,) and iters_out.device == dev
          and iters_out.is_contiguous()):
        iters = iters_out
    else:
        raise ValueError("iters_out must be a contiguous (B,) int32 tensor on the QP's device")
    stream = _lib.stream_handle(dev)
    if schur == "direct":
        nbytes = lib.tmpc_admm_direct_workspace_bytes(ctypes.sizeof(ctypes.c_double) if dt == torch.float64 else 4,
                                                      ctypes.byref(dims))
        ws = _ws("admm_direct", nbytes, dev) if workspace is None else workspace
        if ws.numel() < nbytes:
            raise ValueError(f"workspace of {ws.numel()} bytes, {nbytes} needed")
        if sqp is not None:
            active, tol = sqp
            if active.dtype == torch.bool and active.device == dev and active.shape == (B,) \
                    and active.is_contiguous():
                act_in = active.view(torch.uint8)  # the same bytes (0 / 1), no copy
            else:
                act_in = active.to(device=dev, dtype=torch.uint8).contiguous()
            act_out = torch.empty(B, dtype=torch.uint8, device=dev)
            if tol is None:  # activity given: no check
                conv = eq = iq = g = None
                sq = _lib.SqpStep(_lib.ptr(act_in), _lib.ptr(act_out), 0.0, None, None, None, None)
            else:
                conv = torch.empty(B, dtype=dt, device=dev)
                eq = torch.empty(B, dtype=dt, device=dev)
                iq = torch.empty(B, dtype=dt, device=dev)
                g = torch.empty((B, T, m), dtype=dt, device=dev)
                sq = _lib.SqpStep(_lib.ptr(act_in), _lib.ptr(act_out), float(tol), _lib.ptr(conv), _lib.ptr(eq),
                                  _lib.ptr(iq), _lib.ptr(g))
            if obstacles is not None:
                if not all(t.is_contiguous() for t in (qp.ineq.G, qp.ineq.l, qp.ineq.u)):
                    raise ValueError("the obstacle step writes G, l and u in place: they must be contiguous")
                centers = obstacles.centers.to(device=dev, dtype=dt).contiguous()
                radii = obstacles.radii.to(device=dev, dtype=dt).contiguous()
                fn = f"tmpc_sqp_admm_step_obstacle_{sfx}"
                st = getattr(lib, fn)(
                    stream, ctypes.byref(dims), ctypes.byref(cq), ctypes.byref(sv), ctypes.byref(sv),
                    _lib.ptr(iters), ctypes.byref(cfg), ctypes.byref(sq), int(obstacles.dim), int(obstacles.K),
                    _lib.ptr(centers), _lib.ptr(radii), int(obstacles.row0), _lib.ptr(ws), nbytes,
                )
            elif quadrotor is None:
                fn = f"tmpc_sqp_admm_step_{sfx}"
                st = getattr(lib, fn)(
                    stream, ctypes.byref(dims), ctypes.byref(cq), ctypes.byref(sv), ctypes.byref(sv),
                    _lib.ptr(iters), ctypes.byref(cfg), ctypes.byref(sq), _lib.ptr(ws), nbytes,
                )
            else:
                if not (qp.eq.A_minus.is_contiguous() and qp.eq.c.is_contiguous()):
                    raise ValueError("the quadrotor step writes A_minus and c in place: they must be contiguous")
                dt_q, params_q = quadrotor
                fn = f"tmpc_sqp_admm_step_quadrotor_{sfx}"
                st = getattr(lib, fn)(
                    stream, ctypes.byref(dims), ctypes.byref(cq), ctypes.byref(sv), ctypes.byref(sv),
                    _lib.ptr(iters), ctypes.byref(cfg), ctypes.byref(sq), float(dt_q), params_q, _lib.ptr(ws), nbytes,
                )
            _lib.check(fn, st)
            del keep
            return outs, iters, None, (conv, eq, iq, g, act_out.view(torch.bool))  # the library writes 0 / 1
        st = getattr(lib, f"tmpc_admm_direct_{sfx}")(
            stream, ctypes.byref(dims), ctypes.byref(cq), ctypes.byref(sv), ctypes.byref(sv),
            _lib.ptr(iters), ctypes.byref(cfg), _lib.ptr(ws), nbytes,
        )
        _lib.check(f"tmpc_admm_direct_{sfx}", st)
        pcg_iters = None
    elif schur == "pcg":
        nbytes = lib.tmpc_admm_pcg_workspace_bytes(8 if dt == torch.float64 else 4, ctypes.byref(dims))
        ws = _ws("admm_pcg", nbytes, dev)
        pcg_iters = (torch.zeros((B, max(cfg.max_iter, 1)), dtype=torch.int32, device=dev)
                     if want_pcg_iters and cfg.max_iter > 0 else None)
        st = getattr(lib, f"tmpc_admm_pcg_{sfx}")(
            stream, ctypes.byref(dims), ctypes.byref(cq), ctypes.byref(sv), ctypes.byref(sv),
            _lib.ptr(iters), _lib.ptr(pcg_iters), ctypes.byref(cfg), _lib.ptr(ws), nbytes,
        )
        _lib.check(f"tmpc_admm_pcg_{sfx}", st)
    else:
        raise ValueError(f"unknown schur mode {schur!r}")
    del keep
    return outs, iters, pcg_iters


def schur_build(qp: QPData, rho: torch.Tensor, sigma: float, rho_f_factor: float) -> Tuple[torch.Tensor, torch.Tensor]:
    """compute_S_Phiinv on the device for every problem (rho (B,))."""
    lib = _lib.load()
    B, T, n, nx, n0, m = qp.dims
    dims = _lib.Dims(B, T, n, nx, n0, m)
    cq, keep = qp_struct(qp, None)
    rho = torch.as_tensor(rho, dtype=qp.dtype, device=qp.device).expand(B).contiguous()
    S = torch.empty((B, T, n, 3 * n), dtype=qp.dtype, device=qp.device)
    P = torch.empty_like(S)
    sfx = _lib.suffix(qp.dtype)
    st = getattr(lib, f"tmpc_schur_build_{sfx}")(
        _lib.stream_handle(qp.device), ctypes.byref(dims), ctypes.byref(cq), _lib.ptr(rho), float(sigma),
        float(rho_f_factor), _lib.ptr(S), _lib.ptr(P),
    )
    _lib.check(f"tmpc_schur_build_{sfx}", st)
    del keep
    return S, P
