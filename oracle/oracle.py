"""TEST INFRASTRUCTURE ONLY — ctypes front end of liboracle.so (numpy arrays).

QP and state objects are duck-typed: a QP exposes `.cost.{D,E,q}`,
`.eq.{A0,A_minus,A_plus,c0,c}`, `.ineq.{G,l,u,slack_penalization_weight,
use_slack_variables}` and a state exposes the ADMMState fields
(`x_blocks, y_g, y_f_0, y_f_dyn, z_g, xi_g, rho_bar`), every array carrying a
leading batch axis (turbompc/solvers/qp_data.py:11-100, admm/admm.py:27-34).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from collections import namedtuple
from dataclasses import dataclass
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB = None

OracleState = namedtuple(
    "OracleState", ["x_blocks", "y_g", "y_f_0", "y_f_dyn", "z_g", "xi_g", "rho_bar"]
)


class _Dims(ctypes.Structure):
    _fields_ = [(k, ctypes.c_int32) for k in ("B", "T", "n", "nx", "n0", "m")]


class _QP(ctypes.Structure):
    _fields_ = [
        (k, ctypes.c_void_p)
        for k in ("D", "E", "q", "A0", "A_minus", "A_plus", "G", "l", "u", "c0", "c")
    ] + [("slack_weight", ctypes.c_double), ("use_slack", ctypes.c_int32)]


class _State(ctypes.Structure):
    _fields_ = [(k, ctypes.c_void_p) for k in ("x", "z_g", "y_g", "y_f0", "y_f", "xi_g", "rho")]


class _Cfg(ctypes.Structure):
    _fields_ = [
        ("max_iter", ctypes.c_int32),
        ("check_every", ctypes.c_int32),
        ("adapt_rho_every", ctypes.c_int32),
        ("pcg_max_iter", ctypes.c_int32),
    ] + [
        (k, ctypes.c_double)
        for k in (
            "sigma",
            "eps_abs",
            "eps_rel",
            "rho_min",
            "rho_max",
            "adaptive_rho_tolerance",
            "rho_f_factor",
            "alpha",
            "pcg_eps",
        )
    ]


@dataclass
class OracleCfg:
    """ADMMSolver parameters (turbompc/solvers/admm/admm.py:13-24, :587-622)."""

    max_iter: int = 50
    check_every: int = 1
    adapt_rho_every: int = 5
    pcg_max_iter: int = 200
    sigma: float = 1.0e-6
    eps_abs: float = 1.0e-5
    eps_rel: float = 1.0e-4
    rho_min: float = 1.0e-6
    rho_max: float = 1.0e6
    adaptive_rho_tolerance: float = 5.0
    rho_f_factor: float = 1000.0
    alpha: float = 1.0
    pcg_eps: float = 1.0e-8

    def _c(self) -> _Cfg:
        return _Cfg(
            self.max_iter,
            self.check_every,
            self.adapt_rho_every,
            self.pcg_max_iter,
            self.sigma,
            self.eps_abs,
            self.eps_rel,
            self.rho_min,
            self.rho_max,
            self.adaptive_rho_tolerance,
            self.rho_f_factor,
            self.alpha,
            self.pcg_eps,
        )


def load(so=None):
    """Load liboracle.so (or the library at `so`), building the default one
    with make when it is missing."""
    global _LIB
    if _LIB is not None and so is None:
        return _LIB
    if so is None:
        so = _HERE / "liboracle.so"
        if not so.exists():
            subprocess.run(["make", "-C", str(_HERE)], check=True, capture_output=True)
    lib = ctypes.CDLL(str(so))
    for name in (
        "ora_admm_solve",
        "ora_schur_build",
        "ora_pcg",
        "ora_blktri_solve",
        "ora_adjoint_kkt",
        "ora_quadrotor_rk4_jac",
    ):
        getattr(lib, name).restype = ctypes.c_int
    _LIB = lib
    return lib


def use_native_build(build_dir):
    """Build the oracle with -march=native into `build_dir` (make native) and
    make it the library every oracle call uses from now on.  For the CPU
    baseline, on the host that times it.  Returns the library path."""
    subprocess.run(["make", "-C", str(_HERE), "native", f"NATIVE_DIR={build_dir}"], check=True,
                   capture_output=True)
    so = Path(build_dir) / "liboracle.so"
    load(so)
    return so


def _threads(nthreads):
    return int(nthreads) if nthreads else max(1, len(os.sched_getaffinity(0)))


def _arr(a, dtype):
    return np.ascontiguousarray(np.asarray(a, dtype=dtype))


def _ptr(a):
    return ctypes.c_void_p(a.ctypes.data) if a is not None and a.size else ctypes.c_void_p(0)


def _dims(qp):
    B, T, n, _ = np.shape(qp.cost.D)
    nx = np.shape(qp.eq.A_minus)[-2]
    n0 = np.shape(qp.eq.A0)[-2]
    m = np.shape(qp.ineq.G)[-2]
    return _Dims(B, T, n, nx, n0, m)


def _qp_arrays(qp, dtype):
    arrs = [
        _arr(v, dtype)
        for v in (
            qp.cost.D,
            qp.cost.E,
            qp.cost.q,
            qp.eq.A0,
            qp.eq.A_minus,
            qp.eq.A_plus,
            qp.ineq.G,
            qp.ineq.l,
            qp.ineq.u,
            qp.eq.c0,
            qp.eq.c,
        )
    ]
    cq = _QP(
        *[_ptr(a) for a in arrs],
        float(np.asarray(qp.ineq.slack_penalization_weight)),
        int(bool(qp.ineq.use_slack_variables)),
    )
    return cq, arrs


def admm_solve(qp, state, cfg: OracleCfg, *, schur="direct", dtype=np.float64, nthreads=None):
    """Run the restated ADMM JAX loop; returns (OracleState, iters, pcg_iters)."""
    lib = load()
    dt = np.dtype(dtype)
    d = _dims(qp)
    cq, keep = _qp_arrays(qp, dt)
    ins = [_arr(getattr(state, k), dt) for k in OracleState._fields]
    ins[-1] = _arr(np.broadcast_to(ins[-1], (d.B,)), dt)
    outs = [a.copy() for a in ins]
    sin = _State(*[_ptr(a) for a in (ins[0], ins[4], ins[1], ins[2], ins[3], ins[5], ins[6])])
    sout = _State(*[_ptr(a) for a in (outs[0], outs[4], outs[1], outs[2], outs[3], outs[5], outs[6])])
    iters = np.zeros(d.B, np.int32)
    pcg_iters = np.zeros(d.B, np.int32)
    c = cfg._c()
    rc = lib.ora_admm_solve(
        dt.itemsize,
        {"direct": 0, "pcg": 1}[schur],
        ctypes.byref(d),
        ctypes.byref(cq),
        ctypes.byref(sin),
        ctypes.byref(sout),
        _ptr(iters),
        _ptr(pcg_iters),
        ctypes.byref(c),
        _threads(nthreads),
    )
    if rc != 0:
        raise RuntimeError(f"ora_admm_solve failed: {rc}")
    del keep
    return OracleState(*outs), iters, pcg_iters


def schur_build(qp, rho, sigma, rho_f_factor, *, dtype=np.float64, nthreads=None):
    """compute_S_Phiinv for each problem; returns S, Phiinv of shape (B,T,n,3n)."""
    lib = load()
    dt = np.dtype(dtype)
    d = _dims(qp)
    cq, keep = _qp_arrays(qp, dt)
    r = _arr(np.broadcast_to(rho, (d.B,)), dt)
    S = np.zeros((d.B, d.T, d.n, 3 * d.n), dt)
    P = np.zeros_like(S)
    lib.ora_schur_build(
        dt.itemsize, ctypes.byref(d), ctypes.byref(cq), _ptr(r), ctypes.c_double(sigma),
        ctypes.c_double(rho_f_factor), _ptr(S), _ptr(P), _threads(nthreads),
    )
    del keep
    return S, P


def pcg(S, Phiinv, rhs, x0, *, eps, max_iter, nthreads=None):
    lib = load()
    dt = np.asarray(S).dtype
    S, Phiinv, rhs, x0 = (_arr(a, dt) for a in (S, Phiinv, rhs, x0))
    B, T, n, _ = S.shape
    x = np.zeros_like(rhs)
    iters = np.zeros(B, np.int32)
    lib.ora_pcg(
        dt.itemsize, B, T, n, _ptr(S), _ptr(Phiinv), _ptr(rhs), _ptr(x0), _ptr(x), _ptr(iters),
        ctypes.c_double(eps), ctypes.c_int32(max_iter), _threads(nthreads),
    )
    return x, iters


def blktri_solve(S, rhs, *, nthreads=None):
    lib = load()
    dt = np.asarray(S).dtype
    S, rhs = _arr(S, dt), _arr(rhs, dt)
    B, T, n, _ = S.shape
    x = np.zeros_like(rhs)
    lib.ora_blktri_solve(dt.itemsize, B, T, n, _ptr(S), _ptr(rhs), _ptr(x), _threads(nthreads))
    return x


def adjoint_kkt(qp, *, dtype=np.float64, nthreads=None):
    """Dense adjoint KKT: qp.ineq.G is G_act, qp.cost.q the adjoint linear term."""
    lib = load()
    dt = np.dtype(dtype)
    d = _dims(qp)
    cq, keep = _qp_arrays(qp, dt)
    dz = np.zeros((d.B, d.T, d.n), dt)
    mult = np.zeros((d.B, d.n0 + (d.T - 1) * d.nx + d.T * d.m), dt)
    lib.ora_adjoint_kkt(dt.itemsize, ctypes.byref(d), ctypes.byref(cq), _ptr(dz), _ptr(mult),
                        _threads(nthreads))
    del keep
    return dz, mult


def quadrotor_rk4_jac(xu, dt, params, *, nthreads=None):
    """RK4 step of the rotor-thrust quadrotor and its (13,17) Jacobian per row of xu."""
    lib = load()
    xu = _arr(xu, np.float64).reshape(-1, 17)
    p = _arr(params, np.float64)
    K = xu.shape[0]
    f = np.zeros((K, 13))
    J = np.zeros((K, 13, 17))
    lib.ora_quadrotor_rk4_jac(K, _ptr(xu), ctypes.c_double(dt), _ptr(p), _ptr(f), _ptr(J),
                              _threads(nthreads))
    return f, J
