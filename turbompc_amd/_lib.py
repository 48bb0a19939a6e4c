"""ctypes binding of libtmpc_hip.so (the C ABI declared in include/tmpc.h).

Device memory and streams come from PyTorch-ROCm: every array argument is a
contiguous `torch.Tensor` on a HIP device and every call is enqueued on
`torch.cuda.current_stream()`.  The library allocates nothing; workspaces are
torch byte tensors sized by the *_workspace_bytes() queries.

The library location mirrors the reference's `_find_lib`
(turbompc/solvers/admm/admm_ffi_backend.py:15-38): the in-tree build
`turbompc_amd/lib/libtmpc_hip.so`, overridable with the `TMPC_HIP_LIB`
environment variable.  A missing library raises FileNotFoundError, as the
reference does; there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path
from typing import Optional

import torch

_PKG = Path(__file__).resolve().parent
DEFAULT_LIB = _PKG / "lib" / "libtmpc_hip.so"

FLAG_STD_DYNAMICS = 1
FLAG_GENERIC_KERNEL = 2
FLAG_DIAG_COST = 4  # every D_t diagonal
FLAG_WARM_RECORDS = 8  # the workspace's stage records are the previous SQP step's
FLAG_WARM_INEQ = 16  # with FLAG_WARM_RECORDS: G, l, u changed too
FLAG_WARM_SAME_DYNAMICS = 1 << 13  # with FLAG_WARM_RECORDS: A_minus and c unchanged
FLAG_CONST_G = 32  # every G_t the same for every stage and problem (box rows)
FLAG_INVARIANT_A = 64  # with FLAG_CONST_G (n = 17): stage-invariant A_minus entries resident
NOALLOC_SCRATCH_BYTES = 64 << 20  # TMPC_NOALLOC_SCRATCH_BYTES (scratch of tmpc_admm_direct_noalloc)


def flag_stream_p(p: int) -> int:
    """Forces the problems per wavefront of the streaming kernel (1-3)."""
    return (int(p) & 3) << 8


PCG_KERNEL_DPP, PCG_KERNEL_LDS, PCG_KERNEL_CHUNK = 1, 2, 3
FLAG_FACTOR_GROUPS = 1 << 12  # the lane-group factorization (cross-checks)


def flag_pcg_kernel(k: int) -> int:
    """TMPC_FLAG_PCG_KERNEL: forces the PCG ADMM kernel (1 row-broadcast,
    2 LDS-resident, 3 chunked)."""
    return (int(k) & 3) << 10

_STATUS = {
    0: "ok",
    1: "unsupported dimensions",
    2: "invalid argument",
    3: "workspace too small",
    4: "HIP launch failed",
    5: "problem needs more than the allocation-free scratch",
    6: "non-finite values in the solution",
}


class TmpcError(RuntimeError):
    """Non-zero tmpc_status returned by the library."""

    def __init__(self, fn: str, status: int):
        super().__init__(f"{fn} failed: {_STATUS.get(status, status)} (status {status})")
        self.status = status


class Dims(ctypes.Structure):
    _fields_ = [(k, ctypes.c_int32) for k in ("B", "T", "n", "nx", "n0", "m")]


class QP(ctypes.Structure):
    _fields_ = [
        (k, ctypes.c_void_p)
        for k in ("D", "E", "q", "A0", "A_minus", "A_plus", "G", "l", "u", "c0", "c", "slack_weight")
    ]


class State(ctypes.Structure):
    _fields_ = [(k, ctypes.c_void_p) for k in ("x", "z_g", "y_g", "y_f0", "y_f", "xi_g", "rho")]


class AdmmCfg(ctypes.Structure):
    _fields_ = [
        ("max_iter", ctypes.c_int32),
        ("check_every", ctypes.c_int32),
        ("adapt_rho_every", ctypes.c_int32),
        ("pcg_max_iter", ctypes.c_int32),
        ("use_slack", ctypes.c_int32),
        ("flags", ctypes.c_uint32),
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


class SqpStep(ctypes.Structure):
    _fields_ = [
        ("active_in", ctypes.c_void_p),
        ("active_out", ctypes.c_void_p),
        ("tol", ctypes.c_double),
        ("conv", ctypes.c_void_p),
        ("eq_err", ctypes.c_void_p),
        ("ineq_err", ctypes.c_void_p),
        ("g_out", ctypes.c_void_p),
    ]


class MeritTerms(ctypes.Structure):
    """tmpc_merit_terms: device arrays as c_void_p, the per-row constants as
    host arrays (POINTER(c_double) / POINTER(c_int32))."""
    _PDBL, _PI32 = ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int32)
    _fields_ = [(k, ctypes.c_int32) for k in ("P", "B0", "T", "nx", "nu", "mbox")] + [
        (k, ctypes.c_void_p) for k in ("states", "controls", "next", "x0", "u0", "w", "zref")
    ] + [
        ("scaled", ctypes.c_int32),
        ("state_scale", _PDBL),
        ("control_scale", _PDBL),
        ("box_idx", _PI32),
        ("box_lo", _PDBL),
        ("box_hi", _PDBL),
        ("box_scale", _PDBL),
        ("slacks", ctypes.c_void_p),
        ("gamma", ctypes.c_double),
    ] + [(k, ctypes.c_void_p) for k in ("dstates", "dcontrols", "dslacks", "cost", "dcost", "eq", "iq")] + [
        ("nobs", ctypes.c_int32),
        ("dim", ctypes.c_int32),
        ("centers", ctypes.c_void_p),
        ("radii", ctypes.c_void_p),
        ("obs_scale", ctypes.c_double),
        ("lin_A", ctypes.c_void_p),
        ("lin_B", ctypes.c_void_p),
        ("lin_b", ctypes.c_void_p),
    ]


# name -> argtypes (restype is int unless listed in _SIZE_FNS)
_VP, _I32, _U32, _F64, _SZ = ctypes.c_void_p, ctypes.c_int32, ctypes.c_uint32, ctypes.c_double, ctypes.c_size_t
_PD, _PQ, _PS, _PC, _PSQ = (ctypes.POINTER(t) for t in (Dims, QP, State, AdmmCfg, SqpStep))
SIGNATURES = {
    "tmpc_version": [],
    "tmpc_set_timing_events": [_VP, _VP],
    "tmpc_fill_zero": [_VP, _VP, _SZ],
    "tmpc_status_string": [ctypes.c_int],
    "tmpc_admm_direct_workspace_bytes": [ctypes.c_int, _PD],
    "tmpc_admm_direct_f32": [_VP, _PD, _PQ, _PS, _PS, _VP, _PC, _VP, _SZ],
    "tmpc_admm_direct_f64": [_VP, _PD, _PQ, _PS, _PS, _VP, _PC, _VP, _SZ],
    "tmpc_admm_direct_noalloc": [_VP, ctypes.c_int, _PD, _PQ, _PS, _PS, _VP, _PC],
    "tmpc_sqp_admm_step_f32": [_VP, _PD, _PQ, _PS, _PS, _VP, _PC, _PSQ, _VP, _SZ],
    "tmpc_sqp_admm_step_f64": [_VP, _PD, _PQ, _PS, _PS, _VP, _PC, _PSQ, _VP, _SZ],
    "tmpc_sqp_admm_step_quadrotor_f32": [_VP, _PD, _PQ, _PS, _PS, _VP, _PC, _PSQ, _F64, _VP, _VP, _SZ],
    "tmpc_sqp_admm_step_quadrotor_f64": [_VP, _PD, _PQ, _PS, _PS, _VP, _PC, _PSQ, _F64, _VP, _VP, _SZ],
    "tmpc_sqp_admm_step_obstacle_f32": [_VP, _PD, _PQ, _PS, _PS, _VP, _PC, _PSQ, _I32, _I32, _VP, _VP, _I32,
                                        _VP, _SZ],
    "tmpc_sqp_admm_step_obstacle_f64": [_VP, _PD, _PQ, _PS, _PS, _VP, _PC, _PSQ, _I32, _I32, _VP, _VP, _I32,
                                        _VP, _SZ],
    "tmpc_admm_pcg_workspace_bytes": [ctypes.c_int, _PD],
    "tmpc_admm_pcg_f32": [_VP, _PD, _PQ, _PS, _PS, _VP, _VP, _PC, _VP, _SZ],
    "tmpc_admm_pcg_f64": [_VP, _PD, _PQ, _PS, _PS, _VP, _VP, _PC, _VP, _SZ],
    "tmpc_schur_build_f32": [_VP, _PD, _PQ, _VP, _F64, _F64, _VP, _VP],
    "tmpc_schur_build_f64": [_VP, _PD, _PQ, _VP, _F64, _F64, _VP, _VP],
    "tmpc_schur_pcg_workspace_bytes": [ctypes.c_int, _I32, _I32, _I32],
    "tmpc_schur_pcg_f32": [_VP, _I32, _I32, _I32, _VP, _VP, _VP, _VP, _VP, _VP, _F64, _I32, _VP, _SZ],
    "tmpc_schur_pcg_f64": [_VP, _I32, _I32, _I32, _VP, _VP, _VP, _VP, _VP, _VP, _F64, _I32, _VP, _SZ],
    "tmpc_blktri_workspace_bytes": [ctypes.c_int, _I32, _I32, _I32],
    "tmpc_blktri_factor_f32": [_VP, _I32, _I32, _I32, _VP, _VP, _SZ],
    "tmpc_blktri_factor_f64": [_VP, _I32, _I32, _I32, _VP, _VP, _SZ],
    "tmpc_blktri_solve_f32": [_VP, _I32, _I32, _I32, _VP, _VP, _VP, _VP, _SZ],
    "tmpc_blktri_solve_f64": [_VP, _I32, _I32, _I32, _VP, _VP, _VP, _VP, _SZ],
    "tmpc_adjoint_kkt_workspace_bytes": [ctypes.c_int, _PD],
    "tmpc_adjoint_kkt_f32": [_VP, _PD, _PQ, _VP, _VP, _F64, _I32, _U32, _VP, _SZ],
    "tmpc_adjoint_kkt_f64": [_VP, _PD, _PQ, _VP, _VP, _F64, _I32, _U32, _VP, _SZ],
    "tmpc_sqp_first_order_f32": [_VP, _PD, _PQ, _VP, _VP, _VP, _VP, _VP, _F64, _U32, _VP, _VP, _VP, _VP],
    "tmpc_sqp_first_order_f64": [_VP, _PD, _PQ, _VP, _VP, _VP, _VP, _VP, _F64, _U32, _VP, _VP, _VP, _VP],
    "tmpc_ocp_merit_terms_f32": [_VP, ctypes.POINTER(MeritTerms)],
    "tmpc_ocp_merit_terms_f64": [_VP, ctypes.POINTER(MeritTerms)],
    "tmpc_linesearch_choose_f32": [_VP, _I32, _I32] + [_VP] * 7 + [_VP, _F64, _F64, _F64, _F64, _VP, _VP],
    "tmpc_linesearch_choose_f64": [_VP, _I32, _I32] + [_VP] * 7 + [_VP, _F64, _F64, _F64, _F64, _VP, _VP],
    "tmpc_kkt_active_sets_f32": [_VP, ctypes.c_int64, _VP, _VP, _VP, _VP, _F64, _F64, _F64, _VP, _VP],
    "tmpc_kkt_active_sets_f64": [_VP, ctypes.c_int64, _VP, _VP, _VP, _VP, _F64, _F64, _F64, _VP, _VP],
    "tmpc_quadrotor_linearize_f32": [_VP, _I32, _I32, _VP, _VP, _F64, _VP, _VP, _VP],
    "tmpc_quadrotor_linearize_f64": [_VP, _I32, _I32, _VP, _VP, _F64, _VP, _VP, _VP],
    "tmpc_quadrotor_linearize_strided_f32": [_VP, _I32, _I32, _VP, ctypes.c_int64, _VP, ctypes.c_int64, _F64, _VP,
                                             _VP, _VP],
    "tmpc_quadrotor_linearize_strided_f64": [_VP, _I32, _I32, _VP, ctypes.c_int64, _VP, ctypes.c_int64, _F64, _VP,
                                             _VP, _VP],
    "tmpc_linear_dynamics_f32": [_VP, _I32, _I32, _I32, _I32, _VP, _VP, _VP, _VP, _VP, _VP],
    "tmpc_linear_dynamics_f64": [_VP, _I32, _I32, _I32, _I32, _VP, _VP, _VP, _VP, _VP, _VP],
    "tmpc_quadrotor_dynamics_f32": [_VP, _I32, _I32, _VP, _VP, _F64, _VP, _VP],
    "tmpc_quadrotor_dynamics_f64": [_VP, _I32, _I32, _VP, _VP, _F64, _VP, _VP],
    "tmpc_quadrotor_lagrangian_hessian_f32": [_VP, _I32, _I32, _VP, _VP, _F64, _VP, _VP, _VP],
    "tmpc_quadrotor_lagrangian_hessian_f64": [_VP, _I32, _I32, _VP, _VP, _F64, _VP, _VP, _VP],
    "tmpc_obstacle_linearize_f32": [_VP] + [_I32] * 6 + [_VP] * 3 + [_I32, _I32] + [_VP] * 3,
    "tmpc_obstacle_linearize_f64": [_VP] + [_I32] * 6 + [_VP] * 3 + [_I32, _I32] + [_VP] * 3,
    "tmpc_obstacle_lagrangian_hessian_f32": [_VP] + [_I32] * 6 + [_VP] * 3 + [_I32, _I32] + [_VP] * 2,
    "tmpc_obstacle_lagrangian_hessian_f64": [_VP] + [_I32] * 6 + [_VP] * 3 + [_I32, _I32] + [_VP] * 2,
}
_SIZE_FNS = {
    "tmpc_admm_direct_workspace_bytes",
    "tmpc_admm_pcg_workspace_bytes",
    "tmpc_blktri_workspace_bytes",
    "tmpc_schur_pcg_workspace_bytes",
    "tmpc_adjoint_kkt_workspace_bytes",
}

_LIB: Optional[ctypes.CDLL] = None


def lib_path() -> Path:
    env = os.environ.get("TMPC_HIP_LIB")
    return Path(env) if env else DEFAULT_LIB


def load() -> ctypes.CDLL:
    """Load libtmpc_hip.so; FileNotFoundError if it has not been built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    p = lib_path()
    if not p.exists():
        raise FileNotFoundError(
            f"Could not find {p}. Build it first:\n"
            "  python -c 'import __graft_entry__ as g; g.build()'"
        )
    lib = ctypes.CDLL(str(p))
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        if name in _SIZE_FNS:
            fn.restype = ctypes.c_size_t
        elif name == "tmpc_status_string":
            fn.restype = ctypes.c_char_p
        elif name == "tmpc_set_timing_events":
            fn.restype = None
        else:
            fn.restype = ctypes.c_int
    _LIB = lib
    return lib


def check(fn: str, status: int) -> None:
    if status != 0:
        raise TmpcError(fn, status)


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    if t is None:
        return None
    if not t.is_contiguous():
        raise ValueError("tensor must be contiguous")
    return t.data_ptr() if t.numel() else None


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def suffix(dtype: torch.dtype) -> str:
    if dtype == torch.float32:
        return "f32"
    if dtype == torch.float64:
        return "f64"
    raise TypeError(f"unsupported dtype {dtype}; use float32 or float64")


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


class IterationTimer:
    """Times the ADMM-iteration phase of tmpc_admm_direct_* calls with HIP
    events recorded by the library (tmpc_set_timing_events).  Use as a context
    manager around each solve; read the millisecond durations with results()
    after synchronising the device."""

    def __init__(self):
        self._pairs = []
        self._pool = []
        self._lib = load()

    @staticmethod
    def _new_pair():
        import torch

        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()  # materialise the underlying HIP events
        e1.record()
        return e0, e1

    def reserve(self, n: int):
        """Materialise n event pairs now (their first records are queued here,
        e.g. before a timed region), for the next n solves to use."""
        self._pool.extend(self._new_pair() for _ in range(n))

    def __enter__(self):
        e0, e1 = self._pool.pop() if self._pool else self._new_pair()
        self._lib.tmpc_set_timing_events(ctypes.c_void_p(e0.cuda_event), ctypes.c_void_p(e1.cuda_event))
        self._pairs.append((e0, e1))
        return self

    def __exit__(self, *exc):
        self._lib.tmpc_set_timing_events(None, None)
        return False

    def clear(self):
        self._pairs.clear()

    def results(self):
        return [a.elapsed_time(b) for a, b in self._pairs]
