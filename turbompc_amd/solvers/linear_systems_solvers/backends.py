"""Backend enums (turbompc/solvers/linear_systems_solvers/backends.py:6-21).

The reference members are kept so code that names them still parses; the JAX
and CUDA ones are not available in this package and are rejected where a
solver is constructed.  The HIP members are the new gfx950 backends.
"""
from __future__ import annotations

import enum


class SchurSolverBackend(enum.IntEnum):
    IGNORED = -1
    PCG = 0
    PCG_FFI = 1
    CUDSS_FFI = 2
    JAX_DENSE = 3
    HIP_DIRECT = 4  # batched block-tridiagonal factorize/solve (replaces cuDSS)
    HIP_PCG = 5  # batched Schur PCG with the reference block preconditioner


class AdmmBackend(enum.IntEnum):
    JAX_LOOP = 0
    FUSED_PCG = 1
    FUSED_CUDSS = 2
    HIP_DIRECT = 3  # fused ADMM chunks over the exact block-tridiagonal solve
    HIP_PCG = 4  # fused ADMM chunks over PCG


HIP_SCHUR_BACKENDS = (SchurSolverBackend.HIP_DIRECT, SchurSolverBackend.HIP_PCG)
HIP_ADMM_BACKENDS = (AdmmBackend.HIP_DIRECT, AdmmBackend.HIP_PCG)
