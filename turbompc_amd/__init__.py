"""turbompc_amd — MI355X-native (gfx950) backend for TurboMPC's batched SQP+ADMM solve.

The hot path (ADMM iterations, block-tridiagonal Schur factorization/solve,
Schur PCG, adjoint KKT, quadrotor SQP linearization) runs in the HIP library
`turbompc_amd/lib/libtmpc_hip.so` behind the C ABI of `include/tmpc.h`.  The
Python layer mirrors the reference's solver API (turbompc/solvers/...) over
PyTorch-ROCm device tensors with a leading batch axis.
"""
__version__ = "0.1.0"
