"""TEST INFRASTRUCTURE ONLY — CPU oracle for the batched ADMM / Schur / adjoint path.

Only `tests/`, `__graft_entry__.smoke()` and `bench.py`'s `cpu_baseline` leg may
import this package, and only as the checker (or the timed CPU baseline).  The
product package `turbompc_amd` never imports it.

`liboracle.so` (built from `oracle.cpp` by `make -C oracle`) restates the
reference's pure-JAX CPU path:
  * ADMM loop       turbompc/solvers/admm/admm.py:795-1049 (`_solve_jax_loop`)
  * S / Phiinv      turbompc/solvers/admm/admm.py:71-154 (`compute_S_Phiinv`)
  * PCG             turbompc/solvers/linear_systems_solvers/pcg_primal.py:70-175
  * exact Schur     turbompc/solvers/linear_systems_solvers/linear_solve.py:85-112
                    (restated as a block Cholesky solve)
  * adjoint KKT     turbompc/solvers/backward/backward_kkt_jax.py:10-211
  * quadrotor RK4 Jacobian by complex-step differentiation.
The pins that fix each function are listed at the top of oracle.cpp and live in
tests/test_oracle_*.py.
"""
from .oracle import (  # noqa: F401
    OracleCfg,
    OracleState,
    admm_solve,
    adjoint_kkt,
    blktri_solve,
    load,
    pcg,
    quadrotor_rk4_jac,
    schur_build,
    use_native_build,
)
