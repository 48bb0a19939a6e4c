"""Schur system solvers (turbompc/solvers/linear_systems_solvers/schur_solver.py:20-143).

`SchurSystemSolver.solve(schur, gammas, zs_guess) -> (x, PCGDebugOutput)` keeps
the reference signature; inputs are batched (B,T,...) device tensors.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Dict, NamedTuple, Tuple

import torch

from .backends import SchurSolverBackend
from .hip_backend import hip_blktri_solve, hip_pcg_solve


class PCGDebugOutput(NamedTuple):
    num_iterations: Any
    convergence_eta: Any


class SchurComplementMatrices(NamedTuple):
    """S and the block preconditioner Phiinv, each (B, T, n, 3n) (pcg_primal.py:23-27)."""

    S: torch.Tensor
    preconditioner_Phiinv: torch.Tensor


@dataclass(frozen=True)
class SchurSystemSolver:
    horizon: int
    num_states: int
    num_controls: int
    backend: SchurSolverBackend
    name: str

    def solve(self, schur: SchurComplementMatrices, gammas: torch.Tensor,
              zs_guess: torch.Tensor) -> Tuple[torch.Tensor, PCGDebugOutput]:
        raise NotImplementedError


@dataclass(frozen=True)
class HipDirectSchurSolver(SchurSystemSolver):
    """Exact batched block-tridiagonal solve on the GPU (replaces CudssFfiSchurSolver)."""

    def solve(self, schur, gammas, zs_guess):
        x = hip_blktri_solve(schur.S, gammas)
        return x, PCGDebugOutput(num_iterations=torch.zeros((), dtype=torch.int32), convergence_eta=0.0)


@dataclass(frozen=True)
class HipPcgSchurSolver(SchurSystemSolver):
    """Batched PCG on the GPU (replaces PcgFfiSchurSolver)."""

    pcg_params: Dict[str, Any]

    def solve(self, schur, gammas, zs_guess):
        x, iters = hip_pcg_solve(
            schur.S,
            schur.preconditioner_Phiinv,
            gammas,
            zs_guess,
            eps=float(self.pcg_params["tol_epsilon"]),
            max_iters=int(self.pcg_params["max_iter"]),
        )
        return x, PCGDebugOutput(num_iterations=iters, convergence_eta=0.0)


def make_schur_solver(backend: SchurSolverBackend, horizon: int, num_states: int, num_controls: int, *,
                      pcg_params: Dict[str, Any]) -> SchurSystemSolver:
    """Factory (schur_solver.py:95-143) restricted to the HIP backends."""
    backend = SchurSolverBackend(backend)
    if backend == SchurSolverBackend.HIP_DIRECT:
        return HipDirectSchurSolver(horizon, num_states, num_controls, backend, "HipDirectSchurSolver")
    if backend == SchurSolverBackend.HIP_PCG:
        return HipPcgSchurSolver(horizon, num_states, num_controls, backend, "HipPcgSchurSolver", dict(pcg_params))
    if backend == SchurSolverBackend.IGNORED:
        raise ValueError("SchurSolverBackend.IGNORED cannot be used to construct a solver.")
    raise ValueError(
        f"Schur backend {backend.name} needs the reference's JAX/CUDA stack, which this package does not"
        " provide; use HIP_DIRECT or HIP_PCG."
    )
