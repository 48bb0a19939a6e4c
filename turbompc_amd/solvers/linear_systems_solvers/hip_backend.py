"""Schur-level HIP entry points: direct block-tridiagonal solve and PCG.

Drop-in counterparts of the reference's Schur-only FFI calls:
  hip_blktri_solve   <- cudss_ffi_solve  (linear_systems_solvers/cudss_ffi_backend.py:42-83)
  hip_pcg_solve      <- pcg_ffi_solve    (linear_systems_solvers/pcg_ffi_backend.py:44-108)
Inputs are batched device tensors: S, Phiinv (B,T,n,3n), rhs, x0 (B,T,n).
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from ... import _lib


def _check_blocks(S: torch.Tensor, rhs: torch.Tensor):
    if S.dim() != 4 or S.shape[-1] != 3 * S.shape[-2]:
        raise ValueError(f"S must be (B,T,n,3n), got {tuple(S.shape)}")
    B, T, n, _ = S.shape
    if tuple(rhs.shape) != (B, T, n):
        raise ValueError(f"rhs must be {(B, T, n)}, got {tuple(rhs.shape)}")
    if not S.is_cuda:
        raise ValueError("S must be a device tensor")
    return int(B), int(T), int(n)


class BlockTriFactor:
    """Factor of a batch of SPD block-tridiagonal matrices, reusable across solves."""

    def __init__(self, S: torch.Tensor):
        lib = _lib.load()
        S = S.contiguous()
        B, T, n, _ = S.shape
        self.S, self.B, self.T, self.n = S, int(B), int(T), int(n)
        self.nbytes = lib.tmpc_blktri_workspace_bytes(S.element_size(), self.B, self.T, self.n)
        if self.nbytes == 0:
            raise ValueError(f"unsupported Schur block shape {tuple(S.shape)}")
        self.ws = _lib.workspace(self.nbytes, S.device)
        sfx = _lib.suffix(S.dtype)
        st = getattr(lib, f"tmpc_blktri_factor_{sfx}")(
            _lib.stream_handle(S.device), self.B, self.T, self.n, _lib.ptr(S), _lib.ptr(self.ws), self.nbytes
        )
        _lib.check(f"tmpc_blktri_factor_{sfx}", st)

    def solve(self, rhs: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        lib = _lib.load()
        _check_blocks(self.S, rhs)
        rhs = rhs.to(self.S.dtype).contiguous()
        x = torch.empty_like(rhs) if out is None else out
        sfx = _lib.suffix(self.S.dtype)
        st = getattr(lib, f"tmpc_blktri_solve_{sfx}")(
            _lib.stream_handle(rhs.device), self.B, self.T, self.n, _lib.ptr(self.S), _lib.ptr(rhs), _lib.ptr(x),
            _lib.ptr(self.ws), self.nbytes,
        )
        _lib.check(f"tmpc_blktri_solve_{sfx}", st)
        return x


def hip_blktri_solve(S: torch.Tensor, rhs: torch.Tensor) -> torch.Tensor:
    """Exact solve of S x = rhs for each problem of the batch."""
    _check_blocks(S, rhs)
    return BlockTriFactor(S).solve(rhs)


def hip_pcg_solve(S: torch.Tensor, Phiinv: torch.Tensor, rhs: torch.Tensor, x0: torch.Tensor, *, eps: float,
                  max_iters: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """PCG on S x = rhs from x0 with the reference preconditioner; returns (x, iters)."""
    lib = _lib.load()
    B, T, n = _check_blocks(S, rhs)
    S, Phiinv = S.contiguous(), Phiinv.to(S.dtype).contiguous()
    rhs, x0 = rhs.to(S.dtype).contiguous(), x0.to(S.dtype).contiguous()
    x = torch.empty_like(rhs)
    iters = torch.zeros(B, dtype=torch.int32, device=S.device)
    nbytes = lib.tmpc_schur_pcg_workspace_bytes(S.element_size(), B, T, n)
    ws = _lib.workspace(nbytes, S.device)
    sfx = _lib.suffix(S.dtype)
    st = getattr(lib, f"tmpc_schur_pcg_{sfx}")(
        _lib.stream_handle(S.device), B, T, n, _lib.ptr(S), _lib.ptr(Phiinv), _lib.ptr(rhs), _lib.ptr(x0),
        _lib.ptr(x), _lib.ptr(iters), float(eps), int(max_iters), _lib.ptr(ws), nbytes,
    )
    _lib.check(f"tmpc_schur_pcg_{sfx}", st)
    return x, iters
