"""Batched QP operators in torch (turbompc/solvers/admm/admm.py:185-263).

Host-side helpers for the SQP driver's first-order check, the KKT state and
the gradient assembly; the ADMM iterations themselves never call them.
All tensors carry a leading batch axis.
"""
from __future__ import annotations

from typing import Tuple

import torch

from .qp_data import QPData


# Block products as broadcast-multiply-reduce: the blocks are tiny (at most
# 64 x 64) and batched over B x T, which a batched GEMM library call handles
# far worse than one elementwise pass over the blocks.
def _mv(A: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    return (A * x.unsqueeze(-2)).sum(-1)


def _mtv(A: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    return (A * y.unsqueeze(-1)).sum(-2)


def apply_P(qp: QPData, x: torch.Tensor) -> torch.Tensor:
    """Row t: E_{t-1} x_{t-1} + D_t x_t + E_t^T x_{t+1} (admm.py:185-206)."""
    out = _mv(qp.cost.D, x)
    out[:, 1:] += _mv(qp.cost.E, x[:, :-1])
    out[:, :-1] += _mtv(qp.cost.E, x[:, 1:])
    return out


def apply_C_parts(qp: QPData, x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """A0 x_0 and A_minus_t x_t + A_plus_t x_{t+1} (admm.py:209-221)."""
    return _mv(qp.eq.A0, x[:, 0]), _mv(qp.eq.A_minus, x[:, :-1]) + _mv(qp.eq.A_plus, x[:, 1:])


def apply_Ct(qp: QPData, y0: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    """C^T [y0; y] in stage form (admm.py:229-249)."""
    B, T, n, *_ = qp.dims
    out = torch.zeros((B, T, n), dtype=qp.dtype, device=qp.device)
    out[:, 0] += _mtv(qp.eq.A0, y0)
    out[:, :-1] += _mtv(qp.eq.A_minus, y)
    out[:, 1:] += _mtv(qp.eq.A_plus, y)
    return out


def apply_G(qp: QPData, x: torch.Tensor) -> torch.Tensor:
    return _mv(qp.ineq.G, x)


def apply_Gt(qp: QPData, y: torch.Tensor) -> torch.Tensor:
    return _mtv(qp.ineq.G, y)


def inf_norm(v: torch.Tensor) -> torch.Tensor:
    """Per-problem max |v| over all but the batch axis (0 for empty)."""
    if v.numel() == 0:
        return torch.zeros(v.shape[0], dtype=v.dtype, device=v.device)
    return v.abs().flatten(1).amax(dim=1)
