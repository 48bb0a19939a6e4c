"""Packing helpers (turbompc/solvers/qp_utils.py:22-130), batched over a leading axis."""
from __future__ import annotations

from dataclasses import dataclass
from typing import Tuple

import torch


@dataclass(frozen=True)
class ZShape:
    horizon: int
    num_states: int
    num_controls: int

    @property
    def block_dim(self) -> int:
        return self.num_states + self.num_controls

    @property
    def z_dim(self) -> int:
        return (self.horizon + 1) * self.block_dim


def pack_x(states: torch.Tensor, controls: torch.Tensor) -> torch.Tensor:
    """(..., T, nx), (..., T, nu) -> (..., T, nx+nu)."""
    if states.shape[:-1] != controls.shape[:-1]:
        raise ValueError("states and controls must have the same leading/time dimensions")
    return torch.cat([states, controls], dim=-1)


def unpack_x(x_blocks: torch.Tensor, shape: ZShape) -> Tuple[torch.Tensor, torch.Tensor]:
    if x_blocks.shape[-2] != shape.horizon + 1 or x_blocks.shape[-1] != shape.block_dim:
        raise ValueError(
            f"x_blocks has shape {tuple(x_blocks.shape)}, expected (..., {shape.horizon + 1}, {shape.block_dim})"
        )
    return x_blocks[..., : shape.num_states], x_blocks[..., shape.num_states :]


def pack_z(states: torch.Tensor, controls: torch.Tensor) -> torch.Tensor:
    return pack_x(states, controls).flatten(-2)
