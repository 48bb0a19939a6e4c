"""Batched QP containers (turbompc/solvers/qp_data.py:11-100), torch tensors.

The QP is  min 1/2 z^T P z + q^T z  s.t.  C z = c,  l <= G z <= u  with P block
tridiagonal (D on the diagonal, E below it), C = [A0 rows; A_minus_t, A_plus_t
per stage] and G block diagonal.  Every field carries a leading batch axis B:
  D (B,T,n,n)  E (B,N,n,n)  q (B,T,n)  A0 (B,n0,n)  A_minus, A_plus (B,N,nx,n)
  c0 (B,n0)  c (B,N,nx)  G (B,T,m,n)  l, u (B,T,m)
which is exactly the array layout the HIP library reads.
"""
from __future__ import annotations

from dataclasses import dataclass, field, replace

import torch


@dataclass(frozen=True)
class QPCostBlocks:
    D: torch.Tensor
    E: torch.Tensor
    q: torch.Tensor


@dataclass(frozen=True)
class QPEqualityBlocks:
    A0: torch.Tensor
    A_minus: torch.Tensor
    A_plus: torch.Tensor
    c0: torch.Tensor
    c: torch.Tensor


@dataclass(frozen=True)
class QPInequalityBlocks:
    G: torch.Tensor
    l: torch.Tensor
    u: torch.Tensor
    slack_penalization_weight: torch.Tensor = field(default_factory=lambda: torch.tensor(0.0))
    use_slack_variables: bool = False


@dataclass(frozen=True)
class QPData:
    cost: QPCostBlocks
    eq: QPEqualityBlocks
    ineq: QPInequalityBlocks

    @property
    def batch(self) -> int:
        return int(self.cost.D.shape[0])

    @property
    def dims(self):
        """(B, T, n, nx, n0, m)."""
        B, T, n, _ = self.cost.D.shape
        return (
            int(B),
            int(T),
            int(n),
            int(self.eq.A_minus.shape[-2]),
            int(self.eq.A0.shape[-2]),
            int(self.ineq.G.shape[-2]),
        )

    @property
    def dtype(self) -> torch.dtype:
        return self.cost.D.dtype

    @property
    def device(self) -> torch.device:
        return self.cost.D.device

    def to(self, device=None, dtype=None) -> "QPData":
        def cv(t):
            return t.to(device=device, dtype=dtype).contiguous()

        sw = torch.as_tensor(self.ineq.slack_penalization_weight)
        return QPData(
            cost=QPCostBlocks(cv(self.cost.D), cv(self.cost.E), cv(self.cost.q)),
            eq=QPEqualityBlocks(
                cv(self.eq.A0), cv(self.eq.A_minus), cv(self.eq.A_plus), cv(self.eq.c0), cv(self.eq.c)
            ),
            ineq=QPInequalityBlocks(
                cv(self.ineq.G),
                cv(self.ineq.l),
                cv(self.ineq.u),
                sw.to(device=device, dtype=dtype),
                self.ineq.use_slack_variables,
            ),
        )

    def replace_cost(self, **kw) -> "QPData":
        return replace(self, cost=replace(self.cost, **kw))

    def replace_eq(self, **kw) -> "QPData":
        return replace(self, eq=replace(self.eq, **kw))

    def replace_ineq(self, **kw) -> "QPData":
        return replace(self, ineq=replace(self.ineq, **kw))


def qpdata_from_ocp_blocks(D, E, q, A0, c0, As_next, Bs_next, As, Bs, c_dyn, ineq_blocks, ineq_l, ineq_u,
                           use_slack_variables=False, slack_penalization_weight=0.0) -> QPData:
    """Build QPData from OCP linearization blocks (qp_data.py:140-175), batched."""
    A_minus = torch.cat([As, Bs], dim=-1)
    A_plus = torch.cat([As_next, Bs_next], dim=-1)
    return QPData(
        cost=QPCostBlocks(D, E, q),
        eq=QPEqualityBlocks(A0, A_minus, A_plus, c0, c_dyn),
        ineq=QPInequalityBlocks(
            ineq_blocks, ineq_l, ineq_u, torch.as_tensor(slack_penalization_weight), use_slack_variables
        ),
    )


def scale_qp_data(qp: QPData, state_scale: torch.Tensor, control_scale: torch.Tensor) -> QPData:
    """The QP in the variables z_hat with z = S z_hat, S = diag(state_scale,
    control_scale) (scale_qp_data, qp_data.py:178-211): the cost blocks become
    S D S, S E S and S q, and every constraint block's columns are scaled by S;
    the right-hand sides and bounds are unchanged."""
    s = torch.cat([torch.as_tensor(state_scale), torch.as_tensor(control_scale)]).to(qp.cost.D)
    col = lambda a: a * s  # noqa: E731  (columns: the last axis)
    sym = lambda a: a * s[:, None] * s  # noqa: E731
    return QPData(
        cost=QPCostBlocks(sym(qp.cost.D), sym(qp.cost.E), qp.cost.q * s),
        eq=QPEqualityBlocks(col(qp.eq.A0), col(qp.eq.A_minus), col(qp.eq.A_plus), qp.eq.c0, qp.eq.c),
        ineq=QPInequalityBlocks(col(qp.ineq.G), qp.ineq.l, qp.ineq.u, qp.ineq.slack_penalization_weight,
                                qp.ineq.use_slack_variables),
    )


def is_std_dynamics(qp: QPData) -> bool:
    """True when every A_plus_t == [-I 0] and every E_t == 0 (explicit schemes
    without a control-rate cost, optimal_control_problem.py:1267-1272)."""
    _, _, n, nx, _, _ = qp.dims
    ref = torch.zeros(nx, n, dtype=qp.dtype, device=qp.device)
    ref[:, :nx] = -torch.eye(nx, dtype=qp.dtype, device=qp.device)
    return bool(torch.equal(qp.eq.A_plus, ref.expand_as(qp.eq.A_plus))) and not bool(
        torch.any(qp.cost.E != 0)
    )
