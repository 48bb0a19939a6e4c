"""Adjoint (backward) KKT solve (turbompc/solvers/backward)."""
