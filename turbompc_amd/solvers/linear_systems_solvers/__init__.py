"""Schur linear-system layer (turbompc/solvers/linear_systems_solvers)."""
