"""Solver layer mirroring turbompc/solvers of the reference."""
