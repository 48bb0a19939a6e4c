from .admm import ADMMParams, ADMMSolver, ADMMState, ADMMStats, compute_S_Phiinv  # noqa: F401
