"""Stage-invariant A_minus entries resident in LDS (TMPC_FLAG_INVARIANT_A, the
AINV form of the n = 17 streaming kernel, with the resident G rows of
TMPC_FLAG_CONST_G).

The library finds on the device which entries of A_minus_t are equal, bit for
bit, in every stage of every problem; the kernel keeps those in its LDS slots
(from each problem's stage-0 record) and streams only the others.  The
products read the same values as the form that streams whole records, so the
iterates must be equal bit for bit to both other forms (whole records; G rows
resident only), and match the fp64 oracle (admm.py:795-1049) as those do.
Covered: a quadrotor-like pattern (constant position/velocity columns and a
constant row), linear time-invariant dynamics (every entry invariant: nothing
streamed), all entries varying, a single entry that varies in one stage of one
problem, a partial last wavefront, N = 1, adaptive rho (the later chunks read
the compressed runs the first chunk wrote), a shape outside the form (flag
ignored), the mask itself read back from the workspace, a workspace without
the form's room, and the SQP solver's default.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from helpers import np_qp, random_qp, rel_err, zero_state
from turbompc_amd import _lib
from turbompc_amd.problems.quadrotor import make_quadrotor_config
from turbompc_amd.solvers.admm.admm import ADMMSolver, ADMMState
from turbompc_amd.solvers.admm.admm_hip_backend import cfg_struct, qp_struct, state_struct
from turbompc_amd.solvers.qp_utils import ZShape

pytestmark = pytest.mark.gpu
DEV = "cuda"
FIELDS = ("x_blocks", "z_g", "y_g", "y_f_0", "y_f_dyn", "xi_g", "rho_bar")


def _pattern(qp, kind, seed=0):
    """qp with A_minus made stage-invariant in the entries `kind` names."""
    Am = qp.eq.A_minus.clone()
    B, N, nx, n = Am.shape
    if kind == "quad":  # position and velocity columns, and the last row
        for j in (0, 1, 2, 7, 8, 9) if n == 17 else (0, 1, 2):
            Am[:, :, :, j] = Am[:, :1, :, j]
        Am[:, :, nx - 1, :] = Am[:, :1, nx - 1, :]
    elif kind == "lti":
        Am[:] = Am[:, :1]
    elif kind == "one":  # every entry invariant but one, in one stage of one problem
        Am[:] = Am[:, :1]
        if N > 4:
            Am[min(2, B - 1), 4, 3, 5 if n > 5 else 1] += 0.25
    elif kind != "varying":
        raise ValueError(kind)
    return qp.replace_eq(A_minus=Am)


def _shared_g(qp, seed=0):
    """One G_t (problem 0's stage 0) for every stage and problem, with bounds
    around G z at a point z that satisfies the equality constraints."""
    from helpers import dense_C

    G = qp.ineq.G[:1, :1].expand_as(qp.ineq.G).contiguous()
    a = np_qp(qp)
    B, T, m, n = G.shape
    rng = np.random.default_rng(seed)
    l, u = np.empty((B, T, m)), np.empty((B, T, m))
    for b in range(B):
        C = dense_C(a["A0"][b], a["Am"][b], a["Ap"][b])
        z = np.linalg.lstsq(C, np.concatenate([a["c0"][b], a["c"][b].reshape(-1)]), rcond=None)[0].reshape(T, n)
        gz = np.einsum("tij,tj->ti", G[b].numpy(), z)
        l[b] = gz - rng.uniform(0.05, 0.5, size=(T, m))
        u[b] = gz + rng.uniform(0.05, 0.5, size=(T, m))
    return qp.replace_ineq(G=G, l=torch.tensor(l), u=torch.tensor(u))


def _varying_mask(Am: torch.Tensor) -> np.ndarray:
    """Host restatement of the mask: entry e of the row-major nx x n block
    varies when some problem's A_minus_t differs from its A_minus_0 as bits."""
    B, N, nx, n = Am.shape
    bits = Am.contiguous().view(torch.int64 if Am.dtype == torch.float64 else torch.int32)
    var = (bits != bits[:, :1]).any(dim=0).any(dim=0).reshape(-1).cpu().numpy()
    words = np.zeros(7, dtype=np.uint32)
    for e in np.nonzero(var)[0]:
        words[e // 32] |= np.uint32(1) << np.uint32(e % 32)
    return words


def _solve(qp, cfg, dtype, P, const_g, invariant_a):
    B, T, n, nx, n0, m = qp.dims
    solver = ADMMSolver(ZShape(T - 1, nx, n - nx), {}, sigma=cfg.sigma, max_iter=cfg.max_iter, eps_abs=cfg.eps_abs,
                        eps_rel=cfg.eps_rel, rho_min=cfg.rho_min, rho_max=cfg.rho_max,
                        check_termination_every=cfg.check_every, adapt_rho_every=cfg.adapt_rho_every,
                        adaptive_rho_tolerance=cfg.adaptive_rho_tolerance, rho_f_factor=cfg.rho_f_factor,
                        kernel_flags=_lib.flag_stream_p(P), diag_cost=True, const_g=const_g,
                        invariant_a=invariant_a)
    assert bool(solver._kernel_flags & _lib.FLAG_INVARIANT_A) == invariant_a
    st0 = zero_state(qp, 0.1)
    qpd = qp.to(DEV, dtype)
    state = ADMMState(**{k: torch.as_tensor(np.asarray(getattr(st0, k)), dtype=dtype, device=DEV) for k in FIELDS})
    (_, _), stats, out = solver.solve(qpd, state, alpha=cfg.alpha)
    torch.cuda.synchronize()
    return out, stats


def _cfg(max_iter=20, check=3, adapt=0):
    return oracle.OracleCfg(max_iter=max_iter, check_every=check, adapt_rho_every=adapt, sigma=1e-6, eps_abs=1e-12,
                            eps_rel=1e-12, rho_f_factor=1000.0, alpha=1.6)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("P", [1, 2])
@pytest.mark.parametrize("kind", ["quad", "lti", "varying", "one"])
# n = 17 records (nx + m = 17, 17), and n = 9 (outside the form: the flag is ignored)
@pytest.mark.parametrize("shape", [(8, 11, 17, 13, 4), (7, 9, 17, 12, 5), (8, 11, 9, 6, 3)])
def test_invariant_a_bit_equal_to_whole_records(shape, kind, P, dtype):
    B, T, n, nx, m = shape
    qp = _shared_g(_pattern(random_qp(B, T, n, nx, m, seed=61, std=True, diag=True), kind))
    cfg = _cfg()
    nvar = sum(bin(int(w)).count("1") for w in _varying_mask(qp.eq.A_minus))
    print(f"  {kind}: {nvar} of {nx * n} entries of A_minus vary", flush=True)
    outs, iters = [], []
    for const_g, inv in ((False, False), (True, False), (True, True)):
        out, stats = _solve(qp, cfg, dtype, P, const_g, inv)
        outs.append(out)
        iters.append(stats.num_iter)
    for o, it in zip(outs[:2], iters[:2]):
        assert torch.equal(it, iters[2])
        for k in FIELDS:
            assert torch.equal(getattr(o, k), getattr(outs[2], k)), k
    ref, it_ref, _ = oracle.admm_solve(qp, zero_state(qp, 0.1), cfg, dtype=np.float64)
    np.testing.assert_array_equal(iters[2].cpu().numpy(), it_ref)
    tol = 1e-9 if dtype == torch.float64 else 5e-4
    for k in FIELDS:
        r = np.asarray(getattr(ref, k))
        if r.size:
            assert rel_err(getattr(outs[2], k), r) < tol, (k, rel_err(getattr(outs[2], k), r))


@pytest.mark.parametrize("P", [1, 2])
def test_invariant_a_with_adaptive_rho_chunks(P):
    """Adaptive rho: the solve runs in chunks with a refactorization between
    them; only the first chunk writes the compressed runs, the later ones
    read them."""
    qp = _shared_g(_pattern(random_qp(6, 13, 17, 13, 4, seed=62, std=True, diag=True), "quad"))
    cfg = _cfg(max_iter=40, check=5, adapt=5)
    outs = [_solve(qp, cfg, torch.float64, P, True, inv) for inv in (False, True)]
    assert torch.equal(outs[0][1].num_iter, outs[1][1].num_iter)
    for k in FIELDS:
        assert torch.equal(getattr(outs[0][0], k), getattr(outs[1][0], k)), k
    assert not torch.all(outs[1][0].rho_bar == 0.1)  # rho moved: several chunks ran


@pytest.mark.parametrize("shape", [(5, 2, 17, 13, 4), (4, 7, 17, 14, 3)])
def test_invariant_a_edge_shapes(shape):
    """N = 1 (one stage record: every entry invariant, the mask pass is
    skipped) and nx n > 224 (outside the form: the flag is ignored)."""
    B, T, n, nx, m = shape
    qp = _shared_g(_pattern(random_qp(B, T, n, nx, m, seed=63, std=True, diag=True), "quad"))
    cfg = _cfg()
    outs = [_solve(qp, cfg, torch.float64, 2, True, inv)[0] for inv in (False, True)]
    for k in FIELDS:
        assert torch.equal(getattr(outs[0], k), getattr(outs[1], k)), k


def _c_abi_solve(qp, flags, full_workspace=True):
    """tmpc_admm_direct_f64 through the C ABI with the caller's workspace;
    returns the state and the workspace."""
    lib = _lib.load()
    B, T, n, nx, n0, m = qp.dims
    dims = _lib.Dims(B, T, n, nx, n0, m)
    cfg = cfg_struct(max_iter=12, check_every=4, adapt_rho_every=0, pcg_max_iter=0, use_slack=False, flags=flags,
                     sigma=1e-6, eps_abs=1e-30, eps_rel=1e-30, rho_min=1e-6, rho_max=1e6,
                     adaptive_rho_tolerance=5.0, rho_f_factor=1000.0, alpha=1.6, pcg_eps=0.0)
    cq, keep = qp_struct(qp, None)
    z = lambda *s: torch.zeros(s, dtype=qp.dtype, device=DEV)  # noqa: E731
    zg = torch.clamp(z(B, T, m), qp.ineq.l, qp.ineq.u).contiguous()
    outs = [z(B, T, n), zg, z(B, T, m), z(B, n0), z(B, T - 1, nx), z(B, T, m),
            torch.full((B,), 0.1, dtype=qp.dtype, device=DEV)]
    sv = state_struct(*outs)
    iters = torch.zeros(B, dtype=torch.int32, device=DEV)
    nbytes = lib.tmpc_admm_direct_workspace_bytes(8, ctypes.byref(dims))
    extra = -(-(T - 1) * (B + 1) * 256 * 8 // 256) * 256 + 256  # the AINV part: compressed runs, mask words
    size = nbytes if full_workspace else nbytes - extra
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=DEV)
    st = lib.tmpc_admm_direct_f64(_lib.stream_handle(torch.device(DEV)), ctypes.byref(dims), ctypes.byref(cq),
                                  ctypes.byref(sv), ctypes.byref(sv), _lib.ptr(iters), ctypes.byref(cfg),
                                  _lib.ptr(ws), size)
    _lib.check("tmpc_admm_direct_f64", st)
    torch.cuda.synchronize()
    del keep
    return outs, iters, ws, nbytes


@pytest.mark.parametrize("kind", ["quad", "one", "lti"])
def test_invariant_a_mask_read_back(kind):
    """The mask words (the last 256-byte block of the workspace) equal the host
    restatement, and a workspace without the form's room runs the resident-G
    form with the same result."""
    qp = _shared_g(_pattern(random_qp(9, 10, 17, 13, 4, seed=64, std=True, diag=True), kind)).to(DEV, torch.float64)
    flags = _lib.FLAG_STD_DYNAMICS | _lib.FLAG_DIAG_COST | _lib.FLAG_CONST_G | _lib.FLAG_INVARIANT_A
    outs, iters, ws, nbytes = _c_abi_solve(qp, flags)
    mask = ws[nbytes - 256: nbytes - 256 + 28].cpu().view(torch.int32).numpy().view(np.uint32)
    want = _varying_mask(qp.eq.A_minus)
    print(f"  {kind}: mask {[hex(int(w)) for w in mask]}", flush=True)
    np.testing.assert_array_equal(mask, want)
    outs2, iters2, ws2, _ = _c_abi_solve(qp, flags, full_workspace=False)
    assert torch.all(ws2[nbytes - 256: nbytes - 256 + 28] == 0)  # the form did not run
    assert torch.equal(iters, iters2)
    for a, b in zip(outs, outs2):
        assert torch.equal(a, b)


def test_quadrotor_sqp_invariant_a_default_and_bit_equal():
    """The benchmark's SQP solve (quadrotor, fp32): the solver turns the form
    on with the resident G rows, and the iterates equal those without it."""
    import copy

    from turbompc_amd.solvers.turbompc_solver import DEFAULT_SOLVER_PARAMS, TurboMPCSolver

    prob = make_quadrotor_config(B=300, seed=9, dtype=torch.float32, device=DEV)
    params = copy.deepcopy(DEFAULT_SOLVER_PARAMS)
    params["num_sqp_iteration_max"], params["tol_convergence"] = 3, 0.0
    params["admm"].update(max_iter=20, adapt_rho_every=0, relaxation_parameter=1.0)
    sols = []
    for inv in (True, False):
        solver = TurboMPCSolver(prob, params)
        assert solver._admm_solver_fwd._kernel_flags & _lib.FLAG_INVARIANT_A
        if not inv:
            solver._admm_solver_fwd._kernel_flags &= ~_lib.FLAG_INVARIANT_A
        sols.append(solver.solve(solver.initial_guess()))
    torch.cuda.synchronize()
    for k in ("states", "controls"):
        assert torch.equal(getattr(sols[0], k), getattr(sols[1], k)), k
    for k in sols[0].admm_state._fields:
        assert torch.equal(getattr(sols[0].admm_state, k), getattr(sols[1].admm_state, k)), k
