"""Pins the CPU restatement of the obstacle rows (oracle/sqp_cpu.py) without
the reference: the gradient against central differences of g, known answers
on and beyond the sphere, exactness of the linearization at its own point, and
the Hessian against differences of the gradient and its null direction d."""
import numpy as np

from oracle.sqp_cpu import OBSTACLE_LOWER, linearize_obstacles, obstacle_hessian, obstacle_values


def _g(states, centers, radii, dim):
    """g_k = 1 - |p - c_k| / (r_k + 0.001), straight from the constraint's definition."""
    d = states[..., None, :dim] - centers[:, None]
    return 1.0 - np.linalg.norm(d, axis=-1) / (radii[:, None] + 0.001)


def _case(seed=0, B=3, T=4, nx=6, K=5, dim=3):
    rng = np.random.default_rng(seed)
    return rng.uniform(-4, 4, (B, T, nx)), rng.uniform(-3, 3, (B, K, dim)), rng.uniform(0.3, 0.8, (B, K))


def test_gradient_matches_central_differences():
    s, c, r = _case()
    grad, _, _ = linearize_obstacles(s, c, r, 3)
    h = 1e-6
    for i in range(3):
        e = np.zeros(s.shape[-1])
        e[i] = h
        fd = (_g(s + e, c, r, 3) - _g(s - e, c, r, 3)) / (2 * h)
        np.testing.assert_allclose(grad[..., i], fd, rtol=1e-7, atol=1e-9)


def test_known_answers_on_the_sphere():
    # p on the sphere of radius r + 0.001 along +y: g = 0, gradient -e_y / (r + 0.001);
    # twice as far: g = -1
    c = np.array([[[0.5, -1.0, 2.0]]])
    r = np.array([[0.4]])
    s = np.zeros((1, 2, 6))
    s[0, 0, :3] = c[0, 0] + np.array([0.0, 0.401, 0.0])
    s[0, 1, :3] = c[0, 0] + np.array([0.0, 0.0, -0.802])
    grad, lo, up = linearize_obstacles(s, c, r, 3)
    g = _g(s, c, r, 3)
    np.testing.assert_allclose(g[0, :, 0], [0.0, -1.0], atol=1e-12)
    np.testing.assert_allclose(obstacle_values(s, c, r, 3)[0, :, 0], [0.0, -1.0], atol=1e-12)
    # the centre: g = 1
    s0 = np.zeros((1, 1, 6))
    s0[0, 0, :3] = c[0, 0]
    np.testing.assert_allclose(obstacle_values(s0, c, r, 3), 1.0, rtol=0, atol=0)
    np.testing.assert_allclose(grad[0, 0, 0], [0.0, -1.0 / 0.401, 0.0], atol=1e-12)
    np.testing.assert_allclose(grad[0, 1, 0], [0.0, 0.0, 1.0 / 0.401], atol=1e-12)


def test_linearization_is_exact_at_its_point_and_bounds_are_shifted():
    s, c, r = _case(1)
    grad, lo, up = linearize_obstacles(s, c, r, 3)
    g = _g(s, c, r, 3)
    gz = np.einsum("btkd,btd->btk", grad, s[..., :3])
    # g_lin(z) = grad z + offset <= 0  <=>  grad z <= u = -offset; at z = xbar it equals g(xbar)
    np.testing.assert_allclose(gz - up, g, atol=1e-12)
    np.testing.assert_allclose(lo - up, OBSTACLE_LOWER, rtol=1e-15)
    # a first-order step: g(xbar + dz) - g_lin(xbar + dz) = O(|dz|^2)
    dz = np.zeros_like(s)
    dz[..., :3] = 1e-4
    lin = np.einsum("btkd,btd->btk", grad, (s + dz)[..., :3]) - up
    assert np.max(np.abs(_g(s + dz, c, r, 3) - lin)) < 1e-6


def test_hessian_matches_gradient_differences_and_annihilates_d():
    s, c, r = _case(2, K=4)
    B, T, nx = s.shape
    n = nx + 3
    mus = np.random.default_rng(5).standard_normal((B, T, 4))
    H = obstacle_hessian(s, c, r, 3, mus, n)
    h = 1e-6
    for i in range(3):
        e = np.zeros(nx)
        e[i] = h
        gp, _, _ = linearize_obstacles(s + e, c, r, 3)
        gm, _, _ = linearize_obstacles(s - e, c, r, 3)
        col = np.einsum("btk,btkd->btd", mus, (gp - gm) / (2 * h))
        np.testing.assert_allclose(H[..., :3, i], col, rtol=1e-6, atol=1e-8)
    assert np.all(H[..., 3:, :] == 0) and np.all(H[..., :, 3:] == 0)
    # each obstacle's Hessian is symmetric, has d = p - c in its null space and
    # trace -(dim - 1) / (|d| (r + 0.001))
    one = np.zeros((B, T, 4))
    one[..., 0] = 1.0
    H0 = obstacle_hessian(s, c, r, 3, one, n)[..., :3, :3]
    d = s[..., :3] - c[:, None, 0]
    np.testing.assert_allclose(H0, np.swapaxes(H0, -1, -2), atol=1e-14)
    np.testing.assert_allclose(np.einsum("btij,btj->bti", H0, d), 0.0, atol=1e-12)
    tr = -2.0 / (np.linalg.norm(d, axis=-1) * (r[:, None, 0] + 0.001))
    np.testing.assert_allclose(np.trace(H0, axis1=-2, axis2=-1), tr, rtol=1e-12)
