"""Pins the oracle's eval_sh (sh.py:41-78): the basis functions against
scipy's spherical harmonics (per-function sign convention), the reference's
known answers (sh.py round trip, degree-0 identity) and the VJP against
float64 finite differences."""

import numpy as np
import pytest

from oracle import oracle as O
from refimpl import sh_basis_scipy

C0 = 0.28209479177387814


def _unit_dirs(n, seed):
    d = np.random.default_rng(seed).standard_normal((n, 3))
    return (d / np.linalg.norm(d, axis=1, keepdims=True)).astype(np.float32)


def _basis_from_oracle(degree, dirs):
    n = dirs.shape[0]
    K = (degree + 1) ** 2
    cols = []
    for k in range(K):
        sh = np.zeros((n, K, 1), np.float32)
        sh[:, k, 0] = 1.0
        cols.append(O.eval_sh(degree, sh, dirs)[:, 0] - 0.5)
    return np.stack(cols, -1)


def test_basis_matches_scipy_up_to_sign():
    dirs = _unit_dirs(500, 1)
    ours = _basis_from_oracle(3, dirs).astype(np.float64)
    ref = sh_basis_scipy(3, dirs)
    for k in range(16):
        ratio = ours[:, k] / ref[:, k]
        ok = np.abs(ref[:, k]) > 1e-3
        s = np.sign(np.median(ratio[ok]))
        np.testing.assert_allclose(ours[:, k], s * ref[:, k], atol=2e-6, err_msg=f"basis {k}")


def test_degree0_is_color_and_roundtrip():
    # test_splatting.py:43-54
    rng = np.random.default_rng(2)
    rgb = rng.uniform(size=(64, 3)).astype(np.float32)
    sh = ((rgb - np.float32(0.5)) / np.float32(C0))[:, None, :].astype(np.float32)
    out = O.eval_sh(0, sh, _unit_dirs(64, 3))
    np.testing.assert_allclose(out, rgb, atol=1e-6)


@pytest.mark.parametrize("degree", [0, 1, 2, 3])
def test_eval_sh_vjp(degree):
    rng = np.random.default_rng(4 + degree)
    n, K, C = 40, 16, 3
    sh = (rng.standard_normal((n, K, C)) * 0.3).astype(np.float32)
    dirs = _unit_dirs(n, 7)
    g = rng.standard_normal((n, C)).astype(np.float32)
    g_sh, g_dirs = O.eval_sh_bwd(degree, sh, dirs, g)
    # coefficient gradient = basis value * g (linear); zero beyond the degree
    B = _basis_from_oracle(degree, dirs)
    Ka = (degree + 1) ** 2
    np.testing.assert_allclose(g_sh[:, :Ka, :], B[:, :, None] * g[:, None, :], rtol=1e-6, atol=1e-7)
    assert np.all(g_sh[:, Ka:, :] == 0)
    # direction gradient vs central differences of the scipy-built basis
    eps = 1e-6
    fd = np.zeros((n, 3))
    for a in range(3):
        dp = dirs.astype(np.float64).copy(); dp[:, a] += eps
        dm = dirs.astype(np.float64).copy(); dm[:, a] -= eps
        # the polynomial form differentiates off the unit sphere, as the
        # kernel's VJP does (dirs enter eval_sh unnormalised)
        fp = _poly_basis(degree, dp)
        fm = _poly_basis(degree, dm)
        df = (fp - fm) / (2 * eps)  # (n, Ka)
        fd[:, a] = np.einsum("nk,nkc,nc->n", df, sh[:, :Ka, :].astype(np.float64), g)
    np.testing.assert_allclose(g_dirs, fd, rtol=1e-3, atol=2e-4)


def _poly_basis(degree, d):
    """Polynomial form of the 3DGS basis (sh.py:57-77) in float64."""
    x, y, z = d[:, 0], d[:, 1], d[:, 2]
    C1 = 0.4886025119029199
    C2 = [1.0925484305920792, -1.0925484305920792, 0.31539156525252005, -1.0925484305920792,
          0.5462742152960396]
    C3 = [-0.5900435899266435, 2.890611442640554, -0.4570457994644658, 0.3731763325901154,
          -0.4570457994644658, 1.445305721320277, -0.5900435899266435]
    cols = [np.full_like(x, C0)]
    if degree > 0:
        cols += [-C1 * y, C1 * z, -C1 * x]
    if degree > 1:
        xx, yy, zz = x * x, y * y, z * z
        cols += [C2[0] * x * y, C2[1] * y * z, C2[2] * (2 * zz - xx - yy), C2[3] * x * z,
                 C2[4] * (xx - yy)]
    if degree > 2:
        cols += [C3[0] * y * (3 * xx - yy), C3[1] * x * y * z, C3[2] * y * (4 * zz - xx - yy),
                 C3[3] * z * (2 * zz - 3 * xx - 3 * yy), C3[4] * x * (4 * zz - xx - yy),
                 C3[5] * z * (xx - yy), C3[6] * x * (xx - 3 * yy)]
    return np.stack(cols, -1)


def test_poly_basis_is_scipy_basis():
    # ties the finite-difference helper above to scipy as well
    dirs = _unit_dirs(300, 9)
    P = _poly_basis(3, dirs.astype(np.float64))
    S = sh_basis_scipy(3, dirs)
    s = np.sign(np.sum(P * S, 0))
    # float32 unit vectors are unit only to ~1e-7; the polynomial form sees that
    np.testing.assert_allclose(P, S * s, atol=1e-6)
