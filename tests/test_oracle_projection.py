"""Pins the oracle's EWA projection (projection.py:24-146) and its VJP.

Known answers from the reference's tests (test_splatting.py:57-72,
114-195), an explicit float64 matrix-form restatement, and torch float64
autograd for the gradient."""

import numpy as np
import pytest
import torch

from mlx3d_amd.cameras import Camera
from oracle import oracle as O
from refimpl import oracle_camera, project_matrix_f64


def _project(cam, means, quats, scales, **kw):
    return O.project(oracle_camera(cam), means, quats, scales, **kw)


def test_camera_look_at_closed_form():
    cam = Camera.look_at(eye=(0, 0, -4.0), width=256, height=256)
    np.testing.assert_array_equal(cam.R.numpy(), np.diag([-1.0, -1.0, 1.0]).astype(np.float32))
    np.testing.assert_array_equal(cam.t.numpy(), np.array([0, 0, 4.0], np.float32))
    assert abs(cam.fx - 256 / (2 * np.tan(np.radians(30)))) < 1e-9
    np.testing.assert_array_equal(cam.camera_center.numpy(), np.array([0, 0, -4.0], np.float32))


def test_projection_center_gaussian():
    # test_splatting.py:57-64
    cam = Camera.look_at(eye=(0, 0, -3.0), at=(0, 0, 0), width=64, height=64, fov=60.0)
    out = _project(cam, np.zeros((1, 3)), np.array([[1.0, 0, 0, 0]]), np.full((1, 3), 0.1))
    np.testing.assert_allclose(out["means2d"][0], [32.0, 32.0], atol=1e-3)
    assert abs(out["depths"][0] - 3.0) < 1e-5
    assert out["radii"][0] > 0
    # isotropic closed form: sigma_px = fx * s / z, conic = 1/(sigma^2 + 0.3)
    var = (cam.fx * 0.1 / 3.0) ** 2 + 0.3
    np.testing.assert_allclose(out["conics"][0], [1 / var, 0.0, 1 / var], rtol=1e-5, atol=1e-7)
    assert out["radii"][0] == np.ceil(3 * np.sqrt(var))


def test_projection_culls_behind_camera():
    # test_splatting.py:67-72
    cam = Camera.look_at(eye=(0, 0, -3.0), at=(0, 0, 0), width=64, height=64)
    out = _project(cam, np.array([[0.0, 0.0, -10.0]]), np.array([[1.0, 0, 0, 0]]),
                   np.full((1, 3), 0.1))
    assert out["radii"][0] == 0.0
    assert out["compensation"][0] == 0.0


def test_projection_matches_matrix_formula():
    # test_splatting.py:114-165 setup, float64 matrix restatement
    rng = np.random.default_rng(11)
    cam = Camera.look_at(eye=(0.3, -0.2, -3.0), at=(0, 0, 0), width=80, height=48, fov=55.0)
    means = (rng.standard_normal((256, 3)) * 0.4).astype(np.float32)
    quats = rng.standard_normal((256, 4)).astype(np.float32)
    scales = np.exp(rng.standard_normal((256, 3)) * 0.2 - 2.0).astype(np.float32)
    out = _project(cam, means, quats, scales)
    ref = project_matrix_f64(cam, torch.tensor(means, dtype=torch.float64),
                             torch.tensor(quats, dtype=torch.float64),
                             torch.tensor(scales, dtype=torch.float64))
    np.testing.assert_allclose(out["means2d"], ref["means2d"].numpy(), atol=1e-4)
    np.testing.assert_allclose(out["depths"], ref["depths"].numpy(), atol=1e-5)
    np.testing.assert_allclose(out["conics"], ref["conics"].numpy(), rtol=1e-4, atol=1e-6)
    # radii exact except where 3 sqrt(lam1) sits within float noise of an integer
    r64 = 3.0 * np.sqrt(np.maximum(ref["lam1"].numpy(), 0))
    safe = np.abs(r64 - np.round(r64)) > 1e-3
    np.testing.assert_array_equal(out["radii"][safe], ref["radii"].numpy()[safe])
    assert safe.mean() > 0.98
    np.testing.assert_array_equal(out["compensation"], np.ones(256, np.float32))


def test_projection_antialias_compensation_isotropic():
    # test_splatting.py:168-195
    cam = Camera.look_at(eye=(0, 0, -3.0), at=(0, 0, 0), width=64, height=64, fov=60.0)
    scales = np.array([[0.001] * 3, [0.1] * 3], np.float32)
    out = _project(cam, np.zeros((2, 3)), np.array([[1.0, 0, 0, 0]] * 2), scales,
                   antialias=True)
    var = (cam.fx * scales[:, 0] / 3.0) ** 2
    np.testing.assert_allclose(out["compensation"], var / (var + 0.3), atol=1e-5)
    assert out["compensation"][0] < out["compensation"][1] <= 1.0
    nb = _project(cam, np.zeros((1, 3)), np.array([[1.0, 0, 0, 0]]),
                  np.array([[0.001] * 3]), blur=0.0, antialias=True)
    assert nb["compensation"][0] == 1.0


@pytest.mark.parametrize("antialias", [False, True])
def test_projection_vjp_matches_autograd(antialias):
    rng = np.random.default_rng(5)
    cam = Camera.look_at(eye=(0.4, 0.3, -3.5), at=(0, 0, 0), width=96, height=80, fov=55.0)
    n = 200
    means = (rng.standard_normal((n, 3)) * 0.5).astype(np.float32)
    # a few far off-screen so the frustum clip is active
    means[:8, 0] = 6.0
    quats = rng.standard_normal((n, 4)).astype(np.float32)
    scales = np.exp(rng.standard_normal((n, 3)) * 0.4 - 2.2).astype(np.float32)
    g = {k: rng.standard_normal(s).astype(np.float32)
         for k, s in [("m2", (n, 2)), ("co", (n, 3)), ("z", (n,)), ("cp", (n,))]}
    gm, gq, gs = O.project_bwd(oracle_camera(cam), means, quats, scales, g["m2"], g["co"],
                               g["z"], g["cp"], antialias=antialias)
    tm, tq, ts = (torch.tensor(a, dtype=torch.float64, requires_grad=True)
                  for a in (means, quats, scales))
    r = project_matrix_f64(cam, tm, tq, ts, antialias=antialias)
    loss = ((r["means2d"] * torch.tensor(g["m2"], dtype=torch.float64)).sum()
            + (r["conics"] * torch.tensor(g["co"], dtype=torch.float64)).sum()
            + (r["depths"] * torch.tensor(g["z"], dtype=torch.float64)).sum()
            + (r["compensation"] * torch.tensor(g["cp"], dtype=torch.float64)).sum())
    loss.backward()
    for name, a, b in [("means", gm, tm.grad), ("quats", gq, tq.grad), ("scales", gs, ts.grad)]:
        b = b.numpy()
        err = np.abs(a - b).max() / (np.abs(b).max() + 1e-12)
        assert err < 1e-4, f"{name}: {err}"
