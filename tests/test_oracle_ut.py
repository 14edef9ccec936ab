"""Pins the UT-projection oracle (oracle/ut_oracle.c).

* orc_atanf against numpy's float64 arctan (error bound) and special values.
* Forward values against a float64 restatement of project_gaussians_ut and
  Camera.project_points (tests/refimpl.py) on pinhole, Brown-Conrady (4 and
  5 coefficients), fisheye and orthographic cameras.
* The VJP against float64 torch autograd through that restatement.
* The reference's own UT tests (test_splatting.py:75-111) re-expressed.
* A closed form: through an orthographic (linear) camera the six sigma
  points reproduce the covariance exactly, fx^2 (R Rq S)(R Rq S)^T.
* The fused preprocess under ORC_PROJECT_UT equals orc_project_ut.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from mlx3d_amd.cameras import Camera
from oracle import oracle as O
from refimpl import lens_cameras, oracle_camera, project_ut_f64, quat_to_rot_f64


def test_atanf_error_bound_and_specials():
    r = np.concatenate([np.linspace(0, 2, 20001), np.geomspace(1e-8, 1e8, 20001),
                        np.linspace(2, 50, 20001),
                        [0.41421356, 0.41421357, 1.0, 0.99999994, 1.0000001]]).astype(np.float32)
    got = O.atanf(r).astype(np.float64)
    ref = np.arctan(r.astype(np.float64))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    err = np.abs(got - ref) / ulp
    assert err.max() <= 2.5 and err.mean() < 0.5
    assert O.atanf(np.float32(0.0)) == 0.0
    assert abs(float(O.atanf(np.float32(1e30))) - np.pi / 2) < 1e-7
    # monotone
    s = np.sort(r)
    assert (np.diff(O.atanf(s).astype(np.float64)) >= 0).all()


def _scene(n=400, seed=0, spread=0.8, log_s=-3.0):
    rng = np.random.default_rng(seed)
    means = (rng.standard_normal((n, 3)) * spread).astype(np.float32)
    quats = rng.standard_normal((n, 4)).astype(np.float32)
    scales = np.exp(rng.standard_normal((n, 3)) * 0.4 + log_s).astype(np.float32)
    return means, quats, scales


def _f64(*a):
    return [torch.tensor(x, dtype=torch.float64) for x in a]


# fixed per-camera scene seeds (str hash() changes from process to process)
_SEEDS = {"pinhole": 11, "brown4": 12, "brown5": 13, "fisheye": 14, "ortho": 15}


@pytest.mark.parametrize("name", ["pinhole", "brown4", "brown5", "fisheye", "ortho"])
@pytest.mark.parametrize("antialias", [False, True])
def test_ut_forward_matches_f64(name, antialias):
    cam = lens_cameras()[name]
    means, quats, scales = _scene(seed=_SEEDS[name])
    out = O.project_ut(oracle_camera(cam), means, quats, scales, antialias=antialias)
    ref = project_ut_f64(cam, *_f64(means, quats, scales), antialias=antialias)
    valid = ref["radii"].numpy() > 0
    assert valid.sum() > 100
    np.testing.assert_allclose(out["means2d"], ref["means2d"].numpy(), rtol=1e-5, atol=2e-4)
    np.testing.assert_allclose(out["depths"], ref["depths"].numpy(), rtol=1e-6, atol=1e-6)
    c_ref = ref["conics"].numpy()[valid]
    err = np.abs(out["conics"][valid] - c_ref).max(axis=1) / np.abs(c_ref).max(axis=1)
    assert err.max() < 1e-3, err.max()
    np.testing.assert_allclose(out["compensation"][valid], ref["compensation"].numpy()[valid],
                               rtol=1e-3, atol=1e-5)
    # radii are ceil() of a float: equal except within rounding of an integer
    lam = ref["lam1"].numpy()
    near = np.abs(3 * np.sqrt(np.maximum(lam, 0)) - np.round(3 * np.sqrt(np.maximum(lam, 0))))
    ok = (out["radii"] == ref["radii"].numpy()) | (near < 1e-3)
    assert ok.all()


@pytest.mark.parametrize("name", ["pinhole", "brown4", "brown5", "fisheye", "ortho"])
def test_ut_vjp_matches_autograd(name):
    cam = lens_cameras()[name]
    means, quats, scales = _scene(n=300, seed=7 + len(name))
    rng = np.random.default_rng(3)
    gm2 = rng.standard_normal((300, 2)).astype(np.float32)
    gco = rng.standard_normal((300, 3)).astype(np.float32) * 1e-3
    gd = rng.standard_normal(300).astype(np.float32)
    gc = rng.standard_normal(300).astype(np.float32)
    m, q, s = _f64(means, quats, scales)
    for t in (m, q, s):
        t.requires_grad_(True)
    ref = project_ut_f64(cam, m, q, s, antialias=True)
    valid = ref["radii"] > 0
    loss = ((ref["means2d"] * torch.tensor(gm2, dtype=torch.float64)).sum()
            + (ref["conics"][valid] * torch.tensor(gco, dtype=torch.float64)[valid]).sum()
            + (ref["depths"] * torch.tensor(gd, dtype=torch.float64)).sum()
            + (ref["compensation"] * torch.tensor(gc, dtype=torch.float64)).sum())
    loss.backward()
    gco_masked = np.where(valid.numpy()[:, None], gco, 0.0).astype(np.float32)
    g = O.project_bwd(oracle_camera(cam), means, quats, scales, gm2, gco_masked, gd, gc,
                      antialias=True, ut=True)
    for name_, a, b in zip(("means", "quats", "scales"), g, (m.grad, q.grad, s.grad)):
        b = b.numpy()
        e = np.abs(a - b).max() / np.abs(b).max()
        assert e < 2e-4, (name_, e)


def test_ut_respects_camera_distortion():
    """test_splatting.py:75-98: the UT mean follows the distorted centre, the
    EWA mean (pinhole) does not."""
    base = Camera.look_at(eye=(0, 0, -3.0), at=(0, 0, 0), fov=60.0, width=128, height=128)
    cam = Camera(R=base.R, t=base.t, fx=base.fx, fy=base.fy, cx=base.cx, cy=base.cy,
                 width=128, height=128, distortion=(-0.35, 0.12, 0.002, -0.001))
    means = np.array([[0.75, 0.45, 0.0]], np.float32)
    quats = np.array([[1.0, 0, 0, 0]], np.float32)
    scales = np.full((1, 3), 1e-4, np.float32)
    ut = O.project_ut(oracle_camera(cam), means, quats, scales)
    ewa = O.project(oracle_camera(cam), means, quats, scales)
    centre = cam.project_points(torch.tensor(means))[0].numpy()
    np.testing.assert_allclose(ut["means2d"], centre, atol=1e-3)
    assert np.abs(ewa["means2d"] - centre).max() > 0.25
    assert ut["radii"][0] > 0


def test_ut_close_to_ewa_for_pinhole_small_gaussians():
    """test_splatting.py:101-111."""
    cam = Camera.look_at(eye=(0, 0, -3.0), at=(0, 0, 0), fov=55.0, width=96, height=64)
    means = np.array([[0.0, 0.0, 0.0], [0.2, -0.1, 0.3]], np.float32)
    quats = np.array([[1.0, 0.0, 0.0, 0.0], [0.9, 0.1, 0.2, 0.3]], np.float32)
    scales = np.full((2, 3), 1e-3, np.float32)
    ewa = O.project(oracle_camera(cam), means, quats, scales)
    ut = O.project_ut(oracle_camera(cam), means, quats, scales)
    np.testing.assert_allclose(ut["means2d"], ewa["means2d"], atol=1e-3)
    np.testing.assert_allclose(ut["conics"], ewa["conics"], rtol=0.05)


def test_ut_orthographic_closed_form():
    """A linear camera: the sigma-point covariance is exactly the projected
    covariance fx^2 (R Rq S)(R Rq S)^T (rows x, y), the mean the projected
    centre."""
    cam = lens_cameras()["ortho"]
    means, quats, scales = _scene(n=200, seed=11, log_s=-2.0)
    out = O.project_ut(oracle_camera(cam), means, quats, scales, blur=0.0)
    R = torch.tensor(cam.R.numpy(), dtype=torch.float64)
    m, q, s = _f64(means, quats, scales)
    M = R @ (quat_to_rot_f64(q) * s[:, None, :])
    cov = M @ M.transpose(1, 2)
    fx = cam.fx
    a0, b, c0 = fx * fx * cov[:, 0, 0], fx * fx * cov[:, 0, 1], fx * fx * cov[:, 1, 1]
    det = a0 * c0 - b * b
    conic = torch.stack([c0 / det, -b / det, a0 / det], -1).numpy()
    err = np.abs(out["conics"] - conic).max(axis=1) / np.abs(conic).max(axis=1)
    assert err.max() < 1e-4
    pc = m @ R.T + torch.tensor(cam.t.numpy(), dtype=torch.float64)
    centre = torch.stack([fx * pc[:, 0] + cam.cx, fx * pc[:, 1] + cam.cy], -1).numpy()
    np.testing.assert_allclose(out["means2d"], centre, rtol=1e-6, atol=1e-4)


def test_preprocess_ut_flag_matches_project_ut():
    cam = lens_cameras()["brown5"]
    means, quats, scales = _scene(n=300, seed=5)
    opac = np.full(300, 0.7, np.float32)
    pre = O.preprocess_fwd(oracle_camera(cam), means, quats, scales, opac,
                           flags=O.PROJECT_UT | O.ANTIALIAS, threads=1)
    ut = O.project_ut(oracle_camera(cam), means, quats, scales, antialias=True)
    for k_pre, k_ut in (("means2d", "means2d"), ("conics", "conics"), ("depths", "depths"),
                        ("radii", "radii"), ("compensation", "compensation")):
        np.testing.assert_array_equal(pre[k_pre], ut[k_ut], err_msg=k_pre)
    # and the EWA oracle differs (distortion is not in the EWA model)
    ewa = O.project(oracle_camera(cam), means, quats, scales, antialias=True)
    assert np.abs(ewa["means2d"] - ut["means2d"]).max() > 0.1
