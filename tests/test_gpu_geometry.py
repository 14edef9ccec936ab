"""The 2DGS geometry kernels (gsx_geom_*) against a float64 torch
restatement of trainer.py:187-259 (tests/refimpl.py), values and gradients,
on a pinhole and a Brown-distorted camera."""

import numpy as np
import pytest
import torch

from gpu_util import cu, host, rel_err, say
from mlx3d_amd.cameras import Camera
from mlx3d_amd.splatting.geometry import geometry_loss, surfel_features
from refimpl import geometry_loss_f64, surfel_features_f64

pytestmark = pytest.mark.gpu


def test_surfel_features_and_vjp():
    rng = np.random.default_rng(0)
    n = 5000
    means = rng.normal(0, 1, (n, 3)).astype(np.float32)
    quats = rng.normal(0, 1, (n, 4)).astype(np.float32)
    depths = rng.uniform(1, 6, n).astype(np.float32)
    cam = Camera.look_at(eye=(0.3, -0.2, -4.0), width=64, height=48)
    tq, td = cu(quats).requires_grad_(True), cu(depths).requires_grad_(True)
    f = surfel_features(cu(means), tq, td, cam)
    q64 = torch.tensor(quats, dtype=torch.float64, requires_grad=True)
    d64 = torch.tensor(depths, dtype=torch.float64, requires_grad=True)
    center = cam.camera_center.numpy().astype(np.float64)
    ref = surfel_features_f64(torch.tensor(means, dtype=torch.float64), q64, d64, center)
    np.testing.assert_allclose(host(f), ref.detach().numpy(), rtol=2e-6, atol=2e-6)
    g = rng.normal(0, 1, (n, 5)).astype(np.float32)
    (f * cu(g)).sum().backward()
    (ref * torch.tensor(g, dtype=torch.float64)).sum().backward()
    for name, a, b in [("quats", tq.grad, q64.grad), ("depths", td.grad, d64.grad)]:
        e = rel_err(host(a), b.numpy())
        say(f"surfel features vjp {name}: rel {e:.2e}")
        assert e < 1e-4


def _render_like(rng, H, W):
    """A smooth positive depth field with a consistent second moment, noisy
    normals and an alpha map with holes."""
    yy, xx = np.mgrid[0:H, 0:W].astype(np.float64)
    ed = 3.0 + 0.3 * np.sin(xx / 7.0) + 0.2 * np.cos(yy / 5.0) + rng.normal(0, 0.01, (H, W))
    # the clamp max(E[z^2] - E[z]^2, 0) active on a fifth of the pixels, and
    # every difference far from 0, where float32 and float64 could disagree
    # on its sign
    ed2 = ed * ed + np.where(rng.random((H, W)) < 0.8,
                             0.01 + np.abs(rng.normal(0, 0.05, (H, W))), -0.05)
    nrm = rng.normal(0, 1, (H, W, 3)) + np.array([0.0, 0.0, -2.0])
    F = np.concatenate([ed[..., None], ed2[..., None], nrm], -1).astype(np.float32)
    alpha = rng.uniform(0, 1, (H, W)).astype(np.float32)
    return F, alpha


@pytest.mark.parametrize("lens", ["pinhole", "brown"])
def test_geometry_loss_matches_f64(lens):
    rng = np.random.default_rng(1)
    H, W = 40, 56
    cam = Camera.look_at(eye=(0.5, 0.2, -4.0), width=W, height=H)
    if lens == "brown":
        cam = Camera(R=cam.R, t=cam.t, fx=cam.fx, fy=cam.fy, cx=cam.cx, cy=cam.cy, width=W,
                     height=H, distortion=(0.05, -0.01, 0.001, 0.0005))
    F, alpha = _render_like(rng, H, W)
    tF = cu(F).requires_grad_(True)
    loss, metrics = geometry_loss(tF, cu(alpha), cam, 0.3, 0.7, 0.4)
    F64 = torch.tensor(F, dtype=torch.float64, requires_grad=True)
    rl, rdv, rnc = geometry_loss_f64(F64, torch.tensor(alpha, dtype=torch.float64), cam, 0.3,
                                     0.7, 0.4)
    say(f"{lens}: loss {float(loss):.7f} vs {float(rl):.7f}; dv {float(metrics['depth_variance']):.6f}"
        f" vs {float(rdv):.6f}; nc {float(metrics['normal_consistency']):.6f} vs {float(rnc):.6f}")
    np.testing.assert_allclose(float(loss), float(rl), rtol=2e-5)
    np.testing.assert_allclose(float(metrics["depth_variance"]), float(rdv), rtol=2e-5)
    np.testing.assert_allclose(float(metrics["normal_consistency"]), float(rnc), rtol=2e-5)
    g = float(rng.normal())
    (loss * g).backward()
    (rl * g).backward()
    e = rel_err(host(tF.grad), F64.grad.numpy())
    say(f"{lens}: dL/dF rel {e:.2e}")
    assert e < 1e-3


def test_geometry_loss_terms_switch_off():
    rng = np.random.default_rng(2)
    H, W = 24, 32
    cam = Camera.look_at(eye=(0.0, 0.0, -4.0), width=W, height=H)
    F, alpha = _render_like(rng, H, W)
    tF = cu(F).requires_grad_(True)
    loss, m = geometry_loss(tF, cu(alpha), cam, 0.3, 0.5, 0.0)
    np.testing.assert_allclose(float(loss), 0.5 * float(m["depth_variance"]), rtol=1e-6)
    assert float(m["normal_consistency"]) == 0.0
    loss.backward()
    assert float(tF.grad[..., 2:].abs().max()) == 0.0  # normals only feed the normal term
    # nothing passes the alpha test: zero loss, zero gradient
    tF.grad = None
    loss, m = geometry_loss(tF, cu(np.zeros((H, W), np.float32)), cam, 0.3, 0.5, 0.5)
    loss.backward()
    assert float(loss) == 0.0 and float(tF.grad.abs().max()) == 0.0
