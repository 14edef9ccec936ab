"""The tile renderer against the dense reference path
(render_gaussians_reference, reference.py:16-74) on the device, as the
reference's own tests compare them (test_splatting.py:214-241, 243-277,
340-362, 390-413): images and alpha within 1e-3, gradients within 1e-3 (2e-3
for features) of the largest reference gradient."""

import numpy as np
import pytest
import torch

from gpu_util import cu, host, say
from mlx3d_amd.cameras import Camera
from mlx3d_amd.splatting import (render_gaussian_features, render_gaussians,
                                 render_gaussians_reference)
from refimpl import random_scene

pytestmark = pytest.mark.gpu

BG = np.array([0.1, 0.2, 0.3], np.float32)


def _scene():
    return random_scene(0, n=300, width=96, height=64)


def _max_abs(a, b):
    return float((a.detach() - b.detach()).abs().max())


@pytest.mark.parametrize("refine", [False, True])
def test_tile_matches_dense_forward(refine):
    cam, means, quats, scales, opac, colors = _scene()
    args = [cu(a) for a in (means, quats, scales, opac, colors)]
    with torch.no_grad():
        k = render_gaussians(cam, *args[:4], colors=args[4], background=cu(BG),
                             refine_tiles=refine)
        r = render_gaussians_reference(cam, *args, background=cu(BG))
    for key in ("image", "alpha"):
        e = _max_abs(k[key], r[key])
        say(f"dense vs tile refine={refine} {key}: max abs {e:.2e}")
        assert e <= 1e-3


def test_antialiased_matches_dense_and_reduces_alpha():
    cam, means, quats, scales, opac, colors = _scene()
    args = [cu(a) for a in (means, quats, scales, opac * np.float32(0.1), colors)]
    with torch.no_grad():
        plain = render_gaussians(cam, *args[:4], colors=args[4], background=cu(BG))
        k = render_gaussians(cam, *args[:4], colors=args[4], background=cu(BG), antialias=True)
        r = render_gaussians_reference(cam, *args, background=cu(BG), antialias=True)
    assert _max_abs(k["image"], r["image"]) <= 1e-3
    assert _max_abs(k["alpha"], r["alpha"]) <= 1e-3
    assert float((k["alpha"] - plain["alpha"]).max()) <= 1e-6
    comp = host(k["compensation"])
    assert (comp >= 0).all() and (comp <= 1).all() and (comp < 1).any()


def _grads(fn, leaves):
    leaves = [t.detach().clone().requires_grad_(True) for t in leaves]
    fn(*leaves).backward()
    return [host(t.grad) for t in leaves]


def test_tile_gradients_match_dense():
    cam, means, quats, scales, opac, colors = _scene()
    target = cu(np.random.default_rng(7).uniform(size=(cam.height, cam.width, 3))
                .astype(np.float32))
    bg = torch.zeros(3, device="cuda")
    leaves = [cu(a) for a in (means, quats, scales, opac, colors)]

    def kernel_loss(m, q, s, o, c):
        out = render_gaussians(cam, m, q, s, o, colors=c, background=bg)
        return ((out["image"] - target) ** 2).mean() + 0.05 * out["alpha"].mean()

    def dense_loss(m, q, s, o, c):
        out = render_gaussians_reference(cam, m, q, s, o, c, background=bg)
        return ((out["image"] - target) ** 2).mean() + 0.05 * out["alpha"].mean()

    gk, gr = _grads(kernel_loss, leaves), _grads(dense_loss, leaves)
    for name, a, b in zip(["means", "quats", "scales", "opac", "colors"], gk, gr):
        e = float(np.abs(a - b).max() / (np.abs(b).max() + 1e-12))
        say(f"dense vs tile grad {name}: {e:.2e}")
        assert e < 1e-3, name


def test_feature_gradients_match_dense():
    rng = np.random.default_rng(16)
    n = 40
    cam = Camera.look_at(eye=(0, 0, -3.0), at=(0, 0, 0), width=32, height=24, fov=55.0)
    means = (rng.standard_normal((n, 3)) * 0.35).astype(np.float32)
    quats = rng.standard_normal((n, 4)).astype(np.float32)
    scales = np.exp(rng.standard_normal((n, 3)) * 0.2 - 2.4).astype(np.float32)
    opac = (1 / (1 + np.exp(-rng.standard_normal(n)))).astype(np.float32)
    feats = (rng.standard_normal((n, 5)) * 0.25).astype(np.float32)
    target = cu((rng.standard_normal((cam.height, cam.width, 5)) * 0.1).astype(np.float32))
    bg = cu(np.linspace(0.0, 0.4, 5).astype(np.float32))
    leaves = [cu(a) for a in (means, quats, scales, opac, feats)]

    def kernel_loss(m, q, s, o, f):
        out = render_gaussian_features(cam, m, q, s, o, f, background=bg)
        return ((out["features"] - target) ** 2).mean() + 0.03 * out["alpha"].mean()

    def dense_loss(m, q, s, o, f):
        out = render_gaussians_reference(cam, m, q, s, o, f, background=bg)
        return ((out["image"] - target) ** 2).mean() + 0.03 * out["alpha"].mean()

    gk, gr = _grads(kernel_loss, leaves), _grads(dense_loss, leaves)
    for name, a, b in zip(["means", "quats", "scales", "opac", "features"], gk, gr):
        e = float(np.abs(a - b).max() / (np.abs(b).max() + 1e-12))
        say(f"dense vs tile feature grad {name}: {e:.2e}")
        assert e < 2e-3, name
