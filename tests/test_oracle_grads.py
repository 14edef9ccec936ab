"""Pins the oracle's backward (rasterize.py:100-221 + the VJP of the
projection/SH/activations that MLX autodiff computes) against torch float64
autograd of an independent dense render, with the reference's criterion
max|d| / max|ref| < 1e-3 (test_splatting.py:340-414).  Opacities stay below
0.99 so the forward clamp is inactive (the kernel passes gradient through
it, autograd would not)."""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from refimpl import depth_order, oracle_camera, random_scene, render_f64, tile_mask


def _oracle_grads(cam, means, quats, scales, opac, feats=None, sh=None, degree=0, bg=None,
                  flags=0, g_img=None, g_alpha=None):
    oc = oracle_camera(cam)
    pre = O.preprocess_fwd(oc, means, quats, scales, opac, sh=sh, degree=degree, flags=flags)
    cols = pre["colors"] if sh is not None else feats
    ids, ranges, _, _ = O.bin_gaussians(pre["means2d"], pre["radii"], pre["depths"], cam.width,
                                        cam.height)
    r = O.raster_fwd(pre["means2d"], pre["conics"], pre["opac_eff"], cols, ids, ranges,
                     cam.width, cam.height, bg=bg)
    gr = O.raster_bwd(pre["means2d"], pre["conics"], pre["opac_eff"], cols, ids, ranges,
                      cam.width, cam.height, r["final_T"], r["n_contrib"], g_img,
                      grad_final_T=-g_alpha, bg=bg)
    K = 0 if sh is None else sh.shape[1]
    g = O.preprocess_bwd(oc, means, quats, scales, opac, pre["colors"] if sh is not None else None,
                         K, degree, flags, gr["means2d"], gr["conics"], gr["opacities"],
                         gr["features"] if sh is not None else None)
    if sh is None:
        g["colors"] = gr["features"]
    return g, pre, r


def _check(name, a, b, tol=1e-3):
    b = b.detach().numpy()
    err = np.abs(a - b).max() / (np.abs(b).max() + 1e-12)
    assert err < tol, f"gradient mismatch for {name}: {err}"


@pytest.mark.parametrize("antialias", [False, True])
def test_colors_mode_gradients(antialias):
    cam, means, quats, scales, opac, colors = random_scene(0)
    opac = np.minimum(opac, 0.9).astype(np.float32)
    rng = np.random.default_rng(10)
    g_img = rng.standard_normal((cam.height, cam.width, 3)).astype(np.float32)
    g_alpha = rng.standard_normal((cam.height, cam.width)).astype(np.float32)
    bg = np.array([0.1, 0.2, 0.3], np.float32)
    flags = O.ANTIALIAS if antialias else 0
    g, pre, r = _oracle_grads(cam, means, quats, scales, opac, feats=colors, bg=bg, flags=flags,
                              g_img=g_img, g_alpha=g_alpha)
    t = {k: torch.tensor(v, dtype=torch.float64, requires_grad=True)
         for k, v in dict(means=means, quats=quats, scales=scales, opac=opac, colors=colors).items()}
    mask = tile_mask(pre["means2d"], pre["radii"], cam.width, cam.height)
    img, T, _ = render_f64(cam, t["means"], t["quats"], t["scales"], t["opac"], colors=t["colors"],
                           bg=torch.tensor(bg, dtype=torch.float64), antialias=antialias,
                           mask=mask, order=depth_order(pre["depths"]))
    np.testing.assert_allclose(r["image"], img.detach().numpy(), atol=1e-5)
    loss = (img * torch.tensor(g_img, dtype=torch.float64)).sum() + \
        ((1 - T) * torch.tensor(g_alpha, dtype=torch.float64)).sum()
    loss.backward()
    _check("means", g["means"], t["means"].grad)
    _check("quats", g["quats"], t["quats"].grad)
    _check("scales", g["scales"], t["scales"].grad)
    _check("opacities", g["opacities"], t["opac"].grad)
    _check("colors", g["colors"], t["colors"].grad)


@pytest.mark.parametrize("degree", [0, 3])
def test_sh_raw_param_gradients(degree):
    """GaussianModel path: log-scales, logit opacities, SH colour."""
    cam, means, quats, scales, opac, _ = random_scene(3)
    rng = np.random.default_rng(20 + degree)
    n = means.shape[0]
    sh = (rng.standard_normal((n, 16, 3)) * 0.2).astype(np.float32)
    sh[:, 0, :] = rng.uniform(-0.5, 1.5, (n, 3))
    log_s = np.log(scales).astype(np.float32)
    logit = np.clip(rng.standard_normal(n), -3, 2.0).astype(np.float32)
    g_img = rng.standard_normal((cam.height, cam.width, 3)).astype(np.float32)
    g_alpha = rng.standard_normal((cam.height, cam.width)).astype(np.float32)
    flags = O.LOG_SCALES | O.LOGIT_OPACITY
    g, pre, r = _oracle_grads(cam, means, quats, log_s, logit, sh=sh, degree=degree, flags=flags,
                              g_img=g_img, g_alpha=g_alpha)
    t = {k: torch.tensor(v, dtype=torch.float64, requires_grad=True)
         for k, v in dict(means=means, quats=quats, ls=log_s, lo=logit, sh=sh).items()}
    mask = tile_mask(pre["means2d"], pre["radii"], cam.width, cam.height)
    img, T, _ = render_f64(cam, t["means"], t["quats"], torch.exp(t["ls"]), torch.sigmoid(t["lo"]),
                           sh=t["sh"], degree=degree, mask=mask, order=depth_order(pre["depths"]))
    np.testing.assert_allclose(r["image"], img.detach().numpy(), atol=2e-5)
    loss = (img * torch.tensor(g_img, dtype=torch.float64)).sum() + \
        ((1 - T) * torch.tensor(g_alpha, dtype=torch.float64)).sum()
    loss.backward()
    _check("means", g["means"], t["means"].grad)
    _check("quats", g["quats"], t["quats"].grad)
    _check("log_scales", g["scales"], t["ls"].grad)
    _check("logit_opacities", g["opacities"], t["lo"].grad)
    _check("sh", g["sh"], t["sh"].grad)


def test_feature_gradients_many_channels():
    cam, means, quats, scales, opac, _ = random_scene(4, n=200, width=48, height=32)
    opac = np.minimum(opac, 0.9).astype(np.float32)
    rng = np.random.default_rng(30)
    feats = rng.standard_normal((200, 37)).astype(np.float32)
    g_img = rng.standard_normal((32, 48, 37)).astype(np.float32)
    g_alpha = rng.standard_normal((32, 48)).astype(np.float32)
    g, pre, r = _oracle_grads(cam, means, quats, scales, opac, feats=feats, g_img=g_img,
                              g_alpha=g_alpha)
    t = {k: torch.tensor(v, dtype=torch.float64, requires_grad=True)
         for k, v in dict(means=means, quats=quats, scales=scales, opac=opac, f=feats).items()}
    mask = tile_mask(pre["means2d"], pre["radii"], cam.width, cam.height)
    img, T, _ = render_f64(cam, t["means"], t["quats"], t["scales"], t["opac"], colors=t["f"],
                           mask=mask, order=depth_order(pre["depths"]))
    loss = (img * torch.tensor(g_img, dtype=torch.float64)).sum() + \
        ((1 - T) * torch.tensor(g_alpha, dtype=torch.float64)).sum()
    loss.backward()
    for name, key in [("means", "means"), ("quats", "quats"), ("scales", "scales"),
                      ("opacities", "opac")]:
        _check(name, g[name], t[key].grad)
    _check("features", g["colors"], t["f"].grad)
