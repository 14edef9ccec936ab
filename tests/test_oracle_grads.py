"""Pins the oracle's backward (rasterize.py:100-221 + the VJP of the
projection/SH/activations that MLX autodiff computes) against torch float64
autograd of an independent dense render, with the reference's criterion
max|d| / max|ref| < 1e-3 (test_splatting.py:340-414).  Most scenes keep
opacities below 0.99 so the forward clamp is inactive; the active-clamp
branch (the kernel passes gradient through min(0.99, o G), rasterize.py:193,
where autograd would not) is pinned by a closed form on one splat and by
autograd of a dense render with a straight-through clamp at opacities up
to 1."""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from refimpl import (dense_composite_f64, depth_order, oracle_camera, random_scene, render_f64,
                     tile_mask)


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


def _single_splat(opacity, sigma, offset):
    """One Gaussian straight ahead of a look_at camera: means2d lands on the
    centre pixel's centre plus ``offset`` (pixels, x), isotropic conic 1/sigma^2."""
    W = H = 16
    m2 = np.array([[8.5 + offset, 8.5]], np.float32)
    con = np.array([[1.0 / sigma ** 2, 0.0, 1.0 / sigma ** 2]], np.float32)
    op = np.array([opacity], np.float32)
    col = np.array([[0.7, 0.2, 0.4]], np.float32)
    ids = np.zeros(1, np.int32)
    ranges = np.zeros((1, 2), np.int32)
    ranges[0] = (0, 1)
    return W, H, m2, con, op, col, ids, ranges


@pytest.mark.parametrize("offset", [0.0, 0.3])
def test_active_clamp_gradient_closed_form(offset):
    """o G > 0.99 at the centre pixel, so alpha is clamped there; with the
    loss = image[8, 8, 0] the reference's backward (rasterize.py:187-218)
    gives, in closed form with one splat and a zero background:
        dL/dalpha = c0 (T = 1, nothing behind),
        dL/dG = o dL/dalpha (passes through the clamp, :193),
        dL/dopacity = G dL/dalpha, dL/dc0 = alpha T = 0.99,
        dL/dmean_x = dL/dG * G * (-a dx), dx = mean_x - 8.5 (power = -a dx^2 / 2)."""
    W, H, m2, con, op, col, ids, ranges = _single_splat(1.0, 3.0, offset)
    r = O.raster_fwd(m2, con, op, col, ids, ranges, W, H)
    a = np.float64(con[0, 0])
    dx = np.float64(m2[0, 0]) - 8.5
    G = np.exp(-0.5 * a * dx * dx)
    assert op[0] * G > 0.99  # the clamp is active at the centre pixel
    np.testing.assert_allclose(r["image"][8, 8, 0], 0.99 * col[0, 0], rtol=1e-6)
    g_img = np.zeros((H, W, 3), np.float32)
    g_img[8, 8, 0] = 1.0
    gr = O.raster_bwd(m2, con, op, col, ids, ranges, W, H, r["final_T"], r["n_contrib"], g_img)
    c0 = np.float64(col[0, 0])
    np.testing.assert_allclose(gr["opacities"][0], G * c0, rtol=1e-5)
    np.testing.assert_allclose(gr["features"][0], [0.99, 0.0, 0.0], rtol=1e-6, atol=1e-7)
    dLdG = op[0] * c0
    np.testing.assert_allclose(gr["means2d"][0, 0], dLdG * G * (-a * dx), rtol=1e-4, atol=1e-7)
    np.testing.assert_allclose(gr["means2d"][0, 1], 0.0, atol=1e-7)
    # conic gradient (-G dx^2 / 2, -G dx dy, -G dy^2 / 2) dL/dG
    np.testing.assert_allclose(gr["conics"][0], [-0.5 * G * dx * dx * dLdG, 0.0, 0.0],
                               rtol=1e-4, atol=1e-7)


@pytest.mark.parametrize("antialias", [False, True])
def test_gradients_with_active_clamp(antialias):
    """Opacities up to 1: the 0.99 clamp is active at many pixels.  The
    oracle's raster + preprocess backward against float64 autograd of the
    dense render with the reference kernel's straight-through clamp rule
    (rasterize.py:193), to the reference's 1e-3 criterion."""
    cam, means, quats, scales, opac, colors = random_scene(5)
    rng = np.random.default_rng(50)
    opac = rng.uniform(0.6, 1.0, opac.shape).astype(np.float32)
    opac[::2] = 1.0
    scales = (scales * 4.0).astype(np.float32)
    g_img = rng.standard_normal((cam.height, cam.width, 3)).astype(np.float32)
    g_alpha = rng.standard_normal((cam.height, cam.width)).astype(np.float32)
    flags = O.ANTIALIAS if antialias else 0
    g, pre, r = _oracle_grads(cam, means, quats, scales, opac, feats=colors, flags=flags,
                              g_img=g_img, g_alpha=g_alpha)
    t = {k: torch.tensor(v, dtype=torch.float64, requires_grad=True)
         for k, v in dict(means=means, quats=quats, scales=scales, opac=opac, colors=colors).items()}
    mask = tile_mask(pre["means2d"], pre["radii"], cam.width, cam.height)
    img, T, p = render_f64(cam, t["means"], t["quats"], t["scales"], t["opac"],
                           colors=t["colors"], antialias=antialias, mask=mask,
                           order=depth_order(pre["depths"]), straight_through=True)
    # how often the clamp is active where a pair composites
    with torch.no_grad():
        xs = torch.arange(cam.width, dtype=torch.float64) + 0.5
        ys = torch.arange(cam.height, dtype=torch.float64) + 0.5
        m, co = p["means2d"], p["conics"]
        dx = m[:, 0, None, None] - xs[None, None, :]
        dy = m[:, 1, None, None] - ys[None, :, None]
        power = -0.5 * (co[:, 0, None, None] * dx * dx + co[:, 2, None, None] * dy * dy) \
            - co[:, 1, None, None] * dx * dy
        raw = (t["opac"] * p["compensation"])[:, None, None] * torch.exp(power)
        clamped = int(((raw > 0.99) & torch.as_tensor(mask)).sum())
    assert clamped > 50, clamped
    np.testing.assert_allclose(r["image"], img.detach().numpy(), atol=1e-5)
    loss = (img * torch.tensor(g_img, dtype=torch.float64)).sum() + \
        ((1 - T) * torch.tensor(g_alpha, dtype=torch.float64)).sum()
    loss.backward()
    _check("means", g["means"], t["means"].grad)
    _check("quats", g["quats"], t["quats"].grad)
    _check("scales", g["scales"], t["scales"].grad)
    _check("opacities", g["opacities"], t["opac"].grad)
    _check("colors", g["colors"], t["colors"].grad)


def test_straight_through_rule_differs_from_autodiff():
    """The check above can tell the two clamp rules apart: with the clamp
    active, autodiff's zero-gradient rule moves the opacity gradient by far
    more than the 1e-3 criterion."""
    W, H, m2, con, op, col, ids, ranges = _single_splat(1.0, 3.0, 0.0)
    order = torch.zeros(1, dtype=torch.int64)
    out = {}
    for st in (False, True):
        o = torch.tensor(op, dtype=torch.float64, requires_grad=True)
        img, _, _ = dense_composite_f64(torch.tensor(m2, dtype=torch.float64),
                                        torch.tensor(con, dtype=torch.float64), o,
                                        torch.tensor(col, dtype=torch.float64), order, W, H,
                                        straight_through=st)
        img[8, 8, 0].backward()
        out[st] = float(o.grad[0])
    assert out[False] == 0.0
    np.testing.assert_allclose(out[True], col[0, 0], rtol=1e-6)
