"""Pins the training-step oracle (oracle/train_oracle.c, oracle/density.py)
against checks that do not restate its formulas:

* SSIM value and gradient: a float64 PyTorch autograd evaluation of the
  reference's expression (depthwise conv2d, image_metrics.py:29-55), which
  exercises an independent convolution and differentiates it automatically;
  the zero-padded window against scipy.ndimage.correlate on constant images;
  identities (SSIM(x, x) = 1 with zero gradient, symmetry).
* Adam: the closed form of the first step (m/sqrt(v) = 0.1/sqrt(0.001) sign g)
  and a float64 restatement over several steps.
* Screen-gradient statistics: a known answer (3-4-5 triangle).
* Density control: a hand-built table whose clone / split / prune outcome is
  fixed by construction, and the split-sample covariance.
"""

from __future__ import annotations

import numpy as np
import pytest
import scipy.ndimage
import torch

from oracle import density as DN
from oracle import oracle as O


def _ssim_torch(pred, target, ws=11, sigma=1.5, max_val=1.0):
    x = torch.arange(ws, dtype=torch.float64) - (ws - 1) / 2
    g = torch.exp(-(x * x) / (2 * sigma * sigma))
    g = g / g.sum()
    w = (g[:, None] * g[None, :])[None, None].expand(pred.shape[-1], 1, ws, ws)
    P = pred.permute(2, 0, 1)[None]
    T = target.permute(2, 0, 1)[None]

    def f(z):
        return torch.nn.functional.conv2d(z, w, padding=ws // 2, groups=pred.shape[-1])

    mp, mt = f(P), f(T)
    sp, st, spt = f(P * P) - mp * mp, f(T * T) - mt * mt, f(P * T) - mp * mt
    c1, c2 = (0.01 * max_val) ** 2, (0.03 * max_val) ** 2
    cs = (2 * spt + c2) / (sp + st + c2)
    return ((2 * mp * mt + c1) / (mp * mp + mt * mt + c1) * cs).mean()


@pytest.mark.parametrize("H,W,C,ws,sigma", [(19, 23, 3, 11, 1.5), (8, 5, 1, 11, 1.5),
                                            (16, 16, 3, 3, 0.8), (21, 17, 2, 15, 2.5),
                                            (12, 9, 3, 1, 1.0)])
def test_photometric_matches_autograd(H, W, C, ws, sigma):
    rng = np.random.default_rng(H * W + ws)
    p = rng.random((H, W, C), dtype=np.float32)
    t = rng.random((H, W, C), dtype=np.float32)
    l1, s, g = O.photometric(p, t, ws, sigma, g_l1=0.8, g_ssim=-0.2, grad=True)
    P = torch.tensor(p, dtype=torch.float64, requires_grad=True)
    T = torch.tensor(t, dtype=torch.float64)
    ref_s = _ssim_torch(P, T, ws, sigma)
    ref_l1 = (P - T).abs().mean()
    (0.8 * ref_l1 - 0.2 * ref_s).backward()
    assert abs(s - ref_s.item()) < 1e-12
    assert abs(l1 - ref_l1.item()) < 1e-12
    np.testing.assert_allclose(g, P.grad.numpy(), rtol=0, atol=1e-12 * np.abs(g).max() + 1e-16)


def test_photometric_identities():
    rng = np.random.default_rng(3)
    p = rng.random((20, 26, 3), dtype=np.float32)
    t = rng.random((20, 26, 3), dtype=np.float32)
    l1, s, g = O.photometric(p, p, g_ssim=1.0, grad=True)
    assert l1 == 0.0 and abs(s - 1.0) < 1e-12
    assert np.abs(g).max() < 1e-12  # SSIM is maximal at pred == target
    assert abs(O.photometric(p, t)[1] - O.photometric(t, p)[1]) < 1e-12
    # L1 gradient alone: sign(p - t) / n
    _, _, g = O.photometric(p, t, g_l1=1.0, grad=True)
    np.testing.assert_array_equal(g, np.sign(p.astype(np.float64) - t) / p.size)


@pytest.mark.parametrize("a,b", [(0.3, 0.7), (1.0, 0.0), (0.5, 0.5)])
def test_photometric_constant_images_scipy_window(a, b):
    """Constant images: every filtered map is a multiple of the zero-padded
    window sum, taken here from scipy.ndimage.correlate."""
    H, W, ws, sigma = 13, 18, 11, 1.5
    x = np.arange(ws) - (ws - 1) / 2
    g = np.exp(-x * x / (2 * sigma * sigma))
    g /= g.sum()
    m1 = scipy.ndimage.correlate(np.ones((H, W)), np.outer(g, g), mode="constant", cval=0.0)
    mp, mt = a * m1, b * m1
    sp, st, spt = a * a * m1 - mp * mp, b * b * m1 - mt * mt, a * b * m1 - mp * mt
    c1, c2 = 1e-4, 9e-4
    S = (2 * mp * mt + c1) / (mp * mp + mt * mt + c1) * (2 * spt + c2) / (sp + st + c2)
    p = np.full((H, W, 1), a, np.float32)
    t = np.full((H, W, 1), b, np.float32)
    l1, s = O.photometric(p, t)
    assert abs(s - S.mean()) < 1e-6 * max(1.0, abs(S.mean()))
    assert abs(l1 - abs(np.float32(a) - np.float32(b))) < 1e-7


def test_adam_first_step_closed_form():
    rng = np.random.default_rng(0)
    g = rng.normal(size=1000).astype(np.float32) * np.float32(10.0) ** rng.integers(-6, 3, 1000)
    g[:7] = 0.0
    p0 = rng.normal(size=1000).astype(np.float32)
    lr = 1e-3
    p1, m1, v1 = O.adam(p0, g, np.zeros(1000), np.zeros(1000), lr)
    step = (p0.astype(np.float64) - p1) / lr
    expect = np.sign(g) * 0.1 / np.sqrt(0.001)
    # float32 rounding of p1 (|p0| ~ 1) limits the recovered step to ~1e-4
    np.testing.assert_allclose(step, expect, atol=2e-4 * np.abs(p0).max() / lr * 1e-3 + 1e-3)
    assert (p1[:7] == p0[:7]).all() and (m1[:7] == 0).all() and (v1[:7] == 0).all()


def test_adam_matches_float64_over_steps():
    rng = np.random.default_rng(1)
    n = 4096
    p = rng.normal(size=n).astype(np.float32)
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    pd, md, vd = p.astype(np.float64), np.zeros(n), np.zeros(n)
    for step in range(6):
        g = rng.normal(size=n).astype(np.float32)
        lr = 1e-2 * 0.9 ** step
        p, m, v = O.adam(p, g, m, v, lr, eps=1e-8)
        md = 0.9 * md + 0.1 * g
        vd = 0.999 * vd + 0.001 * g.astype(np.float64) ** 2
        pd = pd - np.float32(lr) * md / (np.sqrt(vd) + 1e-8)
    np.testing.assert_allclose(p, pd, rtol=0, atol=1e-5)
    np.testing.assert_allclose(m, md, rtol=1e-5, atol=1e-7)


def test_accum_screen_grads_known_answer():
    W, H = 200, 100
    # gx = 0.03 * 100 = 3, gy = 0.08 * 50 = 4: norm 5
    g = np.array([[0.03, 0.08], [0.03, 0.08], [0.0, 0.0]], np.float32)
    radii = np.array([2.0, 0.0, 1.0], np.float32)
    acc, cnt = O.accum_screen_grads(g, radii, W, H, np.ones(3), np.full(3, 2.0))
    np.testing.assert_allclose(acc, [6.0, 1.0, 1.0], rtol=1e-6)
    np.testing.assert_array_equal(cnt, [3.0, 2.0, 3.0])


def _table():
    """Five rows with a known density-control outcome (extent 1, percent_dense
    0.01): 0 clone (small, high grad), 1 split (large, high grad), 2 pruned
    (opacity 0.001), 3 pruned (oversized), 4 kept untouched."""
    n = 5
    means = np.arange(15, dtype=np.float32).reshape(n, 3)
    scales = np.log(np.array([[0.005] * 3, [0.1, 0.05, 0.02], [0.01] * 3, [0.7] * 3,
                              [0.02] * 3], np.float32))
    quats = np.array([[1, 0, 0, 0], [0.7, 0.2, -0.5, 0.1], [1, 0, 0, 0], [1, 0, 0, 0],
                      [1, 0, 0, 0]], np.float32)
    opac = np.array([0.0, 1.0, np.log(0.001 / 0.999), 2.0, 0.5], np.float32)
    sh_dc = np.arange(n * 3, dtype=np.float32).reshape(n, 1, 3)
    sh_rest = np.arange(n * 45, dtype=np.float32).reshape(n, 15, 3)
    params = dict(means=means, scales=scales, quats=quats, opacities=opac, sh_dc=sh_dc,
                  sh_rest=sh_rest)
    acc = np.array([0.01, 0.01, 0.0, 0.0, 0.0], np.float32)
    cnt = np.array([10, 10, 10, 10, 10], np.float32)
    return params, acc, cnt


def test_density_known_outcome():
    params, acc, cnt = _table()
    np.random.seed(5)
    out, stats, keep = DN.densify_and_prune(params, acc, cnt)
    assert stats == {"cloned": 1, "split": 1, "pruned": 3}
    np.testing.assert_array_equal(keep, [0, 4])
    assert out["means"].shape == (5, 3)  # kept 0, 4; clone of 0; two halves of 1
    np.testing.assert_array_equal(out["means"][:3], params["means"][[0, 4, 0]])
    np.testing.assert_allclose(out["scales"][3:], params["scales"][[1, 1]] - np.log(1.6),
                               rtol=1e-6)
    np.testing.assert_array_equal(out["sh_rest"][3:], params["sh_rest"][[1, 1]])
    # the split offsets are R diag(s) xi with xi ~ N(0, I): undo R and s
    R = DN.quaternion_to_matrix(params["quats"][1])
    s = np.exp(params["scales"][1])
    local = (out["means"][3:] - params["means"][1]) @ R / s
    np.random.seed(5)
    np.testing.assert_allclose(local, np.random.normal(size=(2, 3)), rtol=1e-4, atol=1e-4)


def test_split_sample_covariance():
    """Many splits of one Gaussian: the offsets' covariance is R diag(s^2) R^T."""
    n = 4000
    q = np.array([0.6, -0.3, 0.5, 0.2], np.float32)
    s = np.array([0.3, 0.1, 0.05], np.float32)
    params = dict(means=np.zeros((n, 3), np.float32),
                  scales=np.tile(np.log(s), (n, 1)).astype(np.float32),
                  quats=np.tile(q, (n, 1)), opacities=np.full(n, 3.0, np.float32),
                  sh_dc=np.zeros((n, 1, 3), np.float32), sh_rest=np.zeros((n, 0, 3), np.float32))
    np.random.seed(0)
    out, stats, _ = DN.densify_and_prune(params, np.ones(n, np.float32), np.ones(n, np.float32),
                                         scene_extent=1.0)
    assert stats["split"] == n
    off = out["means"].astype(np.float64)
    R = DN.quaternion_to_matrix(q).astype(np.float64)
    cov = R @ np.diag(s.astype(np.float64) ** 2) @ R.T
    # standard error of a Gaussian sample covariance entry
    se = np.sqrt((np.outer(np.diag(cov), np.diag(cov)) + cov * cov) / off.shape[0])
    assert (np.abs(np.cov(off.T) - cov) < 5 * se).all()


def test_relocate_selection_known():
    n = 100
    params = dict(means=np.zeros((n, 3), np.float32),
                  opacities=np.linspace(-3, 3, n).astype(np.float32))
    acc = np.arange(n, dtype=np.float32)
    cnt = np.ones(n, np.float32)
    cnt[[3, 50]] = 0.0  # never seen: relocation targets even though opaque enough
    k, dst, src = DN.relocate_select(params, acc, cnt, relocate_frac=0.05, min_opacity=0.05)
    # opacity < 0.05 means logit < -2.944: only row 0 (row 1 is at -2.939);
    # with the unseen rows 3 and 50 that makes 3 underused rows, k = min(5, 3)
    assert k == 3
    np.testing.assert_array_equal(dst, [0, 3, 50])
    np.testing.assert_array_equal(src, [97, 98, 99])
