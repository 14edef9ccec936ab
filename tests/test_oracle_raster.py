"""Pins the oracle's tile compositing (rasterize.py:28-98, 223-290) against
a dense float64 restatement of reference.py restricted to the binned tiles
with the kernel's termination rule, closed forms, and the reference's own
1e-3 comparison with the unrestricted dense oracle (test_splatting.py:214-337)."""

import numpy as np
import torch

from oracle import oracle as O
from refimpl import dense_composite_f64, depth_order, oracle_camera, random_scene, tile_mask


def _render_oracle(cam, means, quats, scales, opac, feats, bg=None, antialias=False, depth=False):
    oc = oracle_camera(cam)
    p = O.project(oc, means, quats, scales, antialias=antialias)
    oe = (opac * p["compensation"]).astype(np.float32)
    ids, ranges, _, _ = O.bin_gaussians(p["means2d"], p["radii"], p["depths"], cam.width, cam.height)
    r = O.raster_fwd(p["means2d"], p["conics"], oe, feats, ids, ranges, cam.width, cam.height,
                     bg=bg, depths=p["depths"] if depth else None)
    return p, oe, ids, ranges, r


def _dense(cam, p, oe, feats, bg=None, restrict=True, kernel_stop=True):
    f64 = lambda a: torch.tensor(np.asarray(a), dtype=torch.float64)  # noqa: E731
    mask = tile_mask(p["means2d"], p["radii"], cam.width, cam.height) if restrict else \
        (p["radii"] > 0)[:, None, None] * np.ones((1, cam.height, cam.width), bool)
    img, T, w = dense_composite_f64(f64(p["means2d"]), f64(p["conics"]), f64(oe), f64(feats),
                                    depth_order(p["depths"]), cam.width, cam.height,
                                    bg=None if bg is None else f64(bg), mask=mask,
                                    kernel_stop=kernel_stop)
    return img.numpy(), T.numpy(), w


def test_forward_matches_dense_restricted_f64():
    cam, means, quats, scales, opac, colors = random_scene(0)
    bg = np.array([0.1, 0.2, 0.3], np.float32)
    p, oe, ids, ranges, r = _render_oracle(cam, means, quats, scales, opac, colors, bg)
    img, T, _ = _dense(cam, p, oe, colors, bg)
    np.testing.assert_allclose(r["image"], img, atol=1e-5)
    np.testing.assert_allclose(r["final_T"], T, atol=1e-5)


def test_forward_matches_reference_dense_oracle_1e3():
    # the reference's own check: unrestricted dense oracle, 1e-3
    cam, means, quats, scales, opac, colors = random_scene(0)
    bg = np.array([0.1, 0.2, 0.3], np.float32)
    p, oe, _, _, r = _render_oracle(cam, means, quats, scales, opac, colors, bg)
    img, T, _ = _dense(cam, p, oe, colors, bg, restrict=False, kernel_stop=False)
    np.testing.assert_allclose(r["image"], img, atol=1e-3)
    np.testing.assert_allclose(1 - r["final_T"], 1 - T, atol=1e-3)


def test_antialias_reduces_alpha():
    # test_splatting.py:243-277
    cam, means, quats, scales, opac, colors = random_scene(0)
    opac = (opac * 0.1).astype(np.float32)
    _, _, _, _, plain = _render_oracle(cam, means, quats, scales, opac, colors)
    p, oe, _, _, aa = _render_oracle(cam, means, quats, scales, opac, colors, antialias=True)
    assert ((1 - aa["final_T"]) - (1 - plain["final_T"])).max() <= 1e-6
    img, T, _ = _dense(cam, p, oe, colors)
    np.testing.assert_allclose(aa["image"], img, atol=1e-5)
    assert (p["compensation"] <= 1).all() and (p["compensation"] < 1).any()


def test_single_gaussian_closed_form():
    # one Gaussian: image = min(0.99, o e^power) * colour where alpha >= 1/255
    W = H = 32
    means2d = np.array([[15.3, 16.8]], np.float32)
    conics = np.array([[0.05, 0.01, 0.08]], np.float32)
    o = np.array([0.8], np.float32)
    col = np.array([[0.2, 0.5, 1.0]], np.float32)
    ids, ranges, _, _ = O.bin_gaussians(means2d, np.array([20.0], np.float32),
                                        np.array([1.0], np.float32), W, H)
    r = O.raster_fwd(means2d, conics, o, col, ids, ranges, W, H)
    ys, xs = np.mgrid[0:H, 0:W] + 0.5
    dx, dy = 15.3 - xs, 16.8 - ys
    power = -0.5 * (0.05 * dx * dx + 0.08 * dy * dy) - 0.01 * dx * dy
    a = np.minimum(0.99, 0.8 * np.exp(power))
    a = np.where((power > 0) | (a < 1 / 255), 0, a)
    np.testing.assert_allclose(r["image"], a[..., None] * col[0], atol=2e-7)
    np.testing.assert_array_equal(r["n_contrib"], (a > 0).astype(np.int32))


def test_opaque_front_splat_terminates():
    # a near-opaque front splat stack drives T below 1e-4: later splats unseen
    W = H = 16
    n = 6
    means2d = np.full((n, 2), 8.0, np.float32)
    conics = np.tile(np.array([[1e-4, 0.0, 1e-4]], np.float32), (n, 1))
    o = np.full(n, 0.99, np.float32)
    col = np.eye(3, dtype=np.float32)[np.arange(n) % 3]
    depths = np.arange(1, n + 1, dtype=np.float32)
    ids, ranges, _, _ = O.bin_gaussians(means2d, np.full(n, 4.0, np.float32), depths, W, H)
    r = O.raster_fwd(means2d, conics, o, col, ids, ranges, W, H)
    # alpha = 0.99 * e^{-tiny}; T after 2 splats ~1e-4 -> the second crossing stops
    assert (r["n_contrib"] <= 2).all() and (r["n_contrib"] >= 1).all()
    assert (r["final_T"] >= 1e-4).all()


def test_depth_and_features():
    # depth kernel semantics (rasterize.py:223-290) and feature padding
    # equivalence (test_splatting.py:280-337)
    cam, means, quats, scales, opac, colors = random_scene(1)
    feats = np.concatenate([means, (np.arange(600, dtype=np.float32).reshape(300, 2) / 300)], 1)
    bg = np.linspace(-0.2, 0.2, 5).astype(np.float32)
    p, oe, ids, ranges, r = _render_oracle(cam, means, quats, scales, opac, feats, bg, depth=True)
    img, T, w = _dense(cam, p, oe, feats, bg)
    np.testing.assert_allclose(r["image"], img, atol=1e-5)
    # expected depth = sum w z / (1 - T)
    z = torch.tensor(p["depths"], dtype=torch.float64)[depth_order(p["depths"])]
    dz = torch.einsum("nhw,n->hw", w, z).numpy()
    al = 1 - T
    ref = np.where(al > 1e-6, dz / np.maximum(al, 1e-12), 0)
    valid = al > 1e-3
    np.testing.assert_allclose(r["depth"][valid], ref[valid], rtol=1e-5)
    assert np.isfinite(r["depth"]).all() and (r["depth"][valid] > 0).all()
    # channels are independent: a 1-channel pass equals the slice
    r1 = O.raster_fwd(p["means2d"], p["conics"], oe, feats[:, 3:4], ids, ranges, cam.width,
                      cam.height, bg=bg[3:4])
    np.testing.assert_array_equal(r1["image"][..., 0], r["image"][..., 3])
    np.testing.assert_array_equal(r1["n_contrib"], r["n_contrib"])


def test_tile_subset_equals_full():
    cam, means, quats, scales, opac, colors = random_scene(2)
    p, oe, ids, ranges, r = _render_oracle(cam, means, quats, scales, opac, colors)
    tiles = np.array([0, 5, 7, 23], np.int32)
    s = O.raster_fwd(p["means2d"], p["conics"], oe, colors, ids, ranges, cam.width, cam.height,
                     tiles=tiles)
    for t in tiles:
        ty, tx = divmod(int(t), 6)
        sl = (slice(16 * ty, 16 * ty + 16), slice(16 * tx, 16 * tx + 16))
        np.testing.assert_array_equal(s["image"][sl], r["image"][sl])
        np.testing.assert_array_equal(s["n_contrib"][sl], r["n_contrib"][sl])
