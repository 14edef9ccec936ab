"""Pins the oracle's bin_gaussians (tiles.py:19-182) against a brute-force
enumerate-and-stable-sort and the reference's invariants
(test_splatting.py:198-211)."""

import numpy as np
import pytest

from oracle import oracle as O
from refimpl import bin_bruteforce, oracle_camera, random_scene


def _proj(seed=0, **kw):
    cam, means, quats, scales, opac, colors = random_scene(seed, **kw)
    p = O.project(oracle_camera(cam), means, quats, scales)
    return cam, p


def test_binning_invariants_reference_scene():
    cam, p = _proj(0)
    ids, ranges, tx, ty = O.bin_gaussians(p["means2d"], p["radii"], p["depths"], cam.width,
                                          cam.height)
    assert (tx, ty) == (6, 4)
    assert (ranges[:, 1] >= ranges[:, 0]).all()
    assert int((ranges[:, 1] - ranges[:, 0]).sum()) == ids.shape[0]
    assert ids.min() >= 0 and ids.max() < 300


@pytest.mark.parametrize("seed,threads", [(0, 1), (1, 1), (2, 4), (3, 8)])
def test_binning_matches_bruteforce(seed, threads):
    cam, p = _proj(seed, n=400, width=112, height=80)
    ids, ranges, _, _ = O.bin_gaussians(p["means2d"], p["radii"], p["depths"], cam.width,
                                        cam.height, threads=threads)
    bids, branges, _, _ = bin_bruteforce(p["means2d"], p["radii"], p["depths"], cam.width,
                                         cam.height)
    np.testing.assert_array_equal(ids, bids)
    np.testing.assert_array_equal(ranges, branges)


def test_binning_depth_ties_break_by_index():
    rng = np.random.default_rng(3)
    n = 200
    means2d = rng.uniform(0, 64, (n, 2)).astype(np.float32)
    radii = rng.integers(1, 20, n).astype(np.float32)
    depths = rng.choice(np.array([1.0, 2.0, 2.0, 3.0], np.float32), n)  # many exact ties
    ids, ranges, _, _ = O.bin_gaussians(means2d, radii, depths, 64, 64)
    bids, branges, _, _ = bin_bruteforce(means2d, radii, depths, 64, 64)
    np.testing.assert_array_equal(ids, bids)
    np.testing.assert_array_equal(ranges, branges)


def test_binning_empty_and_culled():
    ids, ranges, tx, ty = O.bin_gaussians(np.zeros((0, 2)), np.zeros(0), np.zeros(0), 40, 20)
    assert ids.shape == (0,) and ranges.shape == (tx * ty, 2) and not ranges.any()
    # all culled (radius 0) or off screen
    m = np.array([[10.0, 10.0], [-100.0, 5.0], [5.0, 500.0]], np.float32)
    r = np.array([0.0, 3.0, 3.0], np.float32)
    ids, ranges, _, _ = O.bin_gaussians(m, r, np.ones(3, np.float32), 40, 20)
    assert ids.shape == (0,) and not ranges.any()


def test_binning_huge_splat_covers_everything():
    m = np.array([[20.0, 10.0], [5.0, 5.0]], np.float32)
    r = np.array([1e4, 2.0], np.float32)
    ids, ranges, tx, ty = O.bin_gaussians(m, r, np.array([2.0, 1.0], np.float32), 40, 20)
    assert ids.shape[0] == tx * ty + 1
    assert list(ids[ranges[0, 0]:ranges[0, 1]]) == [1, 0]  # depth order in tile 0


def _elongated_scene(seed, n=300, width=128, height=96):
    """Thin, rotated Gaussians whose square 3-sigma boxes cover many tiles
    the ellipse never reaches (what refine_tiles removes)."""
    rng = np.random.default_rng(seed)
    means2d = rng.uniform(-10, [width + 10, height + 10], (n, 2)).astype(np.float32)
    sig_major = rng.uniform(4.0, 30.0, n)
    sig_minor = rng.uniform(0.5, 2.0, n)
    th = rng.uniform(0, np.pi, n)
    c, s = np.cos(th), np.sin(th)
    cov = np.stack([c * c * sig_major**2 + s * s * sig_minor**2,
                    c * s * (sig_major**2 - sig_minor**2),
                    s * s * sig_major**2 + c * c * sig_minor**2], 1)
    det = cov[:, 0] * cov[:, 2] - cov[:, 1] ** 2
    conics = np.stack([cov[:, 2] / det, -cov[:, 1] / det, cov[:, 0] / det], 1).astype(np.float32)
    radii = np.ceil(3.0 * sig_major).astype(np.float32)
    depths = rng.uniform(1, 5, n).astype(np.float32)
    return means2d, radii, depths, conics


@pytest.mark.parametrize("seed,threads", [(0, 1), (1, 4)])
def test_refine_tiles_matches_bruteforce(seed, threads):
    # tiles.py:91-164 restated independently in numpy float32
    m, r, d, co = _elongated_scene(seed)
    ids, ranges, _, _ = O.bin_gaussians(m, r, d, 128, 96, threads=threads, conics=co)
    bids, branges, _, _ = bin_bruteforce(m, r, d, 128, 96, conics=co)
    np.testing.assert_array_equal(ids, bids)
    np.testing.assert_array_equal(ranges, branges)
    full, _, _, _ = O.bin_gaussians(m, r, d, 128, 96)
    assert ids.shape[0] < 0.8 * full.shape[0]  # the refinement does remove tiles


def test_refine_tiles_keeps_order_and_subset():
    m, r, d, co = _elongated_scene(2)
    ids, ranges, _, _ = O.bin_gaussians(m, r, d, 128, 96, conics=co)
    fids, franges, _, _ = O.bin_gaussians(m, r, d, 128, 96)
    for t in range(ranges.shape[0]):
        kept = list(ids[ranges[t, 0]:ranges[t, 1]])
        full = list(fids[franges[t, 0]:franges[t, 1]])
        it = iter(full)
        assert all(g in it for g in kept)  # an order-preserving subsequence


def test_refine_tiles_does_not_change_the_image():
    # q > 12 means alpha = o exp(-q/2) < exp(-6) < 1/255 for o <= 1, so the
    # dropped pairs never composite: image and final_T are bit-identical
    m, r, d, co = _elongated_scene(3)
    rng = np.random.default_rng(3)
    opac = rng.uniform(0.2, 1.0, m.shape[0]).astype(np.float32)
    cols = rng.uniform(size=(m.shape[0], 3)).astype(np.float32)
    a = O.raster_fwd(m, co, opac, cols, *O.bin_gaussians(m, r, d, 128, 96, conics=co)[:2], 128, 96)
    b = O.raster_fwd(m, co, opac, cols, *O.bin_gaussians(m, r, d, 128, 96)[:2], 128, 96)
    np.testing.assert_array_equal(a["image"], b["image"])
    np.testing.assert_array_equal(a["final_T"], b["final_T"])


def test_refine_tiles_thin_diagonal_known_answer():
    # a needle along the main diagonal of a 64x64 image: its 3-sigma box
    # covers all 16 tiles, the ellipse only the diagonal band of tiles
    s_major, s_minor = 30.0, 0.6
    c, s = np.cos(np.pi / 4), np.sin(np.pi / 4)
    cov = np.array([c * c * s_major**2 + s * s * s_minor**2, c * s * (s_major**2 - s_minor**2),
                    s * s * s_major**2 + c * c * s_minor**2])
    det = cov[0] * cov[2] - cov[1] ** 2
    co = np.array([[cov[2] / det, -cov[1] / det, cov[0] / det]], np.float32)
    ids, ranges, tx, ty = O.bin_gaussians(np.array([[32.0, 32.0]], np.float32),
                                          np.array([90.0], np.float32),
                                          np.array([1.0], np.float32), 64, 64, conics=co)
    kept = {t for t in range(tx * ty) if ranges[t, 1] > ranges[t, 0]}
    diag = {i * tx + i for i in range(4)}
    assert diag <= kept
    assert 0 * tx + 3 not in kept and 3 * tx + 0 not in kept  # far corners dropped
