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
