"""Pins the mesh-rasterizer oracle (oracle/mesh_oracle.c) against an
all-faces float64 z-buffer (tests/refimpl.py) over the binned lists, and
restates the reference's own rasterizer tests (test_rasterizer.py:20-57)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from mlx3d_amd.cameras import Camera
from oracle import oracle as O
from refimpl import ico_sphere, mesh_zbuffer_f64


def _prep(cam, verts, faces):
    xy, z = cam.project_points(torch.tensor(verts))
    xy, z = xy.numpy(), z.numpy()
    tri_xy = xy[faces]
    tri_z = z[faces]
    centroid = tri_xy.mean(1)
    radii = np.sqrt(((tri_xy - centroid[:, None, :]) ** 2).sum(-1).max(1)).astype(np.float32)
    depths = tri_z.mean(1).astype(np.float32)
    ids, ranges, _, _ = O.bin_gaussians(centroid.astype(np.float32), radii, depths, cam.width,
                                        cam.height)
    return tri_xy.reshape(-1, 6), tri_z, ids, ranges


@pytest.mark.parametrize("level,eye", [(2, (2.2, 1.6, 2.2)), (3, (0.3, 0.2, -2.5))])
def test_mesh_oracle_matches_all_faces_zbuffer(level, eye):
    verts, faces = ico_sphere(level)
    cam = Camera.look_at(eye=eye, at=(0, 0, 0), fov=45.0, width=72, height=56)
    tri_xy, tri_z, ids, ranges = _prep(cam, verts, faces)
    p2f, zb = O.mesh_raster(tri_xy, tri_z, ids, ranges, cam.width, cam.height)
    best, bz, margin, amb = mesh_zbuffer_f64(tri_xy, tri_z, cam.width, cam.height)
    clear = (margin > 1e-4) & ~amb
    assert (p2f >= 0).mean() > 0.3 and clear.mean() > 0.9
    np.testing.assert_array_equal(p2f[clear], best[clear])
    np.testing.assert_allclose(zb[clear], bz[clear], rtol=1e-5, atol=1e-6)
    assert ((p2f >= 0) == (best >= 0))[~amb].all()


def _tri_cam():
    cam = Camera.look_at(eye=(0, 0, -3.0), at=(0, 0, 0), fov=60.0, width=32, height=32)
    verts = np.array([[-0.6, -0.5, 0.0], [0.6, -0.5, 0.0], [0.0, 0.6, 0.0]], np.float32)
    return cam, verts, np.array([[0, 1, 2]], np.int32)


def test_triangle_hit_and_miss():
    cam, verts, faces = _tri_cam()
    p2f, zb = O.mesh_raster(*_prep(cam, verts, faces), cam.width, cam.height)
    assert p2f[16, 16] == 0 and p2f[0, 0] == -1 and zb[0, 0] == 0.0
    assert abs(zb[16, 16] - 3.0) < 1e-5  # the triangle lies in the plane z_cam = 3


def test_depth_ordering_near_face_wins():
    cam = Camera.look_at(eye=(0, 0, -3.0), at=(0, 0, 0), fov=60.0, width=16, height=16)
    verts = np.array([[-0.6, -0.5, 0.5], [0.6, -0.5, 0.5], [0.0, 0.6, 0.5],
                      [-0.6, -0.5, -0.5], [0.6, -0.5, -0.5], [0.0, 0.6, -0.5]], np.float32)
    faces = np.array([[0, 1, 2], [3, 4, 5]], np.int32)
    p2f, _ = O.mesh_raster(*_prep(cam, verts, faces), cam.width, cam.height)
    assert p2f[8, 8] == 1


def test_behind_camera_and_empty():
    cam, verts, faces = _tri_cam()
    behind = verts + np.array([0, 0, -4.0], np.float32)  # z_cam = -1
    p2f, zb = O.mesh_raster(*_prep(cam, behind, faces), cam.width, cam.height)
    assert (p2f == -1).all() and (zb == 0).all()
    p2f, zb = O.mesh_raster(np.zeros((0, 6)), np.zeros((0, 3)), np.zeros(0, np.int32),
                            np.zeros((4, 2), np.int32), 32, 32)
    assert (p2f == -1).all()
