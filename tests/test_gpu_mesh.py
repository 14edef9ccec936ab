"""GPU mesh rasterizer (gsx_mesh_raster on the shared tile binning) against
the CPU oracle bit for bit, plus the reference's own rasterizer tests
(test_rasterizer.py:20-84) and a 1080p timing."""

from __future__ import annotations

import time

import numpy as np
import pytest
import torch

from gpu_util import cu, host, say
from mlx3d_amd.cameras import Camera
from mlx3d_amd.renderer import interpolate_face_attributes, rasterize_meshes
from oracle import oracle as O
from refimpl import ico_sphere

pytestmark = pytest.mark.gpu


def _oracle(cam, verts_gpu, faces):
    xy, z = cam.project_points(verts_gpu)
    xy, z = host(xy), host(z)
    tri_xy, tri_z = xy[faces], z[faces]
    centroid = tri_xy.mean(1).astype(np.float32)
    radii = np.sqrt(((tri_xy - centroid[:, None, :]) ** 2).sum(-1).max(1)).astype(np.float32)
    depths = tri_z.mean(1).astype(np.float32)
    ids, ranges, _, _ = O.bin_gaussians(centroid, radii, depths, cam.width, cam.height)
    return O.mesh_raster(tri_xy.reshape(-1, 6), tri_z, ids, ranges, cam.width, cam.height,
                         threads=O.default_threads())


@pytest.mark.parametrize("level,eye,size", [(3, (2.2, 1.6, 2.2), (96, 80)),
                                            (5, (0.4, -0.3, -2.2), (640, 360))])
def test_mesh_raster_bitexact(level, eye, size):
    say(f"mesh raster level {level} {size}")
    verts, faces = ico_sphere(level)
    cam = Camera.look_at(eye=eye, at=(0, 0, 0), fov=50.0, width=size[0], height=size[1])
    v = cu(verts)
    frag = rasterize_meshes(cam, v, cu(faces))
    p2f, zb = _oracle(cam, v, faces)
    np.testing.assert_array_equal(host(frag.pix_to_face), p2f)
    np.testing.assert_array_equal(host(frag.zbuf).view(np.int32), zb.view(np.int32))
    assert (p2f >= 0).mean() > 0.2


def _tri_cam():
    cam = Camera.look_at(eye=(0, 0, -3.0), at=(0, 0, 0), fov=60.0, width=32, height=32)
    verts = cu(np.array([[-0.6, -0.5, 0.0], [0.6, -0.5, 0.0], [0.0, 0.6, 0.0]], np.float32))
    return cam, verts, cu(np.array([[0, 1, 2]], np.int32))


def test_reference_rasterizer_behaviour():
    cam, verts, faces = _tri_cam()
    frag = rasterize_meshes(cam, verts, faces)
    assert int(frag.pix_to_face[16, 16]) == 0 and int(frag.pix_to_face[0, 0]) == -1
    assert not bool(frag.valid[0, 0])
    s = frag.bary.sum(-1)
    assert float((torch.where(frag.valid, s, torch.ones_like(s)) - 1).abs().max()) < 1e-4
    colors = cu(np.eye(3, dtype=np.float32))
    img = interpolate_face_attributes(frag, colors)
    cs = img.sum(-1)
    assert float((torch.where(frag.valid, cs, torch.ones_like(cs)) - 1).abs().max()) < 1e-4
    assert float(img.min()) >= -1e-5
    cam2 = Camera.look_at(eye=(0, 0, -3.0), at=(0, 0, 0), fov=60.0, width=16, height=16)
    v2 = cu(np.array([[-0.6, -0.5, 0.5], [0.6, -0.5, 0.5], [0.0, 0.6, 0.5],
                      [-0.6, -0.5, -0.5], [0.6, -0.5, -0.5], [0.0, 0.6, -0.5]], np.float32))
    f2 = cu(np.array([[0, 1, 2], [3, 4, 5]], np.int32))
    assert int(rasterize_meshes(cam2, v2, f2).pix_to_face[8, 8]) == 1


def test_gradient_flows_to_vertices():
    verts, faces = ico_sphere(2)
    cam = Camera.look_at(eye=(2.2, 1.6, 2.2), at=(0, 0, 0), fov=45.0, width=48, height=48)
    v = cu(verts).requires_grad_(True)
    vc = (0.5 * v + 0.5).detach()
    frag = rasterize_meshes(cam, v, cu(faces))
    interpolate_face_attributes(frag, vc).sum().backward()
    g = v.grad
    assert bool(torch.isfinite(g).all()) and float(g.abs().sum()) > 0.0


def test_mesh_raster_1080p_timing():
    verts, faces = ico_sphere(6)  # 81920 faces
    cam = Camera.look_at(eye=(1.2, 0.8, -1.6), at=(0, 0, 0), fov=60.0, width=1920, height=1080)
    v, f = cu(verts), cu(faces)
    for _ in range(3):
        rasterize_meshes(cam, v, f)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(20):
        frag = rasterize_meshes(cam, v, f)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / 20
    say(f"rasterize_meshes icosphere-6 ({faces.shape[0]} faces) 1920x1080: {ms:.3f} ms "
        f"({1e3 / ms:.0f} fps), coverage {float(frag.valid.float().mean()):.2f}")
    assert ms < 50.0
