"""Hard z-buffer mesh rasterizer on the Gaussian tile binning
(``src/mlx3d/renderer/rasterizer.py``).

Faces are binned into 16x16 tiles by ``bin_gaussians`` with a per-face
bounding circle (centroid, largest vertex distance, mean depth;
rasterizer.py:140-146); ``gsx_mesh_raster`` resolves the nearest face per
pixel; barycentrics are then recomputed with torch from the projected
vertices so gradients reach vertex positions and attributes
(rasterizer.py:173-186), exactly as the reference recomputes them in MLX.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .. import _lib
from ..cameras import Camera
from ..splatting.tiles import bin_gaussians

__all__ = ["Fragments", "interpolate_face_attributes", "rasterize_meshes"]

_EPS = 1e-12


@dataclass
class Fragments:
    """Per-pixel rasterizer output (rasterizer.py:89-103): ``pix_to_face``
    (H, W) int32 (-1 empty), ``zbuf`` (H, W) camera depth (0 empty), ``bary``
    (H, W, 3) differentiable barycentrics, ``valid`` (H, W) bool,
    ``vert_ids`` (H, W, 3) vertex indices of the hit face."""

    pix_to_face: torch.Tensor
    zbuf: torch.Tensor
    bary: torch.Tensor
    valid: torch.Tensor
    vert_ids: torch.Tensor


def _as_verts_faces(mesh_or_verts, faces):
    if hasattr(mesh_or_verts, "verts_packed"):
        if len(mesh_or_verts) != 1:
            raise ValueError("rasterize_meshes renders one mesh at a time.")
        return mesh_or_verts.verts_packed(), mesh_or_verts.faces_packed()
    if faces is None:
        raise ValueError("faces must be provided when verts are passed directly.")
    return mesh_or_verts, faces


def rasterize_meshes(camera: Camera, mesh_or_verts, faces=None) -> Fragments:
    """Rasterize one triangle mesh to per-pixel :class:`Fragments`
    (rasterizer.py:121-194).  ``mesh_or_verts``: (V, 3) vertices on the GPU
    (or an object with ``verts_packed`` / ``faces_packed``); ``faces`` (F, 3)."""
    verts, faces_idx = _as_verts_faces(mesh_or_verts, faces)
    dev = _lib.require_device(verts)
    faces_idx = torch.as_tensor(faces_idx, device=dev).long()
    if verts.ndim != 2 or verts.shape[1] != 3 or faces_idx.ndim != 2 or faces_idx.shape[1] != 3:
        raise ValueError("verts must be (V, 3) and faces (F, 3).")
    h, w = int(camera.height), int(camera.width)
    xy, z = camera.project_points(verts.to(torch.float32))
    tri_xy = xy[faces_idx]
    tri_z = z[faces_idx]
    sxy = tri_xy.detach()
    centroid = sxy.mean(dim=1)
    radii = torch.sqrt(((sxy - centroid[:, None, :]) ** 2).sum(-1).max(dim=1).values)
    depths = tri_z.detach().mean(dim=1)
    sorted_ids, tile_ranges, _, _ = bin_gaussians(centroid.contiguous(), radii.contiguous(),
                                                  depths.contiguous(), w, h)
    pix_to_face = torch.empty((h, w), dtype=torch.int32, device=dev)
    zbuf = torch.empty((h, w), dtype=torch.float32, device=dev)
    txy = sxy.reshape(-1, 6).contiguous()
    tz = tri_z.detach().reshape(-1, 3).contiguous()
    ids = sorted_ids.to(torch.int32).contiguous()
    ranges = tile_ranges.to(torch.int32).contiguous()
    _lib.check(_lib.load().gsx_mesh_raster(
        faces_idx.shape[0], _lib.ptr(txy), _lib.ptr(tz), _lib.ptr(ids), ids.numel(),
        _lib.ptr(ranges), w, h, float(camera.znear), _lib.ptr(pix_to_face), _lib.ptr(zbuf),
        _lib.stream_handle(dev)), "gsx_mesh_raster")
    valid = pix_to_face >= 0
    fidx = torch.where(valid, pix_to_face, torch.zeros_like(pix_to_face)).long()
    vert_ids = faces_idx[fidx]
    tri = xy[vert_ids]
    ax, ay = tri[..., 0, 0], tri[..., 0, 1]
    bx, by = tri[..., 1, 0], tri[..., 1, 1]
    cxv, cyv = tri[..., 2, 0], tri[..., 2, 1]
    px = (torch.arange(w, dtype=torch.float32, device=dev) + 0.5)[None, :]
    py = (torch.arange(h, dtype=torch.float32, device=dev) + 0.5)[:, None]
    denom = (by - cyv) * (ax - cxv) + (cxv - bx) * (ay - cyv)
    denom = torch.where(denom.abs() < _EPS, torch.ones_like(denom), denom)
    l0 = ((by - cyv) * (px - cxv) + (cxv - bx) * (py - cyv)) / denom
    l1 = ((cyv - ay) * (px - cxv) + (ax - cxv) * (py - cyv)) / denom
    l2 = 1.0 - l0 - l1
    bary = torch.stack([l0, l1, l2], dim=-1) * valid[..., None]
    return Fragments(pix_to_face=pix_to_face, zbuf=zbuf, bary=bary, valid=valid,
                     vert_ids=vert_ids)


def interpolate_face_attributes(frag: Fragments, attrs: torch.Tensor) -> torch.Tensor:
    """(H, W, C) barycentric interpolation of (V, C) vertex values, zero on
    empty pixels (rasterizer.py:209-226); differentiable in ``attrs`` and the
    vertex positions."""
    tri_attr = attrs[frag.vert_ids]
    return (frag.bary[..., None] * tri_attr).sum(dim=-2) * frag.valid[..., None]
