"""2DGS geometry regularisers on the device (``gsx_geom_*`` kernels).

The 2DGS training method (splatting/trainer.py:187-259) renders per-Gaussian
(depth, depth^2, surfel normal) features, normalised by alpha, and
penalises

- the ray-depth variance E[z^2] - E[z]^2 where alpha > min_alpha, and
- the disagreement 1 - |n_render . n_depth| between the rendered normal and
  the normal of the surface spanned by the expected depths, over 2x2 pixel
  quads whose four pixels pass the alpha test.

:func:`surfel_features` and :func:`geometry_loss` are autograd functions
over the kernels; :func:`unprojection_maps` gives the per-pixel affine
unprojection P = base + z dir the loss kernels use for any camera model.
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from .. import _lib
from ..cameras import Camera

__all__ = ["surfel_features", "geometry_loss", "unprojection_maps"]


class _SurfelFeatures(torch.autograd.Function):
    @staticmethod
    def forward(ctx, means, quats, depths, center):
        dev = _lib.require_device(means, quats, depths)
        n = means.shape[0]
        out = torch.empty((n, 5), dtype=torch.float32, device=dev)
        c = np.ascontiguousarray(center, np.float32)
        _lib.check(_lib.load().gsx_geom_features(
            n, _lib.ptr(means), _lib.ptr(quats), _lib.ptr(depths),
            c.ctypes.data_as(ctypes.c_void_p), _lib.ptr(out), _lib.stream_handle(dev)),
            "gsx_geom_features")
        ctx.save_for_backward(means, quats, depths)
        ctx.center = c
        return out

    @staticmethod
    def backward(ctx, g_out):
        means, quats, depths = ctx.saved_tensors
        dev = means.device
        n = means.shape[0]
        g = _lib.f32c(g_out)
        g_depths = torch.empty((n,), dtype=torch.float32, device=dev)
        g_quats = torch.empty((n, 4), dtype=torch.float32, device=dev)
        c = ctx.center
        _lib.check(_lib.load().gsx_geom_features_bwd(
            n, _lib.ptr(means), _lib.ptr(quats), _lib.ptr(depths),
            c.ctypes.data_as(ctypes.c_void_p), _lib.ptr(g), _lib.ptr(g_depths),
            _lib.ptr(g_quats), _lib.stream_handle(dev)), "gsx_geom_features_bwd")
        return None, g_quats, g_depths, None


def surfel_features(means: torch.Tensor, quats: torch.Tensor, depths: torch.Tensor,
                    camera: Camera) -> torch.Tensor:
    """(N, 5) = (z, z^2, normal facing the camera); differentiable w.r.t.
    quats and depths (the facing flip is a sign and carries no gradient)."""
    center = camera.camera_center.detach().cpu().numpy().astype(np.float32)
    return _SurfelFeatures.apply(_lib.f32c(means.detach()), _lib.f32c(quats),
                                 _lib.f32c(depths), center)


def unprojection_maps(camera: Camera, device) -> tuple[torch.Tensor, torch.Tensor]:
    """(base, dir), (H, W, 3) each: the world point of pixel centre (x+0.5,
    y+0.5) at z-depth z is base + z dir (Camera.unproject_points is affine in
    the depth for every lens model)."""
    H, W = int(camera.height), int(camera.width)
    u = torch.arange(W, dtype=torch.float32) + 0.5
    v = torch.arange(H, dtype=torch.float32) + 0.5
    uv = torch.stack([u[None, :].expand(H, W), v[:, None].expand(H, W)], dim=-1)
    at0 = camera.unproject_points(uv, torch.zeros((H, W)))
    at1 = camera.unproject_points(uv, torch.ones((H, W)))
    return (at0.to(torch.float32).contiguous().to(device),
            (at1 - at0).to(torch.float32).contiguous().to(device))


class _GeometryLoss(torch.autograd.Function):
    @staticmethod
    def forward(ctx, F, alpha, base, dirs, min_alpha, lam_dv, lam_nc):
        dev = _lib.require_device(F, alpha, base, dirs)
        H, W = alpha.shape
        L = _lib.load()
        ws = torch.empty(int(L.gsx_geom_loss_workspace_bytes(W, H)), dtype=torch.uint8,
                         device=dev)
        out = torch.empty(5, dtype=torch.float32, device=dev)
        _lib.check(L.gsx_geom_loss_fwd(W, H, _lib.ptr(F), _lib.ptr(alpha), _lib.ptr(base),
                                       _lib.ptr(dirs), min_alpha, lam_dv, lam_nc, _lib.ptr(ws),
                                       ws.numel(), _lib.ptr(out), _lib.stream_handle(dev)),
                   "gsx_geom_loss_fwd")
        ctx.save_for_backward(F, alpha, base, dirs, out)
        ctx.args = (min_alpha, lam_dv, lam_nc)
        metrics = out[1:3].clone()
        ctx.mark_non_differentiable(metrics)
        return out[0].clone(), metrics

    @staticmethod
    def backward(ctx, g_loss, _g_metrics):
        F, alpha, base, dirs, out = ctx.saved_tensors
        min_alpha, lam_dv, lam_nc = ctx.args
        H, W = alpha.shape
        g = _lib.f32c(g_loss.reshape(1))
        g_F = torch.empty_like(F)
        _lib.check(_lib.load().gsx_geom_loss_bwd(
            W, H, _lib.ptr(F), _lib.ptr(alpha), _lib.ptr(base), _lib.ptr(dirs), min_alpha,
            lam_dv, lam_nc, _lib.ptr(out), _lib.ptr(g), _lib.ptr(g_F),
            _lib.stream_handle(F.device)), "gsx_geom_loss_bwd")
        return g_F, None, None, None, None, None, None


def geometry_loss(features: torch.Tensor, alpha: torch.Tensor, camera: Camera,
                  min_alpha: float, lambda_depth_variance: float,
                  lambda_normal_consistency: float, maps=None):
    """(loss, {"depth_variance", "normal_consistency"}) from the
    alpha-normalised (H, W, 5) feature render and alpha; differentiable
    w.r.t. ``features`` (the alpha test is a step: no gradient).  ``maps``
    = unprojection_maps(camera, device) when already at hand."""
    dev = features.device
    base, dirs = maps if maps is not None else unprojection_maps(camera, dev)
    loss, metrics = _GeometryLoss.apply(_lib.f32c(features), _lib.f32c(alpha.detach()),
                                           base, dirs, float(min_alpha),
                                           float(lambda_depth_variance),
                                           float(lambda_normal_consistency))
    return loss, {"depth_variance": metrics[0], "normal_consistency": metrics[1]}
