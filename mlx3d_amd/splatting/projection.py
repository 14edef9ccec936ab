"""Projection of 3D Gaussians (``src/mlx3d/splatting/projection.py``).

``project_gaussians`` (EWA, :24-146) runs ``gsx_project_fwd`` and
``project_gaussians_ut`` (unscented transform through the camera's lens
model, :149-205) ``gsx_project_ut_fwd``; their VJPs (what MLX autodiff
computes through the reference's expressions) are the ``_bwd`` entry
points.
"""

from __future__ import annotations

import torch

from .. import _lib
from ..cameras import Camera

__all__ = ["quat_scale_to_cov3d", "project_gaussians", "project_gaussians_ut"]


def quat_scale_to_cov3d(quats: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """3D covariances R diag(s)^2 R^T, (N, 3, 3), from (N, 4) wxyz quaternions
    (normalised here) and (N, 3) standard deviations (projection.py:17-21).
    Differentiable torch ops on the tensors' device; the render path never
    calls it (its kernels form the same covariance per Gaussian)."""
    from ..transforms import quaternion_to_matrix

    if quats.ndim != 2 or quats.shape[1] != 4 or scales.shape != (quats.shape[0], 3):
        raise ValueError("quats must be (N, 4) and scales (N, 3).")
    rs = quaternion_to_matrix(quats) * scales[:, None, :]  # columns scaled: R diag(s)
    return rs @ rs.transpose(1, 2).contiguous()


class _Project(torch.autograd.Function):
    @staticmethod
    def forward(ctx, means, quats, scales, cam, blur, antialias, ut=False):
        dev = _lib.require_device(means, quats, scales)
        n = means.shape[0]
        f = lambda *s: torch.empty(s, dtype=torch.float32, device=dev)  # noqa: E731
        means2d, conics, depths, radii, comp = f(n, 2), f(n, 3), f(n), f(n), f(n)
        L = _lib.load()
        fwd = L.gsx_project_ut_fwd if ut else L.gsx_project_fwd
        _lib.check(fwd(cam, n, _lib.ptr(means), _lib.ptr(quats), _lib.ptr(scales), blur,
                       int(antialias), _lib.ptr(means2d), _lib.ptr(conics), _lib.ptr(depths),
                       _lib.ptr(radii), _lib.ptr(comp), _lib.stream_handle(dev)),
                   "gsx_project_ut_fwd" if ut else "gsx_project_fwd")
        ctx.save_for_backward(means, quats, scales)
        ctx.cam, ctx.blur, ctx.antialias, ctx.ut = cam, blur, antialias, ut
        ctx.mark_non_differentiable(radii)
        ctx.set_materialize_grads(False)  # unused outputs: no zero-filled cotangents
        return means2d, conics, depths, radii, comp

    @staticmethod
    def backward(ctx, g_means2d, g_conics, g_depths, _g_radii, g_comp):
        means, quats, scales = ctx.saved_tensors
        n = means.shape[0]
        dev = means.device
        gm = torch.empty((n, 3), dtype=torch.float32, device=dev)
        gq = torch.empty((n, 4), dtype=torch.float32, device=dev)
        gs = torch.empty((n, 3), dtype=torch.float32, device=dev)
        c = lambda t: None if t is None else t.contiguous()  # noqa: E731
        g_means2d, g_conics, g_depths, g_comp = map(c, (g_means2d, g_conics, g_depths, g_comp))
        L = _lib.load()
        bwd = L.gsx_project_ut_bwd if ctx.ut else L.gsx_project_bwd
        _lib.check(bwd(ctx.cam, n, _lib.ptr(means), _lib.ptr(quats), _lib.ptr(scales), ctx.blur,
                       int(ctx.antialias), _lib.ptr(g_means2d), _lib.ptr(g_conics),
                       _lib.ptr(g_depths), _lib.ptr(g_comp), _lib.ptr(gm), _lib.ptr(gq),
                       _lib.ptr(gs), _lib.stream_handle(dev)),
                   "gsx_project_ut_bwd" if ctx.ut else "gsx_project_bwd")
        return gm, gq, gs, None, None, None, None


def _check(means, quats, scales):
    if means.ndim != 2 or means.shape[1] != 3:
        raise ValueError("means must have shape (N, 3).")
    if quats.shape != (means.shape[0], 4) or scales.shape != means.shape:
        raise ValueError("quats must be (N, 4) and scales (N, 3).")


def project_gaussians(camera: Camera, means: torch.Tensor, quats: torch.Tensor,
                      scales: torch.Tensor, blur: float = 0.3,
                      antialias: bool = False) -> dict[str, torch.Tensor]:
    """Project 3D Gaussians into screen space (projection.py:24-146).

    Args:
        camera: the viewing camera.
        means: (N, 3) centres; quats: (N, 4) wxyz rotations (need not be
            normalised); scales: (N, 3) per-axis standard deviations.
        blur: screen-space dilation added to the covariance diagonal.
        antialias: also return Mip-Splatting opacity compensation.

    Returns:
        ``means2d`` (N, 2), ``conics`` (N, 3), ``depths`` (N,), ``radii``
        (N,) (float, 0 for culled Gaussians) and ``compensation`` (N,).
    """
    _check(means, quats, scales)
    means2d, conics, depths, radii, comp = _Project.apply(
        _lib.f32c(means), _lib.f32c(quats), _lib.f32c(scales), camera.to_gsx(), float(blur),
        bool(antialias))
    return {"means2d": means2d, "conics": conics, "depths": depths, "radii": radii,
            "compensation": comp}


def project_gaussians_ut(camera: Camera, means: torch.Tensor, quats: torch.Tensor,
                         scales: torch.Tensor, blur: float = 0.3,
                         antialias: bool = False) -> dict[str, torch.Tensor]:
    """Project with a 3D unscented transform (projection.py:149-205): the
    six sigma points mean +- sqrt(3) R diag(s) e_k go through the camera's
    ``project_points`` (perspective or orthographic, Brown-Conrady or fisheye
    distortion), and their pixel mean and covariance replace the EWA
    Jacobian.  Same outputs as :func:`project_gaussians`; ``depths`` are the
    centres' camera-space z."""
    _check(means, quats, scales)
    means2d, conics, depths, radii, comp = _Project.apply(
        _lib.f32c(means), _lib.f32c(quats), _lib.f32c(scales), camera.to_gsx(), float(blur),
        bool(antialias), True)
    return {"means2d": means2d, "conics": conics, "depths": depths, "radii": radii,
            "compensation": comp}
