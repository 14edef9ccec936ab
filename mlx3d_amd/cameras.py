"""Cameras in the OpenCV convention (x right, y down, z forward).

Mirrors the parts of ``mlx3d.cameras`` the splatting path consumes
(``src/mlx3d/cameras/cameras.py:32-34, 42-113, 139-336``): ``Camera`` with
its lens model (orthographic, Brown-Conrady or fisheye distortion, used by
the UT projection), ``look_at``, ``fov_to_focal``, ``Camera.from_fov``,
``Camera.look_at``, ``Camera.orthographic_camera``, ``camera_center``,
``project_points`` and ``unproject_points``.  ``R`` and ``t`` are float32
CPU tensors, as the reference keeps them as float32 arrays; the intrinsics
are Python floats.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

__all__ = ["Camera", "look_at", "fov_to_focal", "focal_to_fov"]


def fov_to_focal(fov: float, pixels: int) -> float:
    """Focal length in pixels from a field of view in radians (cameras.py:32-34)."""
    return pixels / (2.0 * math.tan(fov / 2.0))


def focal_to_fov(focal: float, pixels: int) -> float:
    return 2.0 * math.atan(pixels / (2.0 * focal))


def _as_f32(v) -> np.ndarray:
    if isinstance(v, torch.Tensor):
        v = v.detach().cpu().numpy()
    return np.asarray(v, dtype=np.float32)


def _norm32(v: np.ndarray) -> np.float32:
    s = np.float32(0.0)
    for c in v:
        s = np.float32(s + np.float32(c * c))
    return np.float32(np.sqrt(s))


def _brown_distort(x, y, c):
    """Brown-Conrady distortion of normalised coordinates, c = (k1, k2, p1, p2[, k3])
    (cameras.py:42-51)."""
    k1, k2, p1, p2 = c[0], c[1], c[2], c[3]
    k3 = c[4] if len(c) > 4 else 0.0
    r2 = x * x + y * y
    radial = 1.0 + r2 * (k1 + r2 * (k2 + r2 * k3))
    xd = x * radial + 2.0 * p1 * x * y + p2 * (r2 + 2.0 * x * x)
    yd = y * radial + p1 * (r2 + 2.0 * y * y) + 2.0 * p2 * x * y
    return xd, yd


def _brown_undistort(xd, yd, c, iters: int = 8):
    """Fixed-point inversion of the Brown-Conrady model (cameras.py:54-66)."""
    k1, k2, p1, p2 = c[0], c[1], c[2], c[3]
    k3 = c[4] if len(c) > 4 else 0.0
    x, y = xd, yd
    for _ in range(iters):
        r2 = x * x + y * y
        radial = 1.0 + r2 * (k1 + r2 * (k2 + r2 * k3))
        dx = 2.0 * p1 * x * y + p2 * (r2 + 2.0 * x * x)
        dy = p1 * (r2 + 2.0 * y * y) + 2.0 * p2 * x * y
        x = (xd - dx) / radial
        y = (yd - dy) / radial
    return x, y


def _fisheye_distort(x, y, c, eps: float = 1e-9):
    """OpenCV equidistant fisheye, c = (k1, k2, k3, k4) (cameras.py:69-77)."""
    k1, k2, k3, k4 = (list(c) + [0.0, 0.0, 0.0, 0.0])[:4]
    r = torch.sqrt(x * x + y * y)
    theta = torch.atan(r)
    th2 = theta * theta
    theta_d = theta * (1.0 + th2 * (k1 + th2 * (k2 + th2 * (k3 + th2 * k4))))
    scale = theta_d / torch.clamp(r, min=eps)
    return x * scale, y * scale


def _fisheye_undistort(xd, yd, c, iters: int = 8, eps: float = 1e-9):
    """Fixed-point inversion of the fisheye model (cameras.py:80-91)."""
    k1, k2, k3, k4 = (list(c) + [0.0, 0.0, 0.0, 0.0])[:4]
    theta_d = torch.sqrt(xd * xd + yd * yd)
    theta = theta_d
    for _ in range(iters):
        th2 = theta * theta
        theta = theta_d / (1.0 + th2 * (k1 + th2 * (k2 + th2 * (k3 + th2 * k4))))
    scale = torch.tan(theta) / torch.clamp(theta_d, min=eps)
    return xd * scale, yd * scale


def look_at(eye, at, up) -> tuple[torch.Tensor, torch.Tensor]:
    """OpenCV extrinsics ``(R, t)`` with ``X_cam = R X_world + t`` (cameras.py:94-113).

    z = normalize(at - eye), x = normalize(z x up), y = z x x, R = [x; y; z],
    t = -R eye, all in float32.
    """
    eye, at, up = _as_f32(eye), _as_f32(at), _as_f32(up)
    z = (at - eye).astype(np.float32)
    z = (z / _norm32(z)).astype(np.float32)
    x = np.cross(z, up).astype(np.float32)
    x = (x / _norm32(x)).astype(np.float32)
    y = np.cross(z, x).astype(np.float32)
    R = np.stack([x, y, z], axis=0).astype(np.float32)
    t = -(R @ eye).astype(np.float32)
    return torch.from_numpy(R.copy()), torch.from_numpy(t.astype(np.float32).copy())


@dataclass
class Camera:
    """A camera (cameras.py:139-173).

    Attributes:
        R: (3, 3) world-to-camera rotation.  t: (3,) translation.
        fx, fy, cx, cy: intrinsics in pixels.  width, height: image size.
        znear, zfar: clipping range (only ``znear`` culls Gaussians).
        orthographic: parallel projection, ``fx``/``fy`` in pixels per world
            unit.  distortion: Brown-Conrady ``(k1, k2, p1, p2[, k3])``, or
            fisheye ``(k1, k2, k3, k4)`` with ``fisheye=True``.  The lens
            model is honoured by ``project_points`` and the UT projection;
            the EWA projection is pinhole, as in the reference.
    """

    R: torch.Tensor
    t: torch.Tensor
    fx: float
    fy: float
    cx: float
    cy: float
    width: int
    height: int
    znear: float = 0.01
    zfar: float = 100.0
    orthographic: bool = False
    distortion: tuple | None = None
    fisheye: bool = False

    def __post_init__(self):
        self.R = torch.as_tensor(_as_f32(self.R)).reshape(3, 3)
        self.t = torch.as_tensor(_as_f32(self.t)).reshape(3)
        if self.distortion is not None:
            self.distortion = tuple(float(v) for v in self.distortion)
            n = len(self.distortion)
            if (self.fisheye and n > 4) or (not self.fisheye and n not in (4, 5)):
                raise ValueError("distortion must be (k1, k2, p1, p2[, k3]) or, with "
                                 "fisheye=True, up to (k1, k2, k3, k4).")

    @classmethod
    def orthographic_camera(cls, scale: float, width: int, height: int, R=None, t=None,
                            **kwargs) -> "Camera":
        """Orthographic camera whose view spans [-scale, scale] world units
        vertically (cameras.py:174-207)."""
        ppwu = (height / 2.0) / float(scale)
        if R is None:
            R = torch.eye(3)
        if t is None:
            t = torch.zeros(3)
        return cls(R=R, t=t, fx=ppwu, fy=ppwu, cx=width / 2.0, cy=height / 2.0, width=width,
                   height=height, orthographic=True, **kwargs)

    @classmethod
    def from_fov(cls, fov: float, width: int, height: int, R=None, t=None, degrees: bool = True,
                 **kwargs) -> "Camera":
        """Camera from a vertical field of view (cameras.py:209-239)."""
        if degrees:
            fov = math.radians(fov)
        f = fov_to_focal(fov, height)
        if R is None:
            R = torch.eye(3)
        if t is None:
            t = torch.zeros(3)
        return cls(R=R, t=t, fx=f, fy=f, cx=width / 2.0, cy=height / 2.0, width=width,
                   height=height, **kwargs)

    @classmethod
    def look_at(cls, eye, at=(0.0, 0.0, 0.0), up=(0.0, 1.0, 0.0), fov: float = 60.0,
                width: int = 512, height: int = 512, degrees: bool = True,
                **kwargs) -> "Camera":
        """Camera at ``eye`` looking at ``at`` (cameras.py:241-255)."""
        R, t = look_at(eye, at, up)
        return cls.from_fov(fov, width, height, R=R, t=t, degrees=degrees, **kwargs)

    @property
    def K(self) -> torch.Tensor:
        return torch.tensor([[self.fx, 0.0, self.cx], [0.0, self.fy, self.cy], [0.0, 0.0, 1.0]])

    @property
    def fov_x(self) -> float:
        return focal_to_fov(self.fx, self.width)

    @property
    def fov_y(self) -> float:
        return focal_to_fov(self.fy, self.height)

    @property
    def camera_center(self) -> torch.Tensor:
        """-(R^T t) in float32 (cameras.py:270-273), summed in index order."""
        R = self.R.numpy().astype(np.float32)
        t = self.t.numpy().astype(np.float32)
        c = np.zeros(3, np.float32)
        for j in range(3):
            s = np.float32(R[0, j] * t[0])
            s = np.float32(s + np.float32(R[1, j] * t[1]))
            s = np.float32(s + np.float32(R[2, j] * t[2]))
            c[j] = -s
        return torch.from_numpy(c)

    def world_to_camera(self, points: torch.Tensor) -> torch.Tensor:
        """X_cam = X R^T + t for (..., 3) points (cameras.py:282-284)."""
        R = self.R.to(points.device)
        return points @ R.T + self.t.to(points.device)

    def camera_to_world(self, points: torch.Tensor) -> torch.Tensor:
        """(X_cam - t) R (cameras.py:286-288)."""
        return (points - self.t.to(points.device)) @ self.R.to(points.device)

    def _distort(self, x, y):
        if self.distortion is None:
            return x, y
        if self.fisheye:
            return _fisheye_distort(x, y, self.distortion)
        return _brown_distort(x, y, self.distortion)

    def _undistort(self, x, y):
        if self.distortion is None:
            return x, y
        if self.fisheye:
            return _fisheye_undistort(x, y, self.distortion)
        return _brown_undistort(x, y, self.distortion)

    def project_points(self, points: torch.Tensor, eps: float = 1e-8):
        """World points (..., 3) to (pixel coordinates (..., 2), camera z (...,))
        (cameras.py:290-311)."""
        pc = self.world_to_camera(points)
        z = pc[..., 2]
        if self.orthographic:
            u = self.fx * pc[..., 0] + self.cx
            v = self.fy * pc[..., 1] + self.cy
            return torch.stack([u, v], dim=-1), z
        inv_z = 1.0 / torch.where(z.abs() < eps, torch.full_like(z, eps), z)
        x, y = self._distort(pc[..., 0] * inv_z, pc[..., 1] * inv_z)
        return torch.stack([self.fx * x + self.cx, self.fy * y + self.cy], dim=-1), z

    def unproject_points(self, xy: torch.Tensor, depth: torch.Tensor) -> torch.Tensor:
        """Pixel coordinates (..., 2) with z-depths (...,) to world points
        (cameras.py:327-336)."""
        x = (xy[..., 0] - self.cx) / self.fx
        y = (xy[..., 1] - self.cy) / self.fy
        if self.orthographic:
            return self.camera_to_world(torch.stack([x, y, depth], dim=-1))
        x, y = self._undistort(x, y)
        return self.camera_to_world(torch.stack([x * depth, y * depth, depth], dim=-1))

    def gsx_fields(self) -> dict:
        """The float32 values the rasterizer's arithmetic sees.

        The reference multiplies float32 arrays by the Python-float
        intrinsics, which rounds them to float32; the frustum clip bound
        ``1.3 * (0.5 * width / fx)`` is formed in double and rounded once
        (projection.py:70-73).
        """
        return dict(
            R=self.R.numpy().astype(np.float32).reshape(9),
            t=self.t.numpy().astype(np.float32).reshape(3),
            center=self.camera_center.numpy(),
            fx=float(np.float32(self.fx)),
            fy=float(np.float32(self.fy)),
            cx=float(np.float32(self.cx)),
            cy=float(np.float32(self.cy)),
            lim_x=float(np.float32(1.3 * (0.5 * self.width / self.fx))),
            lim_y=float(np.float32(1.3 * (0.5 * self.height / self.fy))),
            znear=float(np.float32(self.znear)),
            width=int(self.width),
            height=int(self.height),
            orthographic=int(bool(self.orthographic)),
            lens=self._lens_code(),
            dist=self._lens_coefficients(),
        )

    def _lens_code(self) -> int:
        if self.distortion is None:
            return 0
        return 2 if self.fisheye else 1

    def _lens_coefficients(self) -> list[float]:
        """The float32 constants of the lens formulas: Brown k1 k2 p1 p2 k3 and
        2 p1, 2 p2 (products of Python floats, rounded once); fisheye k1..k4."""
        d = [0.0] * 8
        if self.distortion is None:
            return d
        c = list(self.distortion)
        if self.fisheye:
            c = (c + [0.0] * 4)[:4]
            d[:4] = c
        else:
            k3 = c[4] if len(c) > 4 else 0.0
            d[:7] = [c[0], c[1], c[2], c[3], k3, 2.0 * c[2], 2.0 * c[3]]
        return [float(np.float32(v)) for v in d]

    def to_gsx(self):
        """ctypes ``gsx_camera`` for the C ABI."""
        from ._lib import GsxCamera

        f = self.gsx_fields()
        cam = GsxCamera()
        cam.R[:] = [float(v) for v in f["R"]]
        cam.t[:] = [float(v) for v in f["t"]]
        cam.center[:] = [float(v) for v in f["center"]]
        for k in ("fx", "fy", "cx", "cy", "lim_x", "lim_y", "znear", "width", "height",
                  "orthographic", "lens"):
            setattr(cam, k, f[k])
        cam.dist[:] = f["dist"]
        return cam
