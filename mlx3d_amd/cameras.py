"""Pinhole cameras in the OpenCV convention (x right, y down, z forward).

Mirrors the parts of ``mlx3d.cameras`` the splatting path consumes
(``src/mlx3d/cameras/cameras.py:32-34, 94-113, 139-273``): ``Camera``,
``look_at``, ``fov_to_focal``, ``Camera.from_fov``, ``Camera.look_at`` and
``camera_center``.  ``R`` and ``t`` are float32 CPU tensors, as the
reference keeps them as float32 arrays; the intrinsics are Python floats.
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
    """A pinhole camera (cameras.py:139-173).

    Attributes:
        R: (3, 3) world-to-camera rotation.  t: (3,) translation.
        fx, fy, cx, cy: intrinsics in pixels.  width, height: image size.
        znear, zfar: clipping range (only ``znear`` culls Gaussians).
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

    def __post_init__(self):
        self.R = torch.as_tensor(_as_f32(self.R)).reshape(3, 3)
        self.t = torch.as_tensor(_as_f32(self.t)).reshape(3)

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

    def unproject_points(self, xy: torch.Tensor, depth: torch.Tensor) -> torch.Tensor:
        """Pixel coordinates (..., 2) with z-depths (...,) to world points
        (cameras.py:327-336, pinhole)."""
        x = (xy[..., 0] - self.cx) / self.fx
        y = (xy[..., 1] - self.cy) / self.fy
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
        )

    def to_gsx(self):
        """ctypes ``gsx_camera`` for the C ABI."""
        from ._lib import GsxCamera

        f = self.gsx_fields()
        cam = GsxCamera()
        cam.R[:] = [float(v) for v in f["R"]]
        cam.t[:] = [float(v) for v in f["t"]]
        cam.center[:] = [float(v) for v in f["center"]]
        for k in ("fx", "fy", "cx", "cy", "lim_x", "lim_y", "znear", "width", "height"):
            setattr(cam, k, f[k])
        return cam
