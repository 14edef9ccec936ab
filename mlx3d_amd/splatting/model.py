"""The Gaussian scene representation (``src/mlx3d/splatting/model.py:16-207``).

Raw parameters live in ``self.params`` (torch tensors): ``means`` (N, 3),
``scales`` (N, 3) log-sigma, ``quats`` (N, 4) wxyz unnormalised,
``opacities`` (N,) logits, ``sh_dc`` (N, 1, 3), ``sh_rest`` (N, K-1, 3).
``render`` hands the raw tensors to the fused kernels, which apply
exp / sigmoid and read ``sh_dc`` / ``sh_rest`` in place (the reference
materialises ``exp``, ``sigmoid`` and the (N, K, 3) concatenation per call,
model.py:116-126).
"""

from __future__ import annotations

import math

import torch

from .. import _lib
from ..cameras import Camera
from .render import _check_common, _run
from .sh import num_sh_bases, rgb_to_sh

__all__ = ["GaussianModel"]


def _knn_mean_sq(points: torch.Tensor, ref: torch.Tensor, k: int, chunk: int) -> torch.Tensor:
    """Mean squared distance to the k-1 nearest neighbours (skipping a
    zero-distance self hit), as model.py:81-88 derives it from knn_points."""
    out = []
    r2 = (ref * ref).sum(-1)
    for s in range(0, points.shape[0], chunk):
        p = points[s:s + chunk]
        d = (p * p).sum(-1, keepdim=True) - 2.0 * p @ ref.T + r2[None]
        d = torch.clamp(d, min=0.0)
        vals, _ = torch.topk(d, k, dim=1, largest=False, sorted=True)
        self_hit = vals[:, 0] <= 1e-12
        nearest = torch.where(self_hit[:, None], vals[:, 1:k], vals[:, :k - 1])
        out.append(torch.clamp(nearest.mean(-1), min=1e-8))
    return torch.cat(out)


class GaussianModel:
    """A scene of 3D Gaussians with the standard 3DGS parameterisation."""

    def __init__(self, params: dict[str, torch.Tensor], sh_degree: int = 3):
        self.params = params
        self.sh_degree = sh_degree
        # Active degree grows during training (model.py:32-33).
        self.active_sh_degree = 0

    @classmethod
    def from_points(cls, points, colors=None, sh_degree: int = 3, initial_opacity: float = 0.1,
                    scale_init_max_ref: int = 10_000, scale_init_chunk_size: int = 1024,
                    scale_init_max_scale: float | None = None,
                    generator: torch.Generator | None = None) -> "GaussianModel":
        """Initialise from a point cloud (model.py:37-106): isotropic scales
        from the mean squared distance to the 3 nearest neighbours, identity
        rotations, opacity ``initial_opacity``, DC colour from ``colors``."""
        points = torch.as_tensor(points, dtype=torch.float32)
        N = points.shape[0]
        dev = points.device
        if colors is None:
            colors = torch.full((N, 3), 0.5, device=dev)
        colors = torch.as_tensor(colors, dtype=torch.float32, device=dev)
        ref_count = min(N, max(1, int(scale_init_max_ref)))
        if N > ref_count:
            perm = torch.randperm(N, generator=generator)[:ref_count].to(dev)
            ref = points[perm]
        else:
            ref = points
        if ref_count <= 1:
            mean_sq = torch.full((N,), 1e-8, device=dev)
        else:
            mean_sq = _knn_mean_sq(points, ref, min(4, ref_count), scale_init_chunk_size)
        scales = torch.log(torch.sqrt(mean_sq))[:, None] * torch.ones((1, 3), device=dev)
        if scale_init_max_scale is not None:
            scales = torch.clamp(scales, max=math.log(max(scale_init_max_scale, 1e-8)))
        quats = torch.zeros((N, 4), device=dev)
        quats[:, 0] = 1.0
        K = num_sh_bases(sh_degree)
        params = {
            "means": points.clone(),
            "scales": scales,
            "quats": quats,
            "opacities": torch.full((N,), math.log(initial_opacity / (1 - initial_opacity)),
                                    device=dev),
            "sh_dc": rgb_to_sh(colors)[:, None, :].contiguous(),
            "sh_rest": torch.zeros((N, K - 1, 3), device=dev),
        }
        return cls(params, sh_degree=sh_degree)

    # ------------------------------------------------------------ access
    @property
    def num_gaussians(self) -> int:
        return self.params["means"].shape[0]

    def __len__(self) -> int:
        return self.num_gaussians

    @property
    def scales_act(self) -> torch.Tensor:
        return torch.exp(self.params["scales"])

    @property
    def opacities_act(self) -> torch.Tensor:
        return torch.sigmoid(self.params["opacities"])

    @property
    def sh(self) -> torch.Tensor:
        return torch.cat([self.params["sh_dc"], self.params["sh_rest"]], dim=1)

    def to(self, device) -> "GaussianModel":
        self.params = {k: v.detach().to(device).requires_grad_(v.requires_grad)
                       for k, v in self.params.items()}
        return self

    def requires_grad_(self, flag: bool = True) -> "GaussianModel":
        for v in self.params.values():
            v.requires_grad_(flag)
        return self

    def parameters(self):
        return list(self.params.values())

    def one_up_sh_degree(self) -> None:
        if self.active_sh_degree < self.sh_degree:
            self.active_sh_degree += 1

    # ------------------------------------------------------------ render
    def _raw(self):
        p = self.params
        return p["means"], p["quats"], p["scales"], p["opacities"]

    def render(self, camera: Camera, background=None, antialias: bool = False,
               projection: str = "ewa", return_depth: bool = False) -> dict:
        """Render with the active SH degree (model.py:146-164)."""
        _check_common(projection)
        means, quats, scales, opac = self._raw()
        K = self.params["sh_dc"].shape[1] + self.params["sh_rest"].shape[1]
        return _run(camera, means, quats, scales, opac, sh_a=self.params["sh_dc"],
                    sh_b=self.params["sh_rest"], sh_mode="split", K=K,
                    degree=self.active_sh_degree, background=background,
                    flags=_lib.LOG_SCALES | _lib.LOGIT_OPACITY, antialias=antialias,
                    return_depth=return_depth)

    def render_depth(self, camera: Camera, antialias: bool = False,
                     projection: str = "ewa") -> dict:
        """Expected depth, forward only (model.py:166-180)."""
        _check_common(projection)
        means, quats, scales, opac = self._raw()
        with torch.no_grad():
            zeros = torch.zeros((means.shape[0], 1), dtype=torch.float32, device=means.device)
            out = _run(camera, means, quats, scales, opac, colors=zeros,
                       flags=_lib.LOG_SCALES | _lib.LOGIT_OPACITY, antialias=antialias,
                       return_depth=True)
        return {"depth": out["depth"], "alpha": out["alpha"], "final_T": out["final_T"],
                "means2d": out["means2d"], "depths": out["depths"], "radii": out["radii"],
                "compensation": out["compensation"]}

    def render_features(self, camera: Camera, features, background=None, normalize: bool = False,
                        antialias: bool = False, projection: str = "ewa") -> dict:
        """Render per-Gaussian features (model.py:182-203)."""
        from .render import render_gaussian_features

        return render_gaussian_features(camera, self.params["means"], self.params["quats"],
                                        self.scales_act, self.opacities_act, features,
                                        background=background, normalize=normalize,
                                        antialias=antialias, projection=projection)
