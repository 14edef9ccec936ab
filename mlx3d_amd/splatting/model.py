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

import numpy as np
import torch

from .. import _lib
from ..cameras import Camera
from .render import _check_common, _run
from .sh import num_sh_bases, rgb_to_sh

__all__ = ["GaussianModel"]


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
                    generator: torch.Generator | None = None,
                    device=None) -> "GaussianModel":
        """A table initialised from a point cloud (model.py:37-106).

        Isotropic log-scales come from ``gsx_knn_log_scale`` on the GPU: the
        mean squared distance to the 3 nearest of at most
        ``scale_init_max_ref`` reference points (a random subset of a larger
        cloud, drawn with ``generator``), a self hit skipped, optionally capped
        at ``scale_init_max_scale``.  Rotations are the identity, opacity
        logits ``logit(initial_opacity)``, the DC colour ``rgb_to_sh(colors)``
        (grey without colours) and higher SH bands zero.  The table lives on
        ``device`` (default: the GPU).  ``scale_init_chunk_size`` bounded the
        reference's query chunks; the kernel streams the reference points, so
        it is accepted and unused."""
        from .density import knn_log_scales

        dev = torch.device(device if device is not None else "cuda")
        pts = torch.as_tensor(points, dtype=torch.float32).to(dev).contiguous()
        if pts.ndim != 2 or pts.shape[1] != 3:
            raise ValueError("points must have shape (N, 3).")
        count = pts.shape[0]
        rgb = (torch.full((count, 3), 0.5, device=dev) if colors is None
               else torch.as_tensor(colors, dtype=torch.float32).to(dev))
        n_ref = min(count, max(1, int(scale_init_max_ref)))
        if n_ref < count:
            pick = torch.randperm(count, generator=generator)[:n_ref].to(dev)
            ref = pts[pick].contiguous()
        else:
            ref = pts
        if n_ref <= 1:  # no neighbour: the reference's floor of 1e-8
            log_s = torch.full((count,), 0.5 * math.log(1e-8), device=dev)
            if scale_init_max_scale is not None:
                log_s = torch.clamp(log_s, max=math.log(max(scale_init_max_scale, 1e-8)))
        else:
            log_s = knn_log_scales(pts, ref, min(4, n_ref), scale_init_max_scale)
        K = num_sh_bases(sh_degree)
        quats = torch.zeros((count, 4), device=dev)
        quats[:, 0] = 1.0
        logit = math.log(initial_opacity / (1 - initial_opacity))
        params = {
            "means": pts.clone(),
            "scales": log_s[:, None].expand(count, 3).contiguous(),
            "quats": quats,
            "opacities": torch.full((count,), logit, device=dev),
            "sh_dc": rgb_to_sh(rgb)[:, None, :].contiguous(),
            "sh_rest": torch.zeros((count, K - 1, 3), device=dev),
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
        pflags = _check_common(projection)
        means, quats, scales, opac = self._raw()
        K = self.params["sh_dc"].shape[1] + self.params["sh_rest"].shape[1]
        return _run(camera, means, quats, scales, opac, sh_a=self.params["sh_dc"],
                    sh_b=self.params["sh_rest"], sh_mode="split", K=K,
                    degree=self.active_sh_degree, background=background,
                    flags=_lib.LOG_SCALES | _lib.LOGIT_OPACITY | pflags, antialias=antialias,
                    return_depth=return_depth)

    def render_depth(self, camera: Camera, antialias: bool = False,
                     projection: str = "ewa") -> dict:
        """Expected depth, forward only (model.py:166-180)."""
        pflags = _check_common(projection)
        means, quats, scales, opac = self._raw()
        with torch.no_grad():
            zeros = torch.zeros((means.shape[0], 1), dtype=torch.float32, device=means.device)
            out = _run(camera, means, quats, scales, opac, colors=zeros,
                       flags=_lib.LOG_SCALES | _lib.LOGIT_OPACITY | pflags, antialias=antialias,
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

    # ------------------------------------------------------------ checkpoints
    def ply_properties(self) -> list[str]:
        """Vertex properties of the standard 3DGS PLY layout, in file order
        (model.py:338-361): x y z nx ny nz f_dc_0..2 f_rest_* opacity
        scale_0..2 rot_0..3."""
        n_rest = 3 * self.params["sh_rest"].shape[1]
        return (["x", "y", "z", "nx", "ny", "nz", "f_dc_0", "f_dc_1", "f_dc_2"]
                + [f"f_rest_{i}" for i in range(n_rest)] + ["opacity"]
                + [f"scale_{i}" for i in range(3)] + [f"rot_{i}" for i in range(4)])

    def save_ply(self, path: str) -> None:
        """Save in the standard 3DGS PLY layout, binary little-endian
        (model.py:338-361): zero normals, ``f_rest`` channel-major.  The
        (N, P) float32 table is assembled on the device and written with one
        device-to-host copy; the bytes are those of ``io.save_ply`` with
        these properties."""
        import os

        p = {k: v.detach() for k, v in self.params.items()}
        n = self.num_gaussians
        rest = p["sh_rest"].transpose(1, 2).reshape(n, -1)  # channel-major (N, 3 (K-1))
        cols = [p["means"].reshape(n, 3), torch.zeros_like(p["means"]).reshape(n, 3),
                p["sh_dc"].reshape(n, 3), rest, p["opacities"].reshape(n, 1),
                p["scales"].reshape(n, 3), p["quats"].reshape(n, 4)]
        table = torch.cat([c.to(torch.float32) for c in cols], dim=1).cpu().numpy()
        header = ["ply", "format binary_little_endian 1.0", f"element vertex {n}"]
        header += [f"property float {k}" for k in self.ply_properties()]
        header.append("end_header")
        os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
        with open(path, "wb") as f:
            f.write(("\n".join(header) + "\n").encode("ascii"))
            f.write(np.ascontiguousarray(table, dtype="<f4").tobytes())

    @classmethod
    def load_ply(cls, path: str, sh_degree: int = 3, device=None) -> "GaussianModel":
        """Load a 3DGS-format PLY checkpoint (model.py:363-392); the SH degree
        follows the file when its f_rest count disagrees with ``sh_degree``,
        and the active degree is set to the full degree.  An all-float32
        binary file goes to ``device`` (default: the GPU when present) as one
        (N, P) copy and is split there; other files take the generic path."""
        from ..io import load_ply, read_ply_vertices

        if device is None:
            device = "cuda" if torch.cuda.is_available() else "cpu"
        try:
            names, table = read_ply_vertices(path)
            t = torch.from_numpy(table).to(device)
            idx = {k: i for i, k in enumerate(names)}

            def col(k):
                return t[:, idx[k]]
        except ValueError:
            data = load_ply(path)
            cols = dict(data.extra)
            cols["x"], cols["y"], cols["z"] = data.verts.unbind(-1)
            idx = cols

            def col(k):
                return cols[k].to(device)
        n_rest = len([k for k in idx if k.startswith("f_rest_")])
        K = num_sh_bases(sh_degree)
        if n_rest != 3 * (K - 1):
            K = n_rest // 3 + 1
            sh_degree = int(np.sqrt(K)) - 1
        stack = lambda ks: torch.stack([col(k) for k in ks], dim=-1)  # noqa: E731
        n = col("x").shape[0]
        if n_rest > 0:
            rest = stack([f"f_rest_{i}" for i in range(n_rest)])
            sh_rest = rest.reshape(n, 3, K - 1).transpose(1, 2)
        else:
            sh_rest = torch.zeros((n, K - 1, 3), device=device)
        params = {
            "means": stack(["x", "y", "z"]),
            "scales": stack([f"scale_{i}" for i in range(3)]),
            "quats": stack([f"rot_{i}" for i in range(4)]),
            "opacities": col("opacity"),
            "sh_dc": stack(["f_dc_0", "f_dc_1", "f_dc_2"])[:, None, :],
            "sh_rest": sh_rest,
        }
        model = cls({k: v.to(torch.float32).contiguous() for k, v in params.items()},
                    sh_degree=sh_degree)
        model.active_sh_degree = sh_degree
        return model

    # ------------------------------------------------------------ table edits
    # Row edits run on the device; each returns new leaf tensors that keep the
    # requires_grad flag of the ones they replace.
    def _replace(self, params: dict[str, torch.Tensor]) -> None:
        self.params = {k: v.detach().contiguous().requires_grad_(self.params[k].requires_grad)
                       for k, v in params.items()}

    def copy(self) -> "GaussianModel":
        """A detached copy of the table (model.py:273-277)."""
        out = GaussianModel({k: v.detach().clone() for k, v in self.params.items()},
                            self.sh_degree)
        out.active_sh_degree = self.active_sh_degree
        return out

    def select(self, keep_idx) -> None:
        """Keep only the rows ``keep_idx`` (model.py:395-398)."""
        idx = torch.as_tensor(np.asarray(keep_idx), dtype=torch.int64,
                              device=self.params["means"].device)
        with torch.no_grad():
            self._replace({k: v[idx] for k, v in self.params.items()})

    def reorder_spatial(self) -> torch.Tensor:
        """Store the rows in 3D Morton order of their means (``spatial_order``;
        no counterpart in the reference): Gaussians close in space share cache
        lines in the rasterizers' gathers.  Renders are unchanged except for
        Gaussians at exactly equal depths.  Returns the permutation (new row i
        was row ``perm[i]``)."""
        from .layout import spatial_order

        perm = spatial_order(self.params["means"])
        with torch.no_grad():
            self._replace({k: v[perm] for k, v in self.params.items()})
        return perm

    def append(self, new_params: dict[str, torch.Tensor]) -> None:
        """Concatenate rows (model.py:400-404)."""
        with torch.no_grad():
            self._replace({k: torch.cat([v, torch.as_tensor(new_params[k]).to(v)], dim=0)
                           for k, v in self.params.items()})

    def apply_2dgs_constraints(self, max_thickness: float) -> None:
        """Cap the third log-scale at log(max(thickness, 1e-8)) (model.py:128-143)."""
        lim = float(np.log(max(float(max_thickness), 1e-8)))
        with torch.no_grad():
            s = self.params["scales"]
            z = torch.clamp(s[:, 2:3], max=lim)
            params = dict(self.params)
            params["scales"] = torch.cat([s[:, :2], z], dim=1)
            self._replace(params)

    def reset_opacities(self, max_opacity: float = 0.01) -> None:
        """Clamp opacity logits to logit(max_opacity) (model.py:533-538)."""
        logit = float(np.log(max_opacity / (1 - max_opacity)))
        with torch.no_grad():
            params = dict(self.params)
            params["opacities"] = torch.clamp(self.params["opacities"], max=logit)
            self._replace(params)

    def compact(self, min_opacity: float = 0.0, max_gaussians: int | None = None,
                target_sh_degree: int | None = None) -> "GaussianModel":
        """A pruned copy ranked by sigmoid(opacity) max(scale)^2 (model.py:279-335)."""
        if max_gaussians is not None and max_gaussians <= 0:
            raise ValueError("max_gaussians must be positive when provided.")
        if target_sh_degree is not None and not (0 <= target_sh_degree <= self.sh_degree):
            raise ValueError("target_sh_degree must be between 0 and the model sh_degree.")
        n = self.num_gaussians
        if n == 0:
            return self.copy()
        with torch.no_grad():
            opacity = self.opacities_act
            max_scale = self.scales_act.max(dim=1).values
            importance = opacity * max_scale * max_scale
            keep = opacity >= float(min_opacity)
            if not bool(keep.any()):
                keep[int(torch.argmax(importance))] = True
            keep_idx = torch.nonzero(keep).flatten()
            if max_gaussians is not None and keep_idx.numel() > max_gaussians:
                top = torch.topk(importance[keep_idx], max_gaussians).indices
                keep_idx = torch.sort(keep_idx[top]).values
            params = {k: v.detach()[keep_idx].clone() for k, v in self.params.items()}
        sh_degree = self.sh_degree
        if target_sh_degree is not None:
            sh_degree = int(target_sh_degree)
            params["sh_rest"] = params["sh_rest"][:, :max(0, num_sh_bases(sh_degree) - 1), :]
        out = GaussianModel({k: v.contiguous() for k, v in params.items()}, sh_degree=sh_degree)
        out.active_sh_degree = min(self.active_sh_degree, sh_degree)
        return out

    def densify_and_prune(self, grad_accum: torch.Tensor, grad_count: torch.Tensor,
                          grad_threshold: float = 0.0002, scene_extent: float = 1.0,
                          percent_dense: float = 0.01, min_opacity: float = 0.005,
                          return_optimizer_state: bool = False, moments: dict | None = None
                          ) -> dict:
        """Adaptive density control of the 3DGS paper (model.py:406-480), on
        the device (``gsx_density_classify`` / ``gsx_density_emit``).

        A row whose average screen gradient exceeds ``grad_threshold`` is
        cloned when its largest scale is at most ``percent_dense *
        scene_extent`` and split otherwise: two samples N(0, diag(s^2))
        rotated by the Gaussian's rotation (drawn from ``np.random.normal``,
        the reference's generator and order), log-scales reduced by log 1.6.
        Split sources, rows with sigmoid(opacity) < ``min_opacity`` and rows
        larger than half the extent are pruned.  New row order: kept rows,
        clones, split pairs.  ``moments`` ({group: {"m", "v"}}) are edited
        alongside (zero in new rows) and returned under ``"_moments"``.
        """
        from .density import densify

        new, new_moments, stats, keep_idx = densify(
            self.params, grad_accum, grad_count, grad_threshold=grad_threshold,
            scene_extent=scene_extent, percent_dense=percent_dense, min_opacity=min_opacity,
            moments=moments)
        self._replace(new)
        if moments is not None:
            stats["_moments"] = new_moments
        if return_optimizer_state:
            stats["_keep_idx"] = keep_idx.cpu().numpy().astype(np.int32)
            stats["_new_count"] = int(stats["cloned"] + 2 * stats["split"])
        return stats

    def relocate_mcmc(self, grad_accum: torch.Tensor, grad_count: torch.Tensor,
                      relocate_frac: float = 0.02, min_opacity: float = 0.01,
                      jitter_scale: float = 0.25, generator: torch.Generator | None = None,
                      moments: dict | None = None) -> dict:
        """Fixed-budget MCMC relocation (model.py:482-531), in place on the
        device: up to ``relocate_frac`` N underused rows (sigmoid(opacity) <
        ``min_opacity`` or never seen; otherwise the least opaque) take
        jittered copies of the rows with the largest average screen gradient,
        opacity reset to 0.05 and log-scales shrunk by log 1.6.  ``moments``
        of the moved rows are cleared."""
        from .density import relocate

        with torch.no_grad():
            k, dst = relocate(self.params, grad_accum, grad_count, relocate_frac=relocate_frac,
                              min_opacity=min_opacity, jitter_scale=jitter_scale,
                              generator=generator, moments=moments)
        if k == 0:
            return {"relocated": 0}
        return {"relocated": int(k), "_moved_idx": dst}
