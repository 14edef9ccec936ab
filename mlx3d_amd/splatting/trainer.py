"""The training step around the rasterizer (``src/mlx3d/splatting/trainer.py``).

One ``GaussianTrainer.step`` on the vanilla and MCMC methods is

    fused render forward (preprocess, binning, raster)        libgsx
    photometric loss: mean L1 and mean SSIM in one pass       gsx_photometric_fwd
    backward: loss gradient, raster VJP (+ the screen-space    gsx_photometric_bwd,
      gradient statistics of density control), preprocess VJP  gsx_raster_bwd, ...
    Adam on all six parameter groups in one launch            gsx_adam_step

with no host synchronisation except the duplicate count of the binning;
density control runs every ``densify_every`` steps on the device.

The reference probes dL/dmeans2d by adding a zero (N, 2) array to means2d
(trainer.py:264-275, 325, 337); here the backward hands the rasterizer's
dL/dmeans2d straight to ``gsx_accum_screen_grads``.  The 2DGS method renders
through the separate drop-in stages (project, eval_sh, bin, rasterize,
rasterize_features) as the reference does, because its geometry losses
need the projected Gaussians; there the probe is the reference's own.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

from ..cameras import Camera
from ..losses import photometric
from ..optim import Adam, adam_step, exponential_decay
from ..transforms import quaternion_to_matrix
from .. import _lib
from .model import GaussianModel
from .projection import project_gaussians, project_gaussians_ut
from .rasterize import rasterize, rasterize_features
from .render import _check_common, _run
from .sh import eval_sh
from .tiles import bin_gaussians

__all__ = ["TrainerConfig", "GaussianTrainer"]

_GROUPS = ("means", "scales", "quats", "opacities", "sh_dc", "sh_rest")


@dataclass
class TrainerConfig:
    """Training hyper-parameters (trainer.py:27-75); same fields and defaults.
    ``low_memory`` and ``cache_limit_gb`` tune MLX's buffer cache and have no
    effect here."""

    method: str = "vanilla"
    lr_means: float = 1.6e-4
    lr_means_final: float = 1.6e-6
    lr_means_max_steps: int = 30_000
    lr_scales: float = 5e-3
    lr_quats: float = 1e-3
    lr_opacities: float = 5e-2
    lr_sh_dc: float = 2.5e-3
    lr_sh_rest: float = 2.5e-3 / 20.0
    lambda_dssim: float = 0.2
    antialias: bool = False
    projection: str = "ewa"
    lambda_2d_depth_variance: float = 0.0
    lambda_2d_normal_consistency: float = 0.0
    geometry_min_alpha: float = 0.05
    densify_from: int = 500
    densify_until: int = 15000
    densify_every: int = 100
    densify_grad_threshold: float = 0.0002
    mcmc_relocate_frac: float = 0.02
    mcmc_min_opacity: float = 0.01
    mcmc_jitter_scale: float = 0.25
    mcmc_noise_scale: float = 0.01
    two_d_thickness: float = 1e-4
    opacity_reset_every: int = 3000
    sh_increase_every: int = 1000
    white_background: bool = False
    max_gaussians: int | None = None
    low_memory: bool = False
    cache_limit_gb: float = 2.0


class GaussianTrainer:
    """Optimises a :class:`GaussianModel` against posed images (trainer.py:78-421)."""

    def __init__(self, model: GaussianModel, config: TrainerConfig | None = None,
                 scene_extent: float = 1.0, generator: torch.Generator | None = None):
        self.model = model
        self.config = config or TrainerConfig()
        if self.config.method not in {"vanilla", "mcmc", "2dgs"}:
            raise ValueError("TrainerConfig.method must be 'vanilla', 'mcmc', or '2dgs'")
        if self.config.projection not in {"ewa", "ut"}:
            raise ValueError("TrainerConfig.projection must be 'ewa' or 'ut'")
        self.scene_extent = scene_extent
        self.step_count = 0
        # Random draws of the MCMC method (relocation jitter, position noise).
        self.generator = generator
        for k in _GROUPS:
            if model.params[k].device.type != "cuda":
                raise ValueError("GaussianTrainer: model parameters must be on the GPU")
        self._apply_method_constraints()
        self._build_optimizers()
        self._reset_grad_accum()

    # ------------------------------------------------------------ optimiser
    def _build_optimizers(self) -> None:
        """trainer.py:101-128: Adam(eps=1e-15) per group; the means rate
        decays exponentially from lr_means to lr_means_final."""
        c = self.config
        lr_means = c.lr_means * self.scene_extent
        lr_means_final = c.lr_means_final * self.scene_extent
        steps = int(c.lr_means_max_steps)
        if steps > 0 and lr_means > 0 and lr_means_final > 0:
            means_lr = exponential_decay(lr_means, (lr_means_final / lr_means) ** (1.0 / steps))
            if self.step_count:
                offset = self.step_count
                base = means_lr

                def means_lr(step, schedule=base, offset=offset):
                    return schedule(step + offset)
        else:
            means_lr = lr_means
        lrs = {"means": means_lr, "scales": c.lr_scales, "quats": c.lr_quats,
               "opacities": c.lr_opacities, "sh_dc": c.lr_sh_dc, "sh_rest": c.lr_sh_rest}
        self.optimizers = {k: Adam(learning_rate=lr, eps=1e-15) for k, lr in lrs.items()}

    def learning_rates(self) -> dict[str, float]:
        """Current per-group Adam learning rates (trainer.py:130-132)."""
        return {k: float(np.float32(opt.learning_rate)) for k, opt in self.optimizers.items()}

    def _reset_grad_accum(self) -> None:
        n = self.model.num_gaussians
        dev = self.model.params["means"].device
        self.grad_accum = torch.zeros((n,), dtype=torch.float32, device=dev)
        self.grad_count = torch.zeros((n,), dtype=torch.float32, device=dev)

    def _resize_optimizer_states_after_densify(self, result: dict) -> None:
        """Keep Adam moments of surviving rows; zeros for new rows (trainer.py:139-159)."""
        keep = result.get("_keep_idx")
        new_count = int(result.get("_new_count", 0))
        if keep is None:
            return
        for name, opt in self.optimizers.items():
            st = opt.state.get(name)
            if st is None:
                continue
            idx = torch.as_tensor(keep, dtype=torch.int64, device=st["m"].device)
            for slot in ("m", "v"):
                old = st[slot]
                kept = old[idx]
                if new_count > 0:
                    kept = torch.cat([kept, kept.new_zeros((new_count, *old.shape[1:]))])
                st[slot] = kept.contiguous()

    def _zero_optimizer_state_rows(self, idx) -> None:
        """Zero Adam moments of relocated rows (trainer.py:161-179)."""
        if idx is None or len(idx) == 0:
            return
        for name, opt in self.optimizers.items():
            st = opt.state.get(name)
            if st is None:
                continue
            rows = torch.as_tensor(idx, dtype=torch.int64, device=st["m"].device)
            for slot in ("m", "v"):
                st[slot][rows] = 0.0

    def _apply_method_constraints(self) -> None:
        if self.config.method == "2dgs":
            thickness = self.config.two_d_thickness * max(float(self.scene_extent), 1e-8)
            self.model.apply_2dgs_constraints(thickness)

    # ------------------------------------------------------------ losses
    def _photometric(self, img: torch.Tensor, target: torch.Tensor) -> torch.Tensor:
        l1, s = photometric(img, target)
        c = self.config.lambda_dssim
        return (1.0 - c) * l1 + c * (1.0 - s)

    def _geometry_loss_2dgs(self, params, camera: Camera, proj, opacities, sorted_ids,
                            tile_ranges, tiles_x, tiles_y):
        """Ray-depth variance and depth/normal consistency (trainer.py:187-259)."""
        cfg = self.config
        dev = params["means"].device
        zero = torch.zeros((), dtype=torch.float32, device=dev)
        metrics = {"depth_variance": zero, "normal_consistency": zero}
        if cfg.method != "2dgs" or (cfg.lambda_2d_depth_variance <= 0
                                    and cfg.lambda_2d_normal_consistency <= 0):
            return zero, metrics
        depths = proj["depths"]
        normals = quaternion_to_matrix(params["quats"])[:, :, 2]
        view = camera.camera_center.to(dev) - params["means"]
        normals = normals / torch.clamp(torch.linalg.norm(normals, dim=-1, keepdim=True),
                                        min=1e-8)
        normals = torch.where((normals * view).sum(-1, keepdim=True) < 0, -normals, normals)
        features = torch.cat([depths[:, None], (depths * depths)[:, None], normals], dim=1)
        geom = rasterize_features(proj["means2d"], proj["conics"], features, opacities,
                                  sorted_ids, tile_ranges, camera.width, camera.height,
                                  tiles_x, tiles_y, normalize=True)
        alpha = geom["alpha"]
        valid = (alpha > cfg.geometry_min_alpha).to(torch.float32)
        denom = torch.clamp(valid.sum(), min=1.0)
        ed = geom["features"][..., 0]
        ed2 = geom["features"][..., 1]
        depth_var = torch.clamp(ed2 - ed * ed, min=0.0)
        loss = zero
        if cfg.lambda_2d_depth_variance > 0:
            metrics["depth_variance"] = (depth_var * valid).sum() / denom
            loss = loss + float(cfg.lambda_2d_depth_variance) * metrics["depth_variance"]
        if cfg.lambda_2d_normal_consistency > 0 and camera.width > 1 and camera.height > 1:
            u = torch.arange(camera.width, dtype=torch.float32, device=dev) + 0.5
            v = torch.arange(camera.height, dtype=torch.float32, device=dev) + 0.5
            uu = u[None, :].expand(camera.height, camera.width)
            vv = v[:, None].expand(camera.height, camera.width)
            points = camera.unproject_points(torch.stack([uu, vv], dim=-1), ed)
            tx = points[:-1, 1:] - points[:-1, :-1]
            ty = points[1:, :-1] - points[:-1, :-1]
            dn = torch.linalg.cross(tx, ty)
            dn = dn / torch.clamp(torch.linalg.norm(dn, dim=-1, keepdim=True), min=1e-8)
            rn = geom["features"][:-1, :-1, 2:5]
            rn = rn / torch.clamp(torch.linalg.norm(rn, dim=-1, keepdim=True), min=1e-8)
            valid4 = valid[:-1, :-1] * valid[:-1, 1:] * valid[1:, :-1] * valid[1:, 1:]
            denom4 = torch.clamp(valid4.sum(), min=1.0)
            cos = (rn * dn).sum(-1)
            metrics["normal_consistency"] = ((1.0 - cos.abs()) * valid4).sum() / denom4
            loss = loss + float(cfg.lambda_2d_normal_consistency) * metrics["normal_consistency"]
        return loss, metrics

    def _render_loss_fused(self, params, camera: Camera, target, background, stats):
        """trainer.py:261-316 on the fused path (vanilla / MCMC)."""
        p = params
        K = p["sh_dc"].shape[1] + p["sh_rest"].shape[1]
        out = _run(camera, p["means"], p["quats"], p["scales"], p["opacities"], sh_a=p["sh_dc"],
                   sh_b=p["sh_rest"], sh_mode="split", K=K, degree=self.model.active_sh_degree,
                   background=background,
                   flags=(_lib.LOG_SCALES | _lib.LOGIT_OPACITY
                          | _check_common(self.config.projection)),
                   antialias=self.config.antialias, screen_stats=stats)
        img = out["image"]
        return self._photometric(img, target), img, out["radii"], None

    def _render_loss_staged(self, params, probe, camera: Camera, target, background):
        """trainer.py:261-316 stage by stage, with the reference's means2d probe."""
        p = params
        project = project_gaussians_ut if self.config.projection == "ut" else project_gaussians
        proj = project(camera, p["means"], p["quats"], torch.exp(p["scales"]),
                       antialias=self.config.antialias)
        means2d = proj["means2d"] + probe
        opacities = torch.sigmoid(p["opacities"]) * proj["compensation"]
        sh = torch.cat([p["sh_dc"], p["sh_rest"]], dim=1)
        dirs = p["means"] - camera.camera_center.to(p["means"].device)
        dirs = dirs / torch.clamp(torch.linalg.norm(dirs, dim=-1, keepdim=True), min=1e-8)
        colors = torch.clamp(eval_sh(self.model.active_sh_degree, sh, dirs.detach()), min=0.0)
        sorted_ids, tile_ranges, tiles_x, tiles_y = bin_gaussians(
            means2d, proj["radii"], proj["depths"], camera.width, camera.height)
        out = rasterize(means2d, proj["conics"], colors, opacities, sorted_ids, tile_ranges,
                        camera.width, camera.height, tiles_x, tiles_y, background=background)
        img = out["image"]
        loss = self._photometric(img, target)
        geom_loss, geom_metrics = self._geometry_loss_2dgs(p, camera, proj, opacities,
                                                           sorted_ids, tile_ranges, tiles_x,
                                                           tiles_y)
        return loss + geom_loss, img, proj["radii"], geom_metrics

    # ------------------------------------------------------------ step
    def step(self, camera: Camera, target: torch.Tensor) -> dict:
        """One optimisation step on a single view (trainer.py:319-421)."""
        self.step_count += 1
        cfg = self.config
        model = self.model
        dev = model.params["means"].device
        target = _lib.f32c(torch.as_tensor(target, device=dev))
        bg = torch.full((3,), 1.0 if cfg.white_background else 0.0, device=dev)
        densify_stats = None
        opacity_reset = False
        sh_degree_changed = False
        in_window = cfg.densify_from <= self.step_count <= cfg.densify_until

        params = {k: model.params[k].detach().requires_grad_(True) for k in _GROUPS}
        geom_metrics = None
        if cfg.method == "2dgs":
            probe = torch.zeros((model.num_gaussians, 2), device=dev, requires_grad=True)
            loss, img, radii, geom_metrics = self._render_loss_staged(params, probe, camera,
                                                                      target, bg)
            grads = torch.autograd.grad(loss, [params[k] for k in _GROUPS] + [probe],
                                        allow_unused=True)
            probe_grad = grads[-1]
            grads = grads[:-1]
        else:
            stats = (self.grad_accum, self.grad_count) if in_window else None
            loss, img, radii, _ = self._render_loss_fused(params, camera, target, bg, stats)
            grads = torch.autograd.grad(loss, [params[k] for k in _GROUPS], allow_unused=True)
            probe_grad = None

        # One launch updates all six groups in place (trainer.py:339-342).
        updates = []
        for k, g in zip(_GROUPS, grads):
            if g is None:
                g = torch.zeros_like(model.params[k])
            updates.append((self.optimizers[k], {k: g}, {k: model.params[k].data}))
        adam_step(updates)

        if cfg.method == "mcmc" and cfg.mcmc_noise_scale > 0:
            means_lr = max(float(self.learning_rates()["means"]), 0.0)
            sigma = cfg.mcmc_noise_scale * self.scene_extent * math.sqrt(means_lr)
            if sigma > 0:
                m = model.params["means"]
                gdev = self.generator.device if self.generator is not None else dev
                noise = torch.randn(m.shape, generator=self.generator, device=gdev).to(dev)
                with torch.no_grad():
                    m.add_(noise * sigma)
        self._apply_method_constraints()

        if in_window:
            if probe_grad is not None:
                _lib.check(_lib.load().gsx_accum_screen_grads(
                    probe_grad.shape[0], _lib.ptr(_lib.f32c(probe_grad)),
                    _lib.ptr(_lib.f32c(radii.detach())), camera.width, camera.height,
                    _lib.ptr(self.grad_accum), _lib.ptr(self.grad_count),
                    _lib.stream_handle(dev)), "gsx_accum_screen_grads")
            if self.step_count % cfg.densify_every == 0 and self.step_count > cfg.densify_from:
                if cfg.method == "mcmc":
                    result = model.relocate_mcmc(self.grad_accum, self.grad_count,
                                                 relocate_frac=cfg.mcmc_relocate_frac,
                                                 min_opacity=cfg.mcmc_min_opacity,
                                                 jitter_scale=cfg.mcmc_jitter_scale,
                                                 generator=self.generator)
                    self._zero_optimizer_state_rows(result.get("_moved_idx"))
                else:
                    at_cap = (cfg.max_gaussians is not None
                              and model.num_gaussians >= cfg.max_gaussians)
                    threshold = float("inf") if at_cap else cfg.densify_grad_threshold
                    result = model.densify_and_prune(self.grad_accum, self.grad_count,
                                                     grad_threshold=threshold,
                                                     scene_extent=self.scene_extent,
                                                     return_optimizer_state=True)
                    self._resize_optimizer_states_after_densify(result)
                self._apply_method_constraints()
                densify_stats = {k: v for k, v in result.items() if not str(k).startswith("_")}
                self._reset_grad_accum()

        if self.step_count % cfg.opacity_reset_every == 0 and self.step_count <= cfg.densify_until:
            model.reset_opacities()
            opacity_reset = True
        if self.step_count % cfg.sh_increase_every == 0:
            model.one_up_sh_degree()
            sh_degree_changed = True

        geometry = {"depth_variance": 0.0, "normal_consistency": 0.0}
        if geom_metrics is not None:
            geometry = {k: float(v) for k, v in geom_metrics.items()}
        return {
            "loss": float(loss),
            "num_gaussians": model.num_gaussians,
            "step": self.step_count,
            "active_sh_degree": model.active_sh_degree,
            "lr_means": self.learning_rates()["means"],
            "method": cfg.method,
            "densify": densify_stats,
            "opacity_reset": opacity_reset,
            "sh_degree_changed": sh_degree_changed,
            "geometry": geometry,
        }
