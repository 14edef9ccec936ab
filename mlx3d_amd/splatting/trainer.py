"""The training step around the rasterizer (``src/mlx3d/splatting/trainer.py``).

One ``GaussianTrainer.step`` on the vanilla and MCMC methods is

    fused render forward (preprocess, binning, raster)        libgsx
    photometric loss: (1 - lambda) L1 + lambda (1 - SSIM)      gsx_photometric_loss_fwd
      from one pass
    backward: loss gradient, raster VJP (+ the screen-space    gsx_photometric_loss_bwd,
      gradient statistics of density control)                  gsx_raster_bwd, ...
    preprocess VJP with the Adam update of all six parameter   gsx_preprocess_bwd_adam
      groups fused in (fuse_adam=False: the VJP, then one      (gsx_preprocess_bwd,
      multi-group Adam launch)                                  gsx_adam_step)

with no host synchronisation except the duplicate count of the binning
and the step's loss, which is copied to pinned memory right after the loss
kernels: step() waits for that copy, not for the backward or the update,
so the next step is queued while the GPU finishes this one.  Density
control runs every ``densify_every`` steps on the device.

The reference probes dL/dmeans2d by adding a zero (N, 2) array to means2d
(trainer.py:264-275, 325, 337); here the backward hands the rasterizer's
dL/dmeans2d straight to ``gsx_accum_screen_grads``.  The 2DGS method renders
through the separate drop-in stages (project, eval_sh, bin, rasterize,
rasterize_features), because its geometry losses need the projected
Gaussians; its surfel features and losses are the ``gsx_geom_*`` kernels
(``splatting/geometry.py``) and its screen statistics come from a probe.

The Adam moments live in the optimisers; density control edits them with
the parameter table in the same device launches (kept rows keep their
moments, new rows start at zero, relocated rows are cleared).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

from ..cameras import Camera
from ..losses import photometric_loss
from ..optim import Adam, FusedAdam, adam_step, exponential_decay
from .. import _lib
from .density import GROUPS
from .geometry import geometry_loss, surfel_features, unprojection_maps
from .model import GaussianModel
from .projection import project_gaussians, project_gaussians_ut
from .rasterize import rasterize, rasterize_features
from .render import _check_common, _run
from .sh import eval_sh
from .tiles import bin_gaussians

# parameter groups in the order gsx_preprocess_bwd_adam takes them
_FUSED_ORDER = ("means", "quats", "scales", "opacities", "sh_dc", "sh_rest")

__all__ = ["TrainerConfig", "GaussianTrainer"]


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
    # no counterpart in the reference: keep the table in 3D Morton order of
    # the means (GaussianModel.reorder_spatial) from the start and after
    # every density event, the Adam moments permuted alongside
    spatial_order: bool = False


class _StepResult:
    """What one forward+backward of a training step produced."""

    __slots__ = ("loss", "grads", "radii", "probe_grad", "geometry")

    def __init__(self, loss, grads, radii, probe_grad=None, geometry=None):
        self.loss, self.grads, self.radii = loss, grads, radii
        self.probe_grad, self.geometry = probe_grad, geometry


class GaussianTrainer:
    """Optimises a :class:`GaussianModel` against posed images (trainer.py:78-421)."""

    def __init__(self, model: GaussianModel, config: TrainerConfig | None = None,
                 scene_extent: float = 1.0, generator: torch.Generator | None = None,
                 fuse_adam: bool = True):
        self.model = model
        # vanilla / MCMC: the Adam update runs inside the preprocess backward
        # (gsx_preprocess_bwd_adam, the same updates bit for bit); False keeps
        # the separate gradient tensors and one gsx_adam_step launch
        self.fuse_adam = bool(fuse_adam)
        self.config = config or TrainerConfig()
        if self.config.method not in {"vanilla", "mcmc", "2dgs"}:
            raise ValueError("TrainerConfig.method must be 'vanilla', 'mcmc', or '2dgs'")
        if self.config.projection not in {"ewa", "ut"}:
            raise ValueError("TrainerConfig.projection must be 'ewa' or 'ut'")
        for name in GROUPS:
            if model.params[name].device.type != "cuda":
                raise ValueError("GaussianTrainer: model parameters must be on the GPU")
        self.scene_extent = scene_extent
        self.step_count = 0
        # random draws of the MCMC method (relocation jitter, position noise)
        self.generator = generator
        self._unproject = None  # (camera key, maps) of the last 2DGS view
        # the step's scalar results (loss, geometry terms) land in pinned host
        # memory behind the kernels that produce them (_queue_readback)
        self._host_scalars = None
        self._scalars_ready = None
        self._consts = {}  # (name, device) -> small constant tensors reused every step
        self._constrain()
        self.optimizers = {name: Adam(learning_rate=rate, eps=1e-15)
                           for name, rate in self._group_rates().items()}
        self._reorder()
        self._new_screen_stats()

    # ------------------------------------------------------------ set-up
    def _group_rates(self) -> dict:
        """Per-group Adam rates (trainer.py:101-128): constants, except the
        means, whose rate falls geometrically from lr_means to lr_means_final
        over lr_means_max_steps updates (both scaled by the scene extent)."""
        c = self.config
        first = c.lr_means * self.scene_extent
        last = c.lr_means_final * self.scene_extent
        horizon = int(c.lr_means_max_steps)
        means = first
        if horizon > 0 and first > 0 and last > 0:
            means = exponential_decay(first, (last / first) ** (1.0 / horizon))
        return {"means": means, "scales": c.lr_scales, "quats": c.lr_quats,
                "opacities": c.lr_opacities, "sh_dc": c.lr_sh_dc, "sh_rest": c.lr_sh_rest}

    def learning_rates(self) -> dict[str, float]:
        """Current per-group Adam learning rates (trainer.py:130-132)."""
        return {k: float(np.float32(opt.learning_rate)) for k, opt in self.optimizers.items()}

    def _new_screen_stats(self) -> None:
        """Zeroed density-control statistics, one entry per Gaussian."""
        n = self.model.num_gaussians
        dev = self.model.params["means"].device
        self.grad_accum = torch.zeros((n,), dtype=torch.float32, device=dev)
        self.grad_count = torch.zeros((n,), dtype=torch.float32, device=dev)

    def _moments(self) -> dict:
        """{group: {"m", "v"}} of the groups whose Adam state exists."""
        out = {}
        for name, opt in self.optimizers.items():
            st = opt.state.get(name)
            if st is not None:
                out[name] = {"m": st["m"], "v": st["v"]}
        return out

    def _reorder(self) -> None:
        """With ``spatial_order``: the table (and the Adam moments) in Morton
        order."""
        if not self.config.spatial_order:
            return
        perm = self.model.reorder_spatial()
        for name, opt in self.optimizers.items():
            st = opt.state.get(name)
            if st is not None:
                st["m"] = st["m"][perm].contiguous()
                st["v"] = st["v"][perm].contiguous()

    def _constrain(self) -> None:
        """2DGS keeps the third scale a thin surfel (trainer.py:181-185)."""
        if self.config.method == "2dgs":
            limit = self.config.two_d_thickness * max(float(self.scene_extent), 1e-8)
            self.model.apply_2dgs_constraints(limit)

    # ------------------------------------------------------------ forward+backward
    def _photometric(self, img: torch.Tensor, target: torch.Tensor) -> torch.Tensor:
        """(1 - lambda) L1 + lambda (1 - SSIM) (trainer.py:303-305) as one op."""
        return photometric_loss(img, target, self.config.lambda_dssim)

    def _queue_readback(self, values) -> None:
        """Copies the step's scalars to pinned host memory right behind the
        kernels that produce them, before the backward is queued: step()
        then returns them without waiting for the backward and the parameter
        update, and the host queues the next step while the GPU finishes
        this one."""
        if self._host_scalars is None:
            self._host_scalars = torch.empty((4,), dtype=torch.float32, pin_memory=True)
        src = torch.stack([v.detach().reshape(()) for v in values]) if len(values) > 1 \
            else values[0].detach().reshape(1)
        self._host_scalars[:len(values)].copy_(src, non_blocking=True)
        self._scalars_ready = torch.cuda.Event()
        self._scalars_ready.record(torch.cuda.current_stream(src.device))

    def _const(self, name: str, dev, make):
        """A small constant device tensor, built once per device (a per-step
        fill would cost a launch in every step)."""
        key = (name, str(dev))
        t = self._consts.get(key)
        if t is None:
            t = self._consts[key] = make()
        return t

    def _grads(self, loss, wrt):
        """dloss/dwrt with a cached unit cotangent."""
        one = self._const("one", loss.device,
                          lambda: torch.ones((), dtype=loss.dtype, device=loss.device))
        return torch.autograd.grad(loss, wrt, grad_outputs=one, allow_unused=True)

    def _read_back(self, count: int) -> list[float]:
        self._scalars_ready.synchronize()
        return self._host_scalars[:count].tolist()

    def _fused_pass(self, params, camera, target, background, collect: bool) -> _StepResult:
        """Vanilla / MCMC: the fused render, photometric loss and backward;
        the backward adds the screen statistics itself when ``collect``."""
        p = params
        stats = (self.grad_accum, self.grad_count) if collect else None
        # with fuse_adam the backward applies this step's Adam update itself
        # (the kernel's group order: means, quats, scales, opacities, DC, rest)
        adam = (FusedAdam([(self.optimizers[k], k, p[k]) for k in _FUSED_ORDER])
                if self.fuse_adam else None)
        out = _run(camera, p["means"], p["quats"], p["scales"], p["opacities"],
                   sh_a=p["sh_dc"], sh_b=p["sh_rest"], sh_mode="split",
                   K=p["sh_dc"].shape[1] + p["sh_rest"].shape[1],
                   degree=self.model.active_sh_degree, background=background,
                   flags=(_lib.LOG_SCALES | _lib.LOGIT_OPACITY
                          | _check_common(self.config.projection)),
                   antialias=self.config.antialias, screen_stats=stats, adam=adam)
        loss = self._photometric(out["image"], target)
        self._queue_readback([loss])
        grads = self._grads(loss, [p[k] for k in GROUPS])
        return _StepResult(loss, None if adam is not None else grads, out["radii"])

    @staticmethod
    def _camera_key(camera: Camera, dev) -> tuple:
        """Everything the unprojection maps depend on, by value: a Camera is
        a mutable dataclass and a new one may reuse a freed one's id()."""
        R = torch.as_tensor(camera.R, dtype=torch.float32).detach().cpu().contiguous()
        t = torch.as_tensor(camera.t, dtype=torch.float32).detach().cpu().contiguous()
        dist = None if camera.distortion is None else tuple(float(v) for v in camera.distortion)
        return (R.numpy().tobytes(), t.numpy().tobytes(), float(camera.fx), float(camera.fy),
                float(camera.cx), float(camera.cy), int(camera.width), int(camera.height), dist,
                bool(camera.fisheye), bool(camera.orthographic), str(dev))

    def _maps(self, camera: Camera, dev):
        key = GaussianTrainer._camera_key(camera, dev)
        if self._unproject is None or self._unproject[0] != key:
            self._unproject = (key, unprojection_maps(camera, dev))
        return self._unproject[1]

    def _staged_pass(self, params, camera, target, background) -> _StepResult:
        """2DGS: the drop-in stages with a means2d probe, plus the surfel
        geometry losses on a second, alpha-normalised feature render."""
        cfg = self.config
        p = params
        dev = p["means"].device
        probe = torch.zeros((self.model.num_gaussians, 2), device=dev, requires_grad=True)
        project = project_gaussians_ut if cfg.projection == "ut" else project_gaussians
        proj = project(camera, p["means"], p["quats"], torch.exp(p["scales"]),
                       antialias=cfg.antialias)
        xy = proj["means2d"] + probe
        opac = torch.sigmoid(p["opacities"]) * proj["compensation"]
        view = p["means"].detach() - camera.camera_center.to(dev)
        view = view / torch.clamp(torch.linalg.norm(view, dim=-1, keepdim=True), min=1e-8)
        rgb = torch.clamp(eval_sh(self.model.active_sh_degree,
                                  torch.cat([p["sh_dc"], p["sh_rest"]], dim=1), view), min=0.0)
        ids, ranges, tx, ty = bin_gaussians(xy, proj["radii"], proj["depths"], camera.width,
                                            camera.height)
        img = rasterize(xy, proj["conics"], rgb, opac, ids, ranges, camera.width, camera.height,
                        tx, ty, background=background)["image"]
        loss = self._photometric(img, target)
        geometry = None
        if cfg.lambda_2d_depth_variance > 0 or cfg.lambda_2d_normal_consistency > 0:
            feats = surfel_features(p["means"], p["quats"], proj["depths"], camera)
            # the geometry render reads the projection's means2d, not the
            # probed ones (trainer.py:212-213): the probe carries only the
            # photometric render's dL/dmeans2d into the density statistics
            rendered = rasterize_features(proj["means2d"], proj["conics"], feats, opac, ids,
                                          ranges, camera.width, camera.height, tx, ty,
                                          normalize=True)
            g_loss, geometry = geometry_loss(
                rendered["features"], rendered["alpha"], camera, cfg.geometry_min_alpha,
                cfg.lambda_2d_depth_variance, cfg.lambda_2d_normal_consistency,
                maps=self._maps(camera, dev))
            loss = loss + g_loss
        self._queue_readback([loss] if geometry is None else
                             [loss, geometry["depth_variance"], geometry["normal_consistency"]])
        wrt = [p[k] for k in GROUPS] + [probe]
        grads = self._grads(loss, wrt)
        return _StepResult(loss, grads[:-1], proj["radii"], grads[-1], geometry)

    # ------------------------------------------------------------ density control
    def _density_event(self) -> dict:
        """Clone/split/prune or relocate (trainer.py:371-400) with the Adam
        moments edited alongside; fresh statistics afterwards."""
        cfg = self.config
        model = self.model
        moments = self._moments()
        if cfg.method == "mcmc":
            result = model.relocate_mcmc(self.grad_accum, self.grad_count,
                                         relocate_frac=cfg.mcmc_relocate_frac,
                                         min_opacity=cfg.mcmc_min_opacity,
                                         jitter_scale=cfg.mcmc_jitter_scale,
                                         generator=self.generator, moments=moments)
        else:
            # at the size cap only pruning continues (an infinite threshold)
            capped = cfg.max_gaussians is not None and model.num_gaussians >= cfg.max_gaussians
            result = model.densify_and_prune(
                self.grad_accum, self.grad_count,
                grad_threshold=float("inf") if capped else cfg.densify_grad_threshold,
                scene_extent=self.scene_extent, moments=moments)
            for name, slots in result.pop("_moments", {}).items():
                self.optimizers[name].state[name] = slots
        self._constrain()
        self._reorder()
        self._new_screen_stats()
        return {k: v for k, v in result.items() if not str(k).startswith("_")}

    def _mcmc_noise(self) -> None:
        """MCMC position noise scaled by sqrt(current means rate) (trainer.py:343-350)."""
        cfg = self.config
        rate = max(float(self.learning_rates()["means"]), 0.0)
        sigma = cfg.mcmc_noise_scale * self.scene_extent * math.sqrt(rate)
        if sigma <= 0:
            return
        m = self.model.params["means"]
        where = self.generator.device if self.generator is not None else m.device
        noise = torch.randn(m.shape, generator=self.generator, device=where).to(m.device)
        with torch.no_grad():
            m.add_(noise * sigma)

    # ------------------------------------------------------------ step
    def step(self, camera: Camera, target: torch.Tensor) -> dict:
        """One optimisation step on a single view (trainer.py:319-421)."""
        self.step_count += 1
        cfg = self.config
        model = self.model
        dev = model.params["means"].device
        target = _lib.f32c(torch.as_tensor(target, device=dev))
        white = bool(cfg.white_background)
        background = self._const(f"background{int(white)}", dev,
                                 lambda: torch.full((3,), 1.0 if white else 0.0, device=dev))
        collect = cfg.densify_from <= self.step_count <= cfg.densify_until
        leaves = {k: model.params[k].detach().requires_grad_(True) for k in GROUPS}

        if cfg.method == "2dgs":
            res = self._staged_pass(leaves, camera, target, background)
        else:
            res = self._fused_pass(leaves, camera, target, background, collect)

        # every group in one Adam launch (trainer.py:339-342), unless the
        # backward has applied the update already
        if res.grads is not None:
            adam_step([(self.optimizers[k], {k: torch.zeros_like(model.params[k]) if g is None
                                             else g}, {k: model.params[k].data})
                       for k, g in zip(GROUPS, res.grads)])
        if cfg.method == "mcmc" and cfg.mcmc_noise_scale > 0:
            self._mcmc_noise()
        self._constrain()

        densify = None
        if collect:
            if res.probe_grad is not None:  # the staged pass's probe
                g2, r2 = _lib.f32c(res.probe_grad), _lib.f32c(res.radii.detach())
                _lib.check(_lib.load().gsx_accum_screen_grads(
                    g2.shape[0], _lib.ptr(g2), _lib.ptr(r2), camera.width, camera.height,
                    _lib.ptr(self.grad_accum), _lib.ptr(self.grad_count), 0,
                    _lib.stream_handle(dev)), "gsx_accum_screen_grads")
            if self.step_count % cfg.densify_every == 0 and self.step_count > cfg.densify_from:
                densify = self._density_event()

        opacity_reset = (self.step_count % cfg.opacity_reset_every == 0
                         and self.step_count <= cfg.densify_until)
        if opacity_reset:
            model.reset_opacities()
        sh_grew = self.step_count % cfg.sh_increase_every == 0
        if sh_grew:
            model.one_up_sh_degree()

        scalars = self._read_back(1 if res.geometry is None else 3)
        geometry = {"depth_variance": 0.0, "normal_consistency": 0.0}
        if res.geometry is not None:
            geometry = {"depth_variance": scalars[1], "normal_consistency": scalars[2]}
        return {
            "loss": scalars[0],
            "num_gaussians": model.num_gaussians,
            "step": self.step_count,
            "active_sh_degree": model.active_sh_degree,
            "lr_means": self.learning_rates()["means"],
            "method": cfg.method,
            "densify": densify,
            "opacity_reset": opacity_reset,
            "sh_degree_changed": sh_grew,
            "geometry": geometry,
        }
