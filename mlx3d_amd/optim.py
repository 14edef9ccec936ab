"""Adam as the training step uses it (``mlx.optimizers.Adam`` and
``mlx.optimizers.exponential_decay``, mlx >= 0.31, called at
``src/mlx3d/splatting/trainer.py:101-128, 339-342``).

Each parameter group of the trainer has its own ``Adam`` (per-group learning
rate and schedule); ``adam_step`` applies any number of them in one kernel
launch (``gsx_adam_step``).  Semantics (bias correction off, the MLX
default):

    lr = schedule(step)          # step counts earlier updates, from 0
    m = b1 m + (1 - b1) g
    v = b2 v + (1 - b2) g^2
    p = p - lr m / (sqrt(v) + eps)

in float32 with ``m`` and ``v`` starting at zero.  Schedules are evaluated
in double precision and rounded to float32 once.
"""

from __future__ import annotations

import ctypes
from typing import Callable

import torch

from . import _lib
from .profiling import stage

__all__ = ["Adam", "adam_step", "exponential_decay", "FusedAdam"]


def exponential_decay(init: float, decay_rate: float) -> Callable[[int], float]:
    """``init * decay_rate ** step`` (mlx.optimizers.exponential_decay)."""

    def schedule(step: int) -> float:
        return init * decay_rate ** step

    return schedule


class Adam:
    """Adam state for one group of parameters, keyed by name."""

    def __init__(self, learning_rate: float | Callable[[int], float],
                 betas: tuple[float, float] = (0.9, 0.999), eps: float = 1e-8,
                 bias_correction: bool = False):
        if bias_correction:
            raise NotImplementedError("bias_correction=True is not supported (the trainer "
                                      "uses MLX's default, False)")
        self._lr = learning_rate
        self.betas = (float(betas[0]), float(betas[1]))
        self.eps = float(eps)
        self.step = 0
        self.state: dict[str, dict[str, torch.Tensor]] = {}
        self._last_lr = self._schedule(0)

    def _schedule(self, step: int) -> float:
        return float(self._lr(step)) if callable(self._lr) else float(self._lr)

    @property
    def learning_rate(self) -> float:
        """The rate the most recent update used (before any update: step 0)."""
        return self._last_lr

    def _state_for(self, name: str, p: torch.Tensor) -> dict[str, torch.Tensor]:
        st = self.state.get(name)
        if st is None or st["m"].shape != p.shape:
            st = {"m": torch.zeros_like(p), "v": torch.zeros_like(p)}
            self.state[name] = st
        return st

    def _advance(self, lr: float) -> None:
        """Records that the update at the current step (rate ``lr``) was
        enqueued: called only after its launch succeeded, so a failed launch
        leaves the schedule where it was."""
        self._last_lr = lr
        self.step += 1

    def _groups(self, grads: dict[str, torch.Tensor], params: dict[str, torch.Tensor]):
        lr = self._schedule(self.step)
        out = []
        for name, g in grads.items():
            p = params[name]
            if g is None:
                continue
            if p.dtype != torch.float32 or not p.is_contiguous():
                raise ValueError(f"parameter {name!r} must be contiguous float32")
            if g.shape != p.shape:
                raise ValueError(f"gradient of {name!r} has shape {tuple(g.shape)}, "
                                 f"parameter {tuple(p.shape)}")
            st = self._state_for(name, p)
            out.append((p, _lib.f32c(g), st["m"], st["v"], lr, self))
        return out

    def _fused_group(self, name: str, p: torch.Tensor):
        """The bookkeeping of one update of parameter ``name`` whose gradient
        a kernel computes and applies itself: returns (param, m, v, lr) at
        the current step; the caller advances the schedule (``_advance``)
        once the kernel is enqueued."""
        if p.dtype != torch.float32 or not p.is_contiguous():
            raise ValueError(f"parameter {name!r} must be contiguous float32")
        lr = self._schedule(self.step)
        st = self._state_for(name, p)
        return p, st["m"], st["v"], lr

    def apply_gradients(self, grads: dict[str, torch.Tensor],
                        params: dict[str, torch.Tensor]) -> dict[str, torch.Tensor]:
        """Updates ``params`` in place (and returns them)."""
        adam_step([(self, grads, params)])
        return params


def adam_step(updates) -> None:
    """Applies ``[(adam, grads, params), ...]`` in one launch per
    ``ADAM_MAX_GROUPS`` tensors.  All optimisers must share betas and eps."""
    groups = []
    for opt, grads, params in updates:
        groups.extend(opt._groups(grads, params))
    if not groups:
        return
    b1, b2 = groups[0][5].betas
    eps = groups[0][5].eps
    for g in groups:
        if g[5].betas != (b1, b2) or g[5].eps != eps:
            raise ValueError("adam_step: optimisers with different betas/eps")
    dev = _lib.require_device(*[g[0] for g in groups])
    L = _lib.load()
    keep = []
    # each optimiser's schedule advances once, after all its launches succeeded
    advance = {id(opt): (opt, g[4]) for g in groups for opt in (g[5],)}
    for s in range(0, len(groups), _lib.ADAM_MAX_GROUPS):
        chunk = groups[s:s + _lib.ADAM_MAX_GROUPS]
        arr = (_lib.GsxAdamGroup * len(chunk))()
        for k, (p, g, m, v, lr, _) in enumerate(chunk):
            arr[k] = _lib.GsxAdamGroup(p.data_ptr(), g.data_ptr(), m.data_ptr(), v.data_ptr(),
                                       p.numel(), lr)
            keep.append(g)
        with stage("adam"):
            _lib.check(L.gsx_adam_step(len(chunk), ctypes.cast(arr, ctypes.c_void_p), b1, b2,
                                       eps, _lib.stream_handle(dev)), "gsx_adam_step")
    for opt, lr in advance.values():
        opt._advance(lr)


class FusedAdam:
    """One Adam update of several parameters applied by the kernel that
    computes their gradients (``gsx_preprocess_bwd_adam``): built from
    ``[(adam, name, param), ...]`` before the backward runs, it holds the
    ``gsx_adam_group`` records (gradient pointers unused) with each
    optimiser's rate at its current step.  ``commit()``, called once the
    kernel is enqueued, advances each optimiser's schedule once, as
    ``adam_step`` does; an update that never launched leaves them alone."""

    def __init__(self, updates):
        groups = [opt._fused_group(name, p) for opt, name, p in updates]
        opts = [u[0] for u in updates]
        self._advance = {id(o): (o, g[3]) for o, g in zip(opts, groups)}
        self.committed = False
        self.betas, self.eps = opts[0].betas, opts[0].eps
        if any(o.betas != self.betas or o.eps != self.eps for o in opts):
            raise ValueError("FusedAdam: optimisers with different betas/eps")
        self.tensors = [t for g in groups for t in g[:3]]  # kept alive with the records
        self.records = (_lib.GsxAdamGroup * len(groups))()
        for k, (p, m, v, lr) in enumerate(groups):
            self.records[k] = _lib.GsxAdamGroup(p.data_ptr(), None, m.data_ptr(), v.data_ptr(),
                                                p.numel(), lr)

    def commit(self) -> None:
        """Advances the schedules (once per update; later calls do nothing)."""
        if self.committed:
            return
        self.committed = True
        for opt, lr in self._advance.values():
            opt._advance(lr)
