"""Density control and point-cloud initialisation on the device.

Row edits of a Gaussian table (``GaussianModel.params`` plus, in training,
the Adam moments of each group) through the ``gsx_density_*`` kernels:

- :func:`knn_log_scales` -- the isotropic log-scale of ``from_points``
  (splatting/model.py:72-92): one lane per point, reference points streamed
  through LDS, the K nearest kept in registers.
- :func:`densify` -- adaptive density control (model.py:406-480): a
  classification pass with per-block counts, a one-workgroup scan, then one
  emission pass that writes kept rows, clones and split pairs of every
  tensor (moments follow kept rows and start at zero in new ones).  The host
  reads the three totals once, to size the new table and to draw the split
  samples from NumPy's global generator in the reference's order.
- :func:`relocate` -- fixed-budget MCMC relocation (model.py:482-531): the
  selection scores come from one kernel, the k best targets and sources
  from ``torch.topk``, and the rows are rewritten (moments of moved rows
  cleared) by a gather and a scatter launch.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from .. import _lib

__all__ = ["GROUPS", "knn_log_scales", "densify", "relocate"]

# parameter groups of a table, in the order the trainer optimises them
GROUPS = ("means", "scales", "quats", "opacities", "sh_dc", "sh_rest")
_SPLIT_SHRINK = float(np.float32(math.log(1.6)))  # model.py:451, 520


def knn_log_scales(points: torch.Tensor, ref: torch.Tensor, k: int,
                   max_scale: float | None = None) -> torch.Tensor:
    """(N,) log(sqrt(mean squared distance to the k - 1 nearest of ``ref``,
    a zero-distance self hit skipped)), capped at log(max_scale)."""
    dev = _lib.require_device(points, ref)
    p, r = _lib.f32c(points), _lib.f32c(ref)
    out = torch.empty((p.shape[0],), dtype=torch.float32, device=dev)
    cap = math.inf if max_scale is None else math.log(max(float(max_scale), 1e-8))
    _lib.check(_lib.load().gsx_knn_log_scale(p.shape[0], _lib.ptr(p), r.shape[0], _lib.ptr(r),
                                             int(k), cap, _lib.ptr(out),
                                             _lib.stream_handle(dev)), "gsx_knn_log_scale")
    return out


def _column_list(params: dict, moments: dict | None, out_rows: int | None):
    """[(name, slot, src, dst, role)] for the table (dst new tensors when
    out_rows is given, else the sources themselves)."""
    cols = []
    for name in GROUPS:
        src = params[name].detach()
        if not src.is_contiguous() or src.dtype != torch.float32:
            raise ValueError(f"parameter {name!r} must be contiguous float32")
        dst = src if out_rows is None else src.new_empty((out_rows, *src.shape[1:]))
        cols.append((name, None, src, dst, _lib.ROW_PARAM))
    for name, slots in (moments or {}).items():
        for slot, src in slots.items():
            dst = src if out_rows is None else src.new_empty((out_rows, *src.shape[1:]))
            cols.append((name, slot, src, dst, _lib.ROW_MOMENT))
    if any(c[2].shape[0] == 0 for c in cols):
        raise ValueError("empty tables have no rows to edit")
    return cols


def _kernel_table(cols):
    """(GsxRowTable of the columns with a nonzero row width, {group: index}
    of its parameter columns)."""
    live = [c for c in cols if c[2][0].numel() > 0]
    index = {c[0]: k for k, c in enumerate(live) if c[1] is None}
    return _lib.row_table([(c[2], c[3], c[4]) for c in live]), index


def densify(params: dict, grad_accum: torch.Tensor, grad_count: torch.Tensor, *,
            grad_threshold: float, scene_extent: float, percent_dense: float,
            min_opacity: float, moments: dict | None = None):
    """Clone / split / prune (model.py:406-480).

    ``moments`` = {group: {"m": tensor, "v": tensor}} are carried along.
    Returns (new params, new moments, stats, keep_idx (device int64))."""
    n = params["means"].shape[0]
    dev = _lib.require_device(params["means"], grad_accum, grad_count)
    if n == 0:
        empty = torch.zeros(0, dtype=torch.int64, device=dev)
        return dict(params), dict(moments or {}), {"cloned": 0, "split": 0, "pruned": 0}, empty
    L = _lib.load()
    st = _lib.stream_handle(dev)
    ws = torch.empty(int(L.gsx_density_workspace_bytes(n)), dtype=torch.uint8, device=dev)
    totals = torch.zeros(3, dtype=torch.int32, device=dev)
    p = {k: params[k].detach() for k in GROUPS}
    # converted inputs stay bound until the kernels are enqueued
    ls, lo = _lib.f32c(p["scales"]), _lib.f32c(p["opacities"])
    acc, cnt = _lib.f32c(grad_accum), _lib.f32c(grad_count)
    _lib.check(L.gsx_density_classify(
        n, _lib.ptr(ls), _lib.ptr(lo), _lib.ptr(acc), _lib.ptr(cnt), float(grad_threshold),
        float(percent_dense * scene_extent), float(0.5 * scene_extent), float(min_opacity),
        _lib.ptr(ws), ws.numel(), _lib.ptr(totals), st), "gsx_density_classify")
    kept, cloned, split = (int(x) for x in totals.cpu().tolist())  # the one host sync
    rows = kept + cloned + 2 * split
    # the reference's draws: one (2 split, 3) standard-normal array, pair-major
    samples = torch.from_numpy(np.random.normal(size=(2 * split, 3)) if split
                               else np.zeros((1, 3))).to(dev)
    cols = _column_list(p, moments, rows)
    table, col = _kernel_table(cols)
    if rows > 0:
        _lib.check(L.gsx_density_emit(
            n, _lib.ptr(ws), ws.numel(), _lib.ptr(totals), table, col["means"], col["scales"],
            col["quats"], _lib.ptr(samples), _SPLIT_SHRINK, st), "gsx_density_emit")
    new_params = {c[0]: c[3] for c in cols if c[1] is None}
    new_moments: dict = {}
    for name, slot, _, dst, role in cols:
        if role == _lib.ROW_MOMENT:
            new_moments.setdefault(name, {})[slot] = dst
    classes = ws[:n]
    keep_idx = torch.nonzero(classes & 1).flatten()
    stats = {"cloned": cloned, "split": split, "pruned": n - kept}
    return new_params, new_moments, stats, keep_idx


def relocate(params: dict, grad_accum: torch.Tensor, grad_count: torch.Tensor, *,
             relocate_frac: float, min_opacity: float, jitter_scale: float,
             generator: torch.Generator | None = None, moments: dict | None = None):
    """Fixed-budget relocation (model.py:482-531), in place.  Returns
    (number of moved rows, destination rows (device int64) or None)."""
    n = params["means"].shape[0]
    budget = int(max(0.0, min(relocate_frac, 1.0)) * n)
    if budget <= 0 or n <= 1:
        return 0, None
    dev = _lib.require_device(params["means"], grad_accum, grad_count)
    L = _lib.load()
    st = _lib.stream_handle(dev)
    target = torch.empty((n,), dtype=torch.float32, device=dev)
    source = torch.empty((n,), dtype=torch.float32, device=dev)
    under = torch.zeros(1, dtype=torch.int32, device=dev)
    logits = _lib.f32c(params["opacities"].detach())
    acc, cnt = _lib.f32c(grad_accum), _lib.f32c(grad_count)
    _lib.check(L.gsx_relocate_scores(n, _lib.ptr(acc), _lib.ptr(cnt), _lib.ptr(logits),
                                     float(min_opacity), _lib.ptr(target), _lib.ptr(source),
                                     _lib.ptr(under), st), "gsx_relocate_scores")
    n_under = int(under.item())
    k = min(budget if n_under == 0 else min(budget, n_under), n - 1)
    if k <= 0:
        return 0, None
    dst = torch.topk(target, k).indices
    source.index_fill_(0, dst, -1e30)  # destinations are never sources
    src = torch.topk(source, k).indices
    if jitter_scale > 0:  # model.py:519: noise is drawn only for a positive jitter
        gdev = generator.device if generator is not None else dev
        noise = torch.randn((k, 3), generator=generator, device=gdev).to(dev)
    else:
        noise = torch.zeros((k, 3), dtype=torch.float32, device=dev)
    cols = _column_list({g: params[g] for g in GROUPS}, moments, None)
    width = sum(int(c[2][0].numel()) for c in cols if c[4] == _lib.ROW_PARAM)
    staging = torch.empty((k, width), dtype=torch.float32, device=dev)
    table, col = _kernel_table(cols)
    reset = float(np.float32(math.log(0.05 / 0.95)))
    _lib.check(L.gsx_density_relocate(
        k, _lib.ptr(src), _lib.ptr(dst), table, col["means"], col["scales"], col["opacities"],
        _lib.ptr(noise), float(jitter_scale), reset, _SPLIT_SHRINK, _lib.ptr(staging),
        staging.numel(), st), "gsx_density_relocate")
    return k, dst
