"""Real spherical harmonics, degrees 0-3 (``src/mlx3d/splatting/sh.py:1-78``).

``eval_sh`` runs the HIP kernel ``gsx_eval_sh_fwd`` and is differentiable
w.r.t. both the coefficients and the directions (``gsx_eval_sh_bwd``).
"""

from __future__ import annotations

import torch

from .. import _lib

__all__ = ["eval_sh", "rgb_to_sh", "sh_to_rgb", "num_sh_bases"]

# sh.py:7-24 (textbook real-SH normalisations, 3DGS sign convention)
_C0 = 0.28209479177387814


def num_sh_bases(degree: int) -> int:
    """Number of coefficients of an SH expansion up to ``degree`` (sh.py:27-28)."""
    return (degree + 1) ** 2


def rgb_to_sh(rgb: torch.Tensor) -> torch.Tensor:
    """RGB in [0, 1] -> DC coefficient (sh.py:31-33)."""
    return (rgb - 0.5) / _C0


def sh_to_rgb(sh_dc: torch.Tensor) -> torch.Tensor:
    """DC coefficient -> RGB (sh.py:36-38)."""
    return sh_dc * _C0 + 0.5


class _EvalSH(torch.autograd.Function):
    @staticmethod
    def forward(ctx, sh, dirs, degree):
        dev = _lib.require_device(sh, dirs)
        n, K, C = sh.shape
        out = torch.empty((n, C), dtype=torch.float32, device=dev)
        L = _lib.load()
        _lib.check(L.gsx_eval_sh_fwd(n, K, C, degree, _lib.ptr(sh), _lib.ptr(dirs), _lib.ptr(out),
                                     _lib.stream_handle(dev)), "gsx_eval_sh_fwd")
        ctx.save_for_backward(sh, dirs)
        ctx.degree = degree
        return out

    @staticmethod
    def backward(ctx, g_out):
        sh, dirs = ctx.saved_tensors
        n, K, C = sh.shape
        dev = sh.device
        g_sh = torch.empty_like(sh)
        g_dirs = torch.empty((n, 3), dtype=torch.float32, device=dev) if ctx.needs_input_grad[1] else None
        g_in = _lib.f32c(g_out)  # kept alive until the kernel has been enqueued
        L = _lib.load()
        _lib.check(L.gsx_eval_sh_bwd(n, K, C, ctx.degree, _lib.ptr(sh), _lib.ptr(dirs),
                                     _lib.ptr(g_in), _lib.ptr(g_sh), _lib.ptr(g_dirs),
                                     _lib.stream_handle(dev)), "gsx_eval_sh_bwd")
        return (g_sh if ctx.needs_input_grad[0] else None), g_dirs, None


def eval_sh(degree: int, sh: torch.Tensor, dirs: torch.Tensor) -> torch.Tensor:
    """Evaluate SH at unit directions (sh.py:41-78).

    Args:
        degree: SH degree in [0, 3].
        sh: (N, K, C) coefficients with K >= (degree+1)^2.
        dirs: (N, 3) unit view directions.

    Returns:
        (N, C) values offset by +0.5 (callers clamp to >= 0).
    """
    if not 0 <= degree <= 3:
        raise ValueError("degree must be in [0, 3].")
    if sh.ndim != 3 or sh.shape[1] < num_sh_bases(degree):
        raise ValueError(f"sh must have shape (N, K>={num_sh_bases(degree)}, C).")
    if dirs.shape != (sh.shape[0], 3):
        raise ValueError("dirs must have shape (N, 3).")
    return _EvalSH.apply(_lib.f32c(sh), _lib.f32c(dirs), int(degree))
