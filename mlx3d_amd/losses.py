"""Image losses of the training step (``src/mlx3d/losses/image_metrics.py``).

``photometric`` returns mean |pred - target| and mean SSIM of one image from
one fused kernel pass (``gsx_photometric_fwd``), and the gradient of any
combination of the two from a second (``gsx_photometric_bwd``).
``photometric_loss`` is the trainer's ``(1 - lambda) L1 + lambda (1 - SSIM)``
(trainer.py:303-305) as one op: the same kernels form the scalar and take
its cotangent (``gsx_photometric_loss_fwd`` / ``_bwd``), the values that
expression's autograd graph gives.  ``ssim`` is the reference's function on
top of ``photometric``, and ``l1_loss`` the L1 term alone
(``gsx_l1_fwd_signs`` / ``gsx_l1_bwd_signs``).
"""

from __future__ import annotations

import torch

from . import _lib
from .profiling import stage

__all__ = ["l1_loss", "photometric", "photometric_loss", "psnr", "ssim"]


class _PhotometricFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, pred, target, window_size, sigma, max_val):
        H, W, C = pred.shape
        L = _lib.load()
        nbytes = int(L.gsx_photometric_workspace_bytes(H, W, C))
        ws = torch.empty((nbytes,), dtype=torch.uint8, device=pred.device)
        out = torch.empty((2,), dtype=torch.float32, device=pred.device)
        with stage("photometric_fwd"):
            _lib.check(L.gsx_photometric_fwd(H, W, C, _lib.ptr(pred), _lib.ptr(target),
                                             int(window_size), float(sigma), float(max_val),
                                             _lib.ptr(ws), nbytes, _lib.ptr(out),
                                             _lib.stream_handle(pred.device)),
                       "gsx_photometric_fwd")
        ctx.save_for_backward(pred, target, ws)
        ctx.window = (int(window_size), float(sigma))
        return out

    @staticmethod
    def backward(ctx, g_out):
        pred, target, ws = ctx.saved_tensors
        H, W, C = pred.shape
        g = _lib.f32c(g_out)
        grad = torch.empty_like(pred)
        with stage("photometric_bwd"):
            _lib.check(_lib.load().gsx_photometric_bwd(
                H, W, C, _lib.ptr(pred), _lib.ptr(target), ctx.window[0], ctx.window[1],
                _lib.ptr(ws), ws.numel(), _lib.ptr(g), _lib.ptr(grad),
                _lib.stream_handle(pred.device)), "gsx_photometric_bwd")
        return grad, None, None, None, None


class _PhotometricLossFn(torch.autograd.Function):
    """(1 - lam) L1 + lam (1 - SSIM) as one op: the scalar comes out of the
    loss kernels' reduction and its gradient goes straight into the SSIM
    backward, the same float32 values the expression's autograd graph
    produces, without its dozen elementwise launches."""

    @staticmethod
    def forward(ctx, pred, target, lam, window_size, sigma, max_val):
        H, W, C = pred.shape
        L = _lib.load()
        nbytes = int(L.gsx_photometric_workspace_bytes(H, W, C))
        ws = torch.empty((nbytes,), dtype=torch.uint8, device=pred.device)
        out = torch.empty((3,), dtype=torch.float32, device=pred.device)
        with stage("photometric_fwd"):
            _lib.check(L.gsx_photometric_loss_fwd(
                H, W, C, _lib.ptr(pred), _lib.ptr(target), int(window_size), float(sigma),
                float(max_val), float(lam), _lib.ptr(ws), nbytes, _lib.ptr(out),
                _lib.stream_handle(pred.device)), "gsx_photometric_loss_fwd")
        ctx.save_for_backward(pred, target, ws)
        ctx.args = (float(lam), int(window_size), float(sigma))
        return out[2]

    @staticmethod
    def backward(ctx, g_out):
        pred, target, ws = ctx.saved_tensors
        lam, window_size, sigma = ctx.args
        H, W, C = pred.shape
        g = _lib.f32c(g_out.reshape(1))
        grad = torch.empty_like(pred)
        with stage("photometric_bwd"):
            _lib.check(_lib.load().gsx_photometric_loss_bwd(
                H, W, C, _lib.ptr(pred), _lib.ptr(target), window_size, sigma, lam,
                _lib.ptr(ws), ws.numel(), _lib.ptr(g), _lib.ptr(grad),
                _lib.stream_handle(pred.device)), "gsx_photometric_loss_bwd")
        return grad, None, None, None, None, None


def _check_window(window_size: int, sigma: float):
    if window_size < 1 or window_size % 2 == 0 or window_size > 15:
        raise ValueError("window_size must be odd and at most 15.")
    if not sigma > 0:
        raise ValueError("sigma must be positive.")


def photometric(pred: torch.Tensor, target: torch.Tensor, window_size: int = 11,
                sigma: float = 1.5, max_val: float = 1.0) -> tuple[torch.Tensor, torch.Tensor]:
    """(mean |pred - target|, mean SSIM) of (H, W, C) images, differentiable
    with respect to ``pred`` (image_metrics.py:13-14, 29-55)."""
    if pred.shape != target.shape or pred.ndim != 3:
        raise ValueError("pred and target must both have shape (H, W, C).")
    _check_window(window_size, sigma)
    _lib.require_device(pred, target)
    out = _PhotometricFn.apply(_lib.f32c(pred), _lib.f32c(target).detach(), window_size, sigma,
                               max_val)
    return out[0], out[1]


def photometric_loss(pred: torch.Tensor, target: torch.Tensor, lam: float,
                     window_size: int = 11, sigma: float = 1.5,
                     max_val: float = 1.0) -> torch.Tensor:
    """The trainer's objective (1 - lam) mean|pred - target| + lam (1 - mean
    SSIM) (trainer.py:303-305) as a scalar tensor, differentiable with
    respect to ``pred``; the same value and gradient, bit for bit, as that
    expression over :func:`photometric`'s two outputs, in two kernel calls."""
    if pred.shape != target.shape or pred.ndim != 3:
        raise ValueError("pred and target must both have shape (H, W, C).")
    _check_window(window_size, sigma)
    if not 0.0 <= float(lam) <= 1.0:
        raise ValueError("lam must lie in [0, 1].")
    _lib.require_device(pred, target)
    return _PhotometricLossFn.apply(_lib.f32c(pred), _lib.f32c(target).detach(), float(lam),
                                    window_size, sigma, max_val)


def ssim(pred: torch.Tensor, target: torch.Tensor, max_val: float = 1.0, window_size: int = 11,
         sigma: float = 1.5) -> torch.Tensor:
    """Mean SSIM with a Gaussian window (image_metrics.py:66-85).  ``pred``
    (H, W, C) or (N, H, W, C); the mean runs over every pixel and channel."""
    if pred.shape != target.shape:
        raise ValueError("pred and target must have the same shape.")
    if pred.ndim == 3:
        return photometric(pred, target, window_size, sigma, max_val)[1]
    if pred.ndim != 4:
        raise ValueError("pred must have shape (H, W, C) or (N, H, W, C).")
    vals = [photometric(pred[i], target[i], window_size, sigma, max_val)[1]
            for i in range(pred.shape[0])]
    return torch.stack(vals).mean()


class _L1Fn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, pred, target):
        n = pred.numel()
        L = _lib.load()
        nbytes = int(L.gsx_l1_workspace_bytes(n))
        ws = torch.empty((max(nbytes, 1),), dtype=torch.uint8, device=pred.device)
        out = torch.empty((1,), dtype=torch.float32, device=pred.device)
        # the signs of pred - target, kept for the backward (1 byte each)
        signs = torch.empty((n,), dtype=torch.uint8, device=pred.device)
        with stage("l1_fwd"):
            _lib.check(L.gsx_l1_fwd_signs(n, _lib.ptr(pred), _lib.ptr(target), _lib.ptr(ws),
                                          nbytes, _lib.ptr(signs), _lib.ptr(out),
                                          _lib.stream_handle(pred.device)), "gsx_l1_fwd_signs")
        ctx.save_for_backward(pred, target, signs)
        return out[0]

    @staticmethod
    def backward(ctx, g_out):
        pred, target, signs = ctx.saved_tensors
        g = _lib.f32c(g_out.reshape(1))
        grad = torch.empty_like(pred)
        with stage("l1_bwd"):
            _lib.check(_lib.load().gsx_l1_bwd_signs(
                pred.numel(), _lib.ptr(signs), _lib.ptr(pred), _lib.ptr(target), _lib.ptr(g),
                _lib.ptr(grad), _lib.stream_handle(pred.device)), "gsx_l1_bwd_signs")
        return grad, None


def l1_loss(pred: torch.Tensor, target: torch.Tensor) -> torch.Tensor:
    """Mean absolute error (image_metrics.py:13-14), differentiable with
    respect to ``pred``: one reduction kernel forward that also keeps the
    sign of each difference, one elementwise gradient kernel backward from
    those signs (gsx_l1_fwd_signs / gsx_l1_bwd_signs)."""
    if pred.shape != target.shape:
        raise ValueError("pred and target must have the same shape.")
    if pred.numel() == 0:
        raise ValueError("l1_loss of empty tensors.")
    _lib.require_device(pred, target)
    return _L1Fn.apply(_lib.f32c(pred), _lib.f32c(target).detach())


def psnr(pred: torch.Tensor, target: torch.Tensor, max_val: float = 1.0) -> torch.Tensor:
    """Peak signal-to-noise ratio in dB (image_metrics.py:17-20)."""
    mse = ((pred - target) ** 2).mean()
    return 10.0 * torch.log10((max_val * max_val) / torch.clamp(mse, min=1e-12))
