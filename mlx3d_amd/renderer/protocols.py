"""The renderer convention (``src/mlx3d/renderer/protocols.py:32-62``).

Every image-space renderer is a callable ``renderer(camera, *scene) ->
RenderOutput``; ``GaussianModel.render`` and ``render_gaussians`` follow it.
"""

from __future__ import annotations

from typing import Protocol, TypedDict, runtime_checkable

import torch

from ..cameras import Camera

__all__ = ["RenderOutput", "Renderer"]


class RenderOutput(TypedDict, total=False):
    """``image`` (H, W, 3) in [0, 1], ``alpha`` (H, W), ``depth`` (H, W).

    Renderers may attach extra keys (``means2d``, ``radii`` ...); consumers
    read by key.
    """

    image: torch.Tensor
    alpha: torch.Tensor
    depth: torch.Tensor


@runtime_checkable
class Renderer(Protocol):
    """Anything callable as ``renderer(camera, *scene) -> RenderOutput``."""

    def __call__(self, camera: Camera, *args: object, **kwargs: object) -> RenderOutput: ...
