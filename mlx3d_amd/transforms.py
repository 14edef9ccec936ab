"""Rotation helper the training step uses (``src/mlx3d/transforms/rotations.py``)."""

from __future__ import annotations

import torch

__all__ = ["quaternion_to_matrix"]


def quaternion_to_matrix(quaternions: torch.Tensor) -> torch.Tensor:
    """(..., 4) quaternions, (w, x, y, z), to (..., 3, 3) rotation matrices
    (rotations.py:30-49): normalised first, then the standard matrix."""
    q = quaternions / torch.linalg.norm(quaternions, dim=-1, keepdim=True)
    w, x, y, z = q.unbind(-1)
    m = torch.stack([
        1 - 2.0 * (y * y + z * z), 2.0 * (x * y - w * z), 2.0 * (x * z + w * y),
        2.0 * (x * y + w * z), 1 - 2.0 * (x * x + z * z), 2.0 * (y * z - w * x),
        2.0 * (x * z - w * y), 2.0 * (y * z + w * x), 1 - 2.0 * (x * x + y * y),
    ], dim=-1)
    return m.reshape(*quaternions.shape[:-1], 3, 3)
