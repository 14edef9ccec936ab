"""Row order of the Gaussian table (no counterpart in the reference, whose
rows keep the order they were created in).

The rasterizers gather each tile's Gaussians by id: positions, conics and
opacities, colours, and in the backward the gradient record's atomics.  In
creation order the Gaussians of one tile lie anywhere in the table, so every
gather pulls its own cache lines from HBM.  Stored in 3D Morton (Z-order)
order of their means, Gaussians that are close in space -- and so tend to
cover the same tiles -- share cache lines, and a tile's gathers hit in L2.
The order changes no rendered value: it permutes the rows, and the depth
sort breaks equal depths by row, so only Gaussians at exactly the same depth
can swap their compositing order.
"""

from __future__ import annotations

import torch

__all__ = ["spatial_order"]

_BITS = 10  # per axis: a 2^30-cell grid over the means' bounding box


def _spread(v: torch.Tensor) -> torch.Tensor:
    """The 10 low bits of v moved to bit positions 0, 3, 6, ..., 27."""
    v = v & 0x3FF
    v = (v | (v << 16)) & 0x030000FF
    v = (v | (v << 8)) & 0x0300F00F
    v = (v | (v << 4)) & 0x030C30C3
    v = (v | (v << 2)) & 0x09249249
    return v


def morton_codes(means: torch.Tensor) -> torch.Tensor:
    """30-bit Morton codes (int64) of the (N, 3) means, quantised to a
    1024^3 grid over their bounding box.  Non-finite coordinates count as
    the box's lower corner (NaN) or its bounds (+-inf)."""
    if means.ndim != 2 or means.shape[1] != 3:
        raise ValueError("spatial_order: means must be (N, 3)")
    m = torch.nan_to_num(means.detach().to(torch.float64), nan=0.0, posinf=0.0, neginf=0.0)
    if m.shape[0] == 0:
        return torch.zeros(0, dtype=torch.int64, device=means.device)
    lo, hi = m.amin(0), m.amax(0)
    cells = (1 << _BITS) - 1
    q = ((m - lo) * (cells / torch.clamp(hi - lo, min=1e-30))).to(torch.int64)
    q = q.clamp_(0, cells)
    return _spread(q[:, 0]) | (_spread(q[:, 1]) << 1) | (_spread(q[:, 2]) << 2)


def spatial_order(means: torch.Tensor) -> torch.Tensor:
    """The permutation (int64, on the means' device) that sorts the rows by
    the Morton code of their means, ties in row order: ``table[perm]`` is
    the table in spatial order."""
    return torch.argsort(morton_codes(means), stable=True)
