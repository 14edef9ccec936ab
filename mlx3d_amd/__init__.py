"""mlx3d_amd -- MI355X-native (gfx950) tile-based 3D Gaussian-splatting
rasterizer with the API of mlx3D's splatting path.

Compute runs in hand-written HIP kernels (``libgsx.so``, C ABI in
``include/gsx.h``) on PyTorch-ROCm device memory and streams.
"""

__version__ = "0.1.0"

from . import cameras, renderer, splatting  # noqa: F401
from .cameras import Camera  # noqa: F401
