"""splax_amd: the MI355X (gfx950) gaussian-splat render path.

A drop-in for the render path of amacati/splax (``render`` / ``render_log`` / ``project`` /
``rasterize`` / ``opacity_compensation`` / ``clear_cache``, and the ``mcmc`` and ``utils`` modules,
splax/__init__.py:30-47; ``io``, the dataset loader, is not part of the path) on torch-ROCm
tensors. Projection, tile intersection, sort, binning and blend, forward and backward, run as
hand-written gfx950 HIP kernels behind the C ABI in ``include/splat_hip.h`` (libsplat_hip.so,
loaded by ``splax_amd._lib``).
"""

__version__ = "0.1.0"

from splax_amd import mcmc, utils
from splax_amd._ops import clear_cache
from splax_amd._project import opacity_compensation, project, transform_ids
from splax_amd._rasterize import rasterize, rasterize_depth
from splax_amd._render import render, render_log, render_log_loss, render_loss

__all__ = [
    "clear_cache",
    "opacity_compensation",
    "project",
    "rasterize",
    "rasterize_depth",
    "render",
    "render_log",
    "render_log_loss",
    "render_loss",
    "transform_ids",
    "mcmc",
    "utils",
]
