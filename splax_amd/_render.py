"""Rendering entry points (torch), mirroring splax/_render.py:29-168.

``render`` composes ``project`` and ``rasterize``; ``render_log`` maps the unconstrained
log / logit parameterization first. A leading batch dimension on ``viewmat`` (B, 4, 4) renders B
cameras in one batched launch (the reference's ``jax.vmap(render)`` path).
"""

from __future__ import annotations

from collections.abc import Sequence

import torch

from splax_amd._project import project, transform_ids
from splax_amd._rasterize import _rasterize_checked


def render(means3d: torch.Tensor, scales: torch.Tensor, quats: torch.Tensor,
           colors: torch.Tensor, opacities: torch.Tensor, *, viewmat: torch.Tensor,
           background: torch.Tensor, img_shape: tuple[int, int], f: tuple[float, float],
           c: tuple[float, float] | None = None, glob_scale: float = 1.0,
           clip_thresh: float = 0.01, antialiased: bool = False, render_depth: bool = False,
           gaussian_transforms: torch.Tensor | None = None,
           gaussian_slices: Sequence[tuple[int, int]] | None = None):
    """Render a splat; returns (image, depth-or-None) like splax.render (splax/_render.py:29-115)."""
    if (gaussian_transforms is None) != (gaussian_slices is None):
        raise ValueError("gaussian_transforms and gaussian_slices must be passed together")
    tf_ids = None
    if gaussian_transforms is not None and gaussian_slices is not None:
        if tuple(gaussian_transforms.shape[-3:]) != (len(gaussian_slices), 4, 4):
            raise ValueError(
                f"gaussian_transforms shape {tuple(gaussian_transforms.shape)} does not "
                f"match {len(gaussian_slices)} slices, expected (K, 4, 4)")
        tf_ids = transform_ids(means3d.shape[-2], gaussian_slices, device=means3d.device)
    xys, depths, radii, conics, _, cum = project(
        means3d, scales, quats, viewmat, opacities=opacities, img_shape=img_shape, f=f, c=c,
        glob_scale=glob_scale, clip_thresh=clip_thresh, gaussian_transforms=gaussian_transforms,
        transform_ids=tf_ids)
    # antialiased: the blend uses opacities * opacity_compensation(conics, radii) and the tile
    # intersection the raw opacities (splax/_render.py:105-110); the library evaluates the
    # compensation and its gradient inside the blend's record packing and gradient gather.
    img, depth = _rasterize_checked(colors, opacities, background, xys, depths, radii, conics,
                                    cum, img_shape, None, render_depth, compensate=antialiased)
    return img, depth


def render_log(means3d: torch.Tensor, log_scales: torch.Tensor, quats: torch.Tensor,
               logit_colors: torch.Tensor, logit_opacities: torch.Tensor, *,
               viewmat: torch.Tensor, background: torch.Tensor, img_shape: tuple[int, int],
               f: tuple[float, float], c: tuple[float, float] | None = None,
               glob_scale: float = 1.0, clip_thresh: float = 0.01, antialiased: bool = False,
               render_depth: bool = False):
    """Render from log scales / logits (splax/_render.py:118-168)."""
    scales = torch.exp(log_scales)
    quats = quats / (torch.linalg.norm(quats, dim=-1, keepdim=True) + 1e-8)
    colors = torch.sigmoid(logit_colors)
    opacities = torch.sigmoid(logit_opacities)
    return render(means3d, scales, quats, colors, opacities, viewmat=viewmat,
                  background=background, img_shape=img_shape, f=f, c=c, glob_scale=glob_scale,
                  clip_thresh=clip_thresh, antialiased=antialiased, render_depth=render_depth)
