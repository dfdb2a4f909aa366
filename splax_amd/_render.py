"""Rendering entry points (torch), mirroring splax/_render.py:29-168.

``render`` composes ``project`` and ``rasterize``; ``render_log`` maps the unconstrained
log / logit parameterization first. A leading batch dimension on ``viewmat`` (B, 4, 4) renders B
cameras in one batched launch (the reference's ``jax.vmap(render)`` path).
"""

from __future__ import annotations

from collections.abc import Sequence

import torch

from splax_amd import _lib
from splax_amd._project import project, transform_ids
from splax_amd._rasterize import _rasterize_checked


class _LogParamsFn(torch.autograd.Function):
    """exp(log_scales), quats / (|quats| + 1e-8), sigmoid(logit_colors), sigmoid(logit_opac)
    (splax/_render.py:161-164) over flat rows."""

    @staticmethod
    def forward(ctx, log_scales, quats, logit_colors, logit_opacities):
        n = log_scales.numel() // 3
        for name, t, w in (("log_scales", log_scales, 3), ("quats", quats, 4),
                           ("logit_colors", logit_colors, 3),
                           ("logit_opacities", logit_opacities, 1)):
            if t.dtype != torch.float32 or t.numel() != n * w:
                raise ValueError(f"{name} must be float32 with {w} values for each of {n} rows")
        ins = [t.contiguous() for t in (log_scales, quats, logit_colors, logit_opacities)]
        dev = _lib.require_gpu(*ins)
        outs = [torch.empty_like(t) for t in ins]
        p = _lib.ptr
        with torch.cuda.device(dev):
            st = _lib.lib().splat_log_params_fwd(_lib.stream_handle(dev), *map(p, ins), n,
                                                 *map(p, outs))
        _lib.check(st, "log_params_fwd")
        ctx.save_for_backward(*ins)
        ctx.set_materialize_grads(False)
        return tuple(outs)

    @staticmethod
    def backward(ctx, v_scales, v_quats, v_colors, v_opac):
        ins = ctx.saved_tensors
        n = ins[0].numel() // 3
        vs = [None if v is None else v.contiguous() for v in (v_scales, v_quats, v_colors,
                                                               v_opac)]
        outs = [torch.empty_like(t) for t in ins]
        dev = ins[0].device
        p = _lib.ptr
        with torch.cuda.device(dev):
            st = _lib.lib().splat_log_params_bwd(_lib.stream_handle(dev), *map(p, ins), n,
                                                 *map(p, vs), *map(p, outs))
        _lib.check(st, "log_params_bwd")
        return tuple(outs)


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
    """Render from log scales / logits (splax/_render.py:118-168); the parameter map and its
    gradient run as one library pass each (splat_log_params_fwd / _bwd)."""
    scales, quats, colors, opacities = _LogParamsFn.apply(log_scales, quats, logit_colors,
                                                          logit_opacities)
    return render(means3d, scales, quats, colors, opacities, viewmat=viewmat,
                  background=background, img_shape=img_shape, f=f, c=c, glob_scale=glob_scale,
                  clip_thresh=clip_thresh, antialiased=antialiased, render_depth=render_depth)
