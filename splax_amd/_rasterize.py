"""Differentiable rasterization stage (torch).

Mirrors splax/_rasterize/_rasterize.py:24-234: ``rasterize`` blends projected gaussians into an
image; ``_RasterizeFn`` is the counterpart of the ``jax.custom_vjp`` ``_rasterize`` whose forward
keeps final_Ts / final_idx as residuals and whose backward recomputes the (deterministic) sort
inside the library. Differentiable w.r.t. colors, opacities, xys and conics.
"""

from __future__ import annotations

import torch

from splax_amd import _ops
from splax_amd._project import resolve_batch


class _RasterizeFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, colors, opac, map_opac, background, xys, depths, radii, conics, cum,
                statics):
        n, B, img_shape = statics
        img, Ts, fidx, _ = _ops.rasterize_fwd(
            colors.reshape(-1, 3), opac.reshape(-1), map_opac.reshape(-1),
            background.reshape(-1, 3), xys.reshape(-1, 2), depths.reshape(-1), radii.reshape(-1),
            conics.reshape(-1, 3), cum.reshape(-1), n=n, B=B, img_shape=img_shape)
        ctx.save_for_backward(colors, opac, map_opac, background, xys, depths, radii, conics,
                              cum, Ts, fidx)
        ctx.statics = statics
        ctx.mark_non_differentiable(Ts, fidx)
        return img, Ts, fidx

    @staticmethod
    def backward(ctx, v_img, _v_Ts, _v_idx):
        colors, opac, map_opac, background, xys, depths, radii, conics, cum, Ts, fidx = \
            ctx.saved_tensors
        n, B, img_shape = ctx.statics
        if v_img is None:
            v_img = torch.zeros((B * img_shape[0], img_shape[1], 3), device=xys.device)
        v_colors, v_opac, v_xy, v_conic = _ops.rasterize_bwd(
            colors.reshape(-1, 3), opac.reshape(-1), map_opac.reshape(-1),
            background.reshape(-1, 3), xys.reshape(-1, 2), depths.reshape(-1), radii.reshape(-1),
            conics.reshape(-1, 3), cum.reshape(-1), Ts, fidx, v_img.reshape(-1, 3), n=n,
            B_out=B, B_geom=B, img_shape=img_shape)

        def fold(g: torch.Tensor, like: torch.Tensor) -> torch.Tensor:
            if like.numel() == g.numel():
                return g.reshape(like.shape)
            return g.reshape(B, -1).sum(0).reshape(like.shape)  # shared over the batch

        return (fold(v_colors, colors), fold(v_opac, opac), None, None, fold(v_xy, xys), None,
                None, fold(v_conic, conics), None, None)


def rasterize(colors: torch.Tensor, opacities: torch.Tensor, background: torch.Tensor,
              xys: torch.Tensor, depths: torch.Tensor, radii: torch.Tensor, conics: torch.Tensor,
              cum_tiles_hit: torch.Tensor, *, img_shape: tuple[int, int],
              map_opacities: torch.Tensor | None = None) -> torch.Tensor:
    """Blend projected gaussians into an (H, W, 3) image (splax/_rasterize/_rasterize.py:24-60).

    Geometry (xys, depths, radii, conics, cum_tiles_hit) with a leading batch dimension B renders
    B images in one launch and returns (B, H, W, 3); colors / opacities may be shared (N, ...) or
    per image (B, N, ...), background (3,) or (B, 3). map_opacities (default: opacities) drive the
    tile intersection only and carry no gradient.
    """
    n = int(colors.shape[-2])
    H, W = img_shape
    if map_opacities is None:
        map_opacities = opacities
    B = resolve_batch(xys=(xys, 2), conics=(conics, 2))
    batched = B is not None
    Bg = B if batched else 1
    if cum_tiles_hit.numel() != Bg * n or xys.numel() != Bg * n * 2:
        raise ValueError(
            f"geometry rows ({xys.numel() // 2}) do not match {Bg} image(s) of {n} gaussians")
    for name, t, w in (("colors", colors, 3), ("opacities", opacities, 1),
                       ("map_opacities", map_opacities, 1)):
        r = t.numel() // w
        if r not in (n, Bg * n):
            raise ValueError(f"{name} has {r} rows, expected {n} or {Bg * n}")
    if background.numel() not in (3, 3 * Bg):
        raise ValueError(f"background must have 3 or {3 * Bg} entries")
    img, _, _ = _RasterizeFn.apply(colors, opacities, map_opacities, background, xys, depths,
                                   radii, conics, cum_tiles_hit, (n, Bg, (int(H), int(W))))
    return img.reshape(Bg, H, W, 3) if batched else img.reshape(H, W, 3)


def rasterize_depth(*args, **kwargs):
    """Expected-depth twin of rasterize (splax/_rasterize/_rasterize.py:63-99): not built yet."""
    raise NotImplementedError("rasterize_depth (the expected-depth channel) is not built yet")
