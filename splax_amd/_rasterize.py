"""Differentiable rasterization stage (torch).

Mirrors splax/_rasterize/_rasterize.py:24-360: ``rasterize`` blends projected gaussians into an
image and ``rasterize_depth`` adds the expected-depth map; ``_RasterizeFn`` is the counterpart of
the ``jax.custom_vjp`` rules ``_rasterize`` / ``_rasterize_depth``, whose forward keeps final_Ts /
final_idx (here also the sorted lists) as residuals. Differentiable w.r.t. colors, opacities, xys
and conics, and on the depth path also depths.
"""

from __future__ import annotations

import math

import torch

from splax_amd import _ops
from splax_amd._batching import batch_shape, fold, shared_background


def key_layout(B: int, H: int, W: int) -> dict:
    """Fields of the sort key (splax/_rasterize/_sort/_sort.py:51-66): the packed 32-bit key when
    at least 16 depth bits remain, else the 64-bit key, which overflows past 32 image + tile bits.
    """
    tx, ty = (W + 15) // 16, (H + 15) // 16
    nt = tx * ty
    tile_bits = (nt - 1).bit_length()
    image_bits = (B - 1).bit_length()
    depth_bits = 31 - image_bits - tile_bits
    packed = depth_bits >= 16
    return {"tiles_x": tx, "tiles_y": ty, "num_tiles": nt, "tile_bits": tile_bits,
            "image_bits": image_bits, "depth_bits": depth_bits, "packed": packed,
            "overflow": not packed and image_bits + tile_bits > 32}


def check_key_fits(B: int, H: int, W: int) -> None:
    """Raise like the reference when even the 64-bit key cannot hold the image and tile ids
    (splax/_rasterize/_sort/_sort.py:61-66)."""
    lay = key_layout(B, H, W)
    if lay["overflow"]:
        upper = lay["image_bits"] + lay["tile_bits"]
        raise ValueError(
            f"batched intersection key overflow: image_n_bits({lay['image_bits']}) + "
            f"tile_n_bits({lay['tile_bits']}) = {upper} > 32 (batch B={B}, "
            f"n_tiles={lay['num_tiles']}). Reduce batch size or resolution.")


class _RasterizeFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, colors, opac, map_opac, background, xys, depths, radii, conics, cum,
                statics):
        n, B, img_shape, render_depth, compensate = statics
        # The sorted lists stay resident for the backward (the reference re-sorts there,
        # splax/_rasterize/_kernels.py:422); the sort is deterministic, so both are identical.
        img, Ts, fidx, kept, depth = _ops.rasterize_fwd_keep(
            colors.reshape(-1, 3), opac.reshape(-1), map_opac.reshape(-1),
            background.reshape(-1, 3), xys.reshape(-1, 2), depths.reshape(-1), radii.reshape(-1),
            conics.reshape(-1, 3), cum.reshape(-1), n=n, B=B, img_shape=img_shape,
            render_depth=render_depth, compensate=compensate)
        ctx.save_for_backward(colors, opac, background, xys, depths, conics, cum, Ts, fidx,
                              kept.ids, kept.pos, kept.bins, kept.records, kept.order)
        ctx.statics = statics
        ctx.num_intersects = kept.M
        ctx.set_materialize_grads(False)  # no zero tensors for the unused Ts / fidx grads
        if depth is None:
            depth = Ts.new_empty(())  # placeholder output of the colour-only path (never read)
            ctx.mark_non_differentiable(Ts, fidx, depth)  # one call: it replaces the set
        else:
            ctx.mark_non_differentiable(Ts, fidx)
        return img, depth, Ts, fidx

    @staticmethod
    def backward(ctx, v_img, v_depth, _v_Ts, _v_idx):
        (colors, opac, background, xys, depths, conics, cum, Ts, fidx, ids, pos, bins, recs,
         order) = ctx.saved_tensors
        n, B, img_shape, render_depth, compensate = ctx.statics
        H, W = img_shape
        if v_img is None:
            v_img = torch.zeros((B * H, W, 3), device=xys.device)
        if render_depth and v_depth is None:
            v_depth = torch.zeros((B * H, W), device=xys.device)
        fold_here = B > 1 and colors.numel() == n * 3 and opac.numel() == n
        grads = _ops.rasterize_bwd_sorted(
            colors.reshape(-1, 3), opac.reshape(-1), background.reshape(-1, 3),
            xys.reshape(-1, 2), depths.reshape(-1), conics.reshape(-1, 3), cum.reshape(-1),
            _ops.KeptSort(ids, pos, bins, ctx.num_intersects, recs, order), Ts, fidx,
            v_img.reshape(-1, 3), n=n, B_out=B,
            B_geom=B, img_shape=img_shape,
            v_out_depth=v_depth.reshape(-1, W) if render_depth else None, compensate=compensate,
            fold=fold_here)
        v_colors, v_opac, v_xy, v_conic = grads[:4]

        def rows_of(g: torch.Tensor, like: torch.Tensor) -> torch.Tensor:
            if like.numel() == g.numel():
                return g.reshape(like.shape)
            return g.reshape(B, -1).sum(0).reshape(like.shape)  # shared over the batch

        # the depths cotangent exists only on the depth path
        # (splax/_rasterize/_rasterize.py:231 vs :357)
        v_depths = rows_of(grads[4], depths) if render_depth else None
        return (rows_of(v_colors, colors), rows_of(v_opac, opac), None, None, rows_of(v_xy, xys),
                v_depths, None, rows_of(v_conic, conics), None, None)


def _rasterize_checked(colors, opacities, background, xys, depths, radii, conics, cum_tiles_hit,
                       img_shape, map_opacities, render_depth, compensate=False):
    """compensate: ``opacities`` are raw and the blend uses opacities * rho(conics), the
    antialiased render of splax/_render.py:105-110 fused into the library's kernels."""
    n = int(colors.shape[-2])
    H, W = img_shape
    if map_opacities is None:
        map_opacities = opacities
    per_g = lambda t: t.reshape(*t.shape[:-2], n) if t.ndim >= 2 and t.shape[-1] == 1 \
        and t.shape[-2] == n else t  # noqa: E731 ((..., N, 1) -> (..., N))
    opacities, map_opacities = per_g(opacities), per_g(map_opacities)
    background = shared_background(background)
    glead = tuple(xys.shape[:-2])
    G = math.prod(glead)
    if (depths.numel() != G * n or radii.numel() != G * n or cum_tiles_hit.numel() != G * n
            or conics.numel() != G * n * 3):
        raise ValueError(
            f"geometry rows ({xys.numel() // 2}) do not match {G} image(s) of {n} gaussians")
    # geometry, colours, opacities and background broadcast to one batch shape, folded into one
    # flat batch (the nested vmap of splax/_batching.py)
    S = batch_shape(dict(xys=(xys, 2), conics=(conics, 2), colors=(colors, 2),
                         opacities=(opacities, 1), map_opacities=(map_opacities, 1),
                         background=(background, 1)))
    Bg = math.prod(S) if S else 1
    if S:
        if G == Bg:
            xys, conics = xys.reshape(Bg, n, 2), conics.reshape(Bg, n, 3)
            depths, radii = depths.reshape(Bg, n), radii.reshape(Bg, n)
            cum_tiles_hit = cum_tiles_hit.reshape(Bg * n)
        else:
            # geometry batched over some axes only: the library takes one geometry item per
            # (image, gaussian), so it is tiled / repeated like any partly batched operand, and
            # the tile-count prefix, global over the batch, is formed again for the new order
            xys, conics = fold(xys, 2, S, True), fold(conics, 2, S, True)
            depths = fold(depths.reshape(*glead, n), 1, S, True)
            radii = fold(radii.reshape(*glead, n), 1, S, True)
            flat = cum_tiles_hit.reshape(-1).to(torch.int64)
            nth = torch.diff(flat, prepend=flat.new_zeros(1))
            nth = fold(nth.reshape(*glead, n), 1, S, True)
            cum_tiles_hit = torch.cumsum(nth.reshape(-1), 0).to(torch.int32)
        colors, opacities = fold(colors, 2, S), fold(opacities, 1, S)
        map_opacities, background = fold(map_opacities, 1, S), fold(background, 1, S)
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
    if depths.numel() != Bg * n:
        raise ValueError(f"depths has {depths.numel()} entries, expected {Bg * n}")
    check_key_fits(Bg, int(H), int(W))
    img, depth, _, _ = _RasterizeFn.apply(colors, opacities, map_opacities, background, xys,
                                          depths, radii, conics, cum_tiles_hit,
                                          (n, Bg, (int(H), int(W)), render_depth,
                                           bool(compensate)))
    img = img.reshape(*S, H, W, 3)
    if not render_depth:
        return img, None
    return img, depth.reshape(*S, H, W)


def rasterize(colors: torch.Tensor, opacities: torch.Tensor, background: torch.Tensor,
              xys: torch.Tensor, depths: torch.Tensor, radii: torch.Tensor, conics: torch.Tensor,
              cum_tiles_hit: torch.Tensor, *, img_shape: tuple[int, int],
              map_opacities: torch.Tensor | None = None) -> torch.Tensor:
    """Blend projected gaussians into an (H, W, 3) image (splax/_rasterize/_rasterize.py:24-60).

    Geometry (xys, depths, radii, conics, cum_tiles_hit) with leading batch dimensions S (as
    project returns them for batched cameras) renders prod(S) images in one launch and returns
    (*S, H, W, 3); colors / opacities may be shared (N, ...) or batched (..., N, ...), background
    (3,) or (..., 3), all broadcast against S (the nested vmap of splax/_batching.py).
    map_opacities (default: opacities) drive the tile intersection only and carry no gradient.
    """
    return _rasterize_checked(colors, opacities, background, xys, depths, radii, conics,
                              cum_tiles_hit, img_shape, map_opacities, False)[0]


def rasterize_depth(colors: torch.Tensor, opacities: torch.Tensor, background: torch.Tensor,
                    xys: torch.Tensor, depths: torch.Tensor, radii: torch.Tensor,
                    conics: torch.Tensor, cum_tiles_hit: torch.Tensor, *,
                    img_shape: tuple[int, int], map_opacities: torch.Tensor | None = None):
    """rasterize plus the alpha-blended expected depth map (splax/_rasterize/_rasterize.py:63-99).

    Returns (image (H, W, 3), depth (H, W)), batched as rasterize. The depth uses the colour
    blend's weights and no background term; the image is bit-for-bit rasterize's. Gradients flow
    to depths as well (splax/_rasterize/_rasterize.py:316-357).
    """
    return _rasterize_checked(colors, opacities, background, xys, depths, radii, conics,
                              cum_tiles_hit, img_shape, map_opacities, True)
