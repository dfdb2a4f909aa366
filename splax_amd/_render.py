"""Rendering entry points (torch), mirroring splax/_render.py:29-168.

``render`` composes ``project`` and ``rasterize``; ``render_log`` maps the unconstrained
log / logit parameterization first. A leading batch dimension on ``viewmat`` (B, 4, 4) renders B
cameras in one batched launch (the reference's ``jax.vmap(render)`` path).
"""

from __future__ import annotations

from collections.abc import Sequence

import torch

import math

from splax_amd import _lib, _ops
from splax_amd._batching import batch_shape, fold, shared_background
from splax_amd._project import _no_transforms, transform_ids
from splax_amd._rasterize import check_key_fits


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


def _fused_forward(means, scales, quats, colors, opac, viewmat, background, transforms, tf_ids,
                   statics, backward, loss=None):
    """splat_render_fwd over the flat operands; backward=False when no render_bwd will read the
    kept lists (the sort then carries no emission positions). loss: (kind, target, out) fuses the
    pixel loss into the blend, its value into out."""
    n, B, K, has_tf, img_shape, f, c, glob_scale, clip_thresh, compensate, render_depth = statics
    flat = lambda t, w: t.reshape(-1, w) if w > 1 else t.reshape(-1)  # noqa: E731
    kind, target, out = loss if loss is not None else (0, None, None)
    return _ops.render_fwd(
        flat(means, 3), flat(scales, 3), flat(quats, 4), flat(colors, 3), flat(opac, 1),
        viewmat.reshape(-1, 4), flat(background, 3), transforms.reshape(-1, 4, 4),
        tf_ids.reshape(-1), n=n, B=B, num_transforms=K, has_transforms=has_tf,
        img_shape=img_shape, f=f, c=c, glob_scale=glob_scale, clip_thresh=clip_thresh,
        compensate=compensate, render_depth=render_depth, backward=backward, loss_kind=kind,
        loss_target=target, loss_out=out)


def _save_forward(ctx, operands, Ts, fidx, kept, statics, extra=()):
    ks = kept.sort
    ctx.save_for_backward(*operands, Ts, fidx, kept.xys, kept.depths, kept.radii, kept.conics,
                          kept.cum, ks.ids, ks.pos, ks.bins, ks.records, ks.order, *extra)
    ctx.statics = statics
    ctx.num_intersects = ks.M
    ctx.set_materialize_grads(False)


def _backward(ctx, v_img, v_depth, loss=None):
    """splat_render_bwd for a forward saved by _save_forward; loss: (kind, target, image,
    v_loss) when the forward fused the loss (v_img then unused). Returns the cotangents of
    means, scales, quats, colors, opacities, viewmat and transforms."""
    (means, scales, quats, colors, opac, viewmat, background, transforms, tf_ids, Ts, fidx,
     xys, depths, radii, conics, cum, ids, pos, bins, recs, order) = ctx.saved_tensors[:21]
    n, B, K, has_tf, img_shape, f, c, glob_scale, clip_thresh, compensate, render_depth = \
        ctx.statics
    H, W = img_shape
    if v_img is None and loss is None:
        v_img = torch.zeros((B * H, W, 3), device=means.device)
    if render_depth and v_depth is None:
        v_depth = torch.zeros((B * H, W), device=means.device)
    shared = [t.numel() == n * w for t, w in ((means, 3), (scales, 3), (quats, 4),
                                              (colors, 3), (opac, 1))]
    fold_here = B > 1 and all(shared)
    flat = lambda t, w: t.reshape(-1, w) if w > 1 else t.reshape(-1)  # noqa: E731
    kept = _ops.RenderKept(xys, depths, radii, conics, cum,
                           _ops.KeptSort(ids, pos, bins, ctx.num_intersects, recs, order))
    kind, target, image, v_loss = loss if loss is not None else (0, None, None, None)
    gm, gs, gq, gc, go, gv, gt = _ops.render_bwd(
        flat(means, 3), flat(scales, 3), flat(quats, 4), flat(colors, 3), flat(opac, 1),
        viewmat.reshape(-1, 4), flat(background, 3), transforms.reshape(-1, 4, 4),
        tf_ids.reshape(-1), kept, Ts, fidx, None if v_img is None else v_img.reshape(-1, 3),
        n=n, B=B, num_transforms=K, has_transforms=has_tf, img_shape=img_shape, f=f,
        glob_scale=glob_scale, compensate=compensate,
        v_out_depth=v_depth.reshape(-1, W) if render_depth else None, fold=fold_here,
        want_viewmat=ctx.needs_input_grad[5], loss_kind=kind, loss_target=target,
        out_img=image, v_loss=v_loss)

    def rows_of(g: torch.Tensor, like: torch.Tensor, w: int) -> torch.Tensor:
        if g.numel() == like.numel():  # batched, one image, or folded by the library
            return g.reshape(like.shape)
        g = g.reshape(B, n, w) if w > 1 else g.reshape(B, n)
        return g.sum(0).reshape(like.shape)  # shared operand: sum over the batch

    need = ctx.needs_input_grad
    g_view = None
    if need[5]:
        g_view = gv.reshape(B, 4, 4)
        g_view = g_view.reshape(viewmat.shape) if viewmat.ndim == 3 else g_view.sum(0)
    g_tf = None
    if has_tf and need[7]:
        g_tf = gt.reshape(B, K, 4, 4)
        g_tf = g_tf.reshape(transforms.shape) if transforms.ndim == 4 else g_tf.sum(0)
    return (rows_of(gm, means, 3) if need[0] else None,
            rows_of(gs, scales, 3) if need[1] else None,
            rows_of(gq, quats, 4) if need[2] else None,
            rows_of(gc, colors, 3) if need[3] else None,
            rows_of(go, opac, 1) if need[4] else None,
            g_view, g_tf)


class _RenderFn(torch.autograd.Function):
    """project then rasterize (splax/_render.py:94-115) with their custom VJPs
    (splax/_project/_project.py:142-275, splax/_rasterize/_rasterize.py:105-234) as one library
    forward and one library backward (splat_render_fwd / splat_render_bwd): the projection packs
    the blend records and the depth range, and the backward keeps the per-item 2D cotangents in
    library scratch. Operands are shared ([n, ...]) or batched ([B, n, ...]); the forward
    keeps the projection outputs and the sorted lists as residuals."""

    @staticmethod
    def forward(ctx, means, scales, quats, colors, opac, viewmat, background, transforms, tf_ids,
                statics):
        operands = (means, scales, quats, colors, opac, viewmat, background, transforms, tf_ids)
        img, Ts, fidx, kept, depth = _fused_forward(*operands, statics, backward=True)
        _save_forward(ctx, operands, Ts, fidx, kept, statics)
        if depth is None:
            depth = Ts.new_empty(())  # placeholder output of the colour-only path (never read)
            ctx.mark_non_differentiable(depth)
        return img, depth

    @staticmethod
    def backward(ctx, v_img, v_depth):
        gm, gs, gq, gc, go, gv, gt = _backward(ctx, v_img, v_depth)
        return gm, gs, gq, gc, go, gv, None, gt, None, None


class _RenderLossFn(torch.autograd.Function):
    """render's forward and backward with a pixel loss against a target fused into the blends:
    the forward blend sums each tile's loss terms as it writes the image, and the backward blend
    forms each pixel's image cotangent from the image, the target and the loss cotangent, so the
    loss's own passes over the image (two reads forward, two reads and a write backward) do not
    run. Outputs: the loss (differentiable) and the image (not)."""

    @staticmethod
    def forward(ctx, means, scales, quats, colors, opac, viewmat, background, transforms, tf_ids,
                target, statics, kind):
        operands = (means, scales, quats, colors, opac, viewmat, background, transforms, tf_ids)
        loss = torch.empty((), device=means.device, dtype=torch.float32)
        img, Ts, fidx, kept, _ = _fused_forward(*operands, statics, backward=True,
                                                loss=(kind, target, loss))
        _save_forward(ctx, operands, Ts, fidx, kept, statics, extra=(img, target))
        ctx.kind = kind
        ctx.mark_non_differentiable(img)
        return loss, img

    @staticmethod
    def backward(ctx, v_loss, _v_img):
        img, target = ctx.saved_tensors[21:]
        if v_loss is None:
            return (None,) * 12
        v_loss = v_loss.to(torch.float32).contiguous()
        gm, gs, gq, gc, go, gv, gt = _backward(ctx, None, None,
                                               loss=(ctx.kind, target, img, v_loss))
        return gm, gs, gq, gc, go, gv, None, gt, None, None, None, None


def _prepare(means3d, scales, quats, colors, opacities, viewmat, background, img_shape, f, c,
             glob_scale, clip_thresh, antialiased, render_depth, gaussian_transforms,
             gaussian_slices):
    """Operands folded into one flat batch, transform ids and the statics of a render call;
    returns (ops, tf_ids, statics, batch shape)."""
    if (gaussian_transforms is None) != (gaussian_slices is None):
        raise ValueError("gaussian_transforms and gaussian_slices must be passed together")
    n = int(means3d.shape[-2])
    if c is None:
        c = (img_shape[1] / 2, img_shape[0] / 2)
    dev = means3d.device
    if gaussian_transforms is not None and gaussian_slices is not None:
        if tuple(gaussian_transforms.shape[-3:]) != (len(gaussian_slices), 4, 4):
            raise ValueError(
                f"gaussian_transforms shape {tuple(gaussian_transforms.shape)} does not "
                f"match {len(gaussian_slices)} slices, expected (K, 4, 4)")
        tf_ids = transform_ids(n, gaussian_slices, device=dev)
        has_tf, K = True, len(gaussian_slices)
    else:
        gaussian_transforms, tf_ids = _no_transforms(dev)
        has_tf, K = False, 1
    per_g = lambda t: t.reshape(*t.shape[:-2], n) if t.ndim >= 2 and t.shape[-1] == 1 \
        and t.shape[-2] == n else t  # noqa: E731 ((..., N, 1) -> (..., N))
    opacities = per_g(opacities)
    background = shared_background(background)
    # every operand's leading axes broadcast to one batch shape, folded into one flat batch
    # (the nested vmap of splax/_batching.py); the batch folds into one launch
    S = batch_shape(dict(means=(means3d, 2), scales=(scales, 2), quats=(quats, 2),
                         colors=(colors, 2), opacities=(opacities, 1), viewmat=(viewmat, 2),
                         background=(background, 1), gaussian_transforms=(gaussian_transforms, 3)))
    B = math.prod(S) if S else 1
    ops = [fold(t, w, S) for t, w in ((means3d, 2), (scales, 2), (quats, 2), (colors, 2),
                                      (opacities, 1), (viewmat, 2), (background, 1),
                                      (gaussian_transforms, 3))]
    H, W = img_shape
    check_key_fits(B, int(H), int(W))
    # antialiased: the blend uses opacities * opacity_compensation(conics, radii) and the tile
    # intersection the raw opacities (splax/_render.py:105-110); the library evaluates the
    # compensation and its gradient inside the record packing and the gradient gather.
    statics = (n, B, K, has_tf, (int(H), int(W)), tuple(map(float, f)), tuple(map(float, c)),
               float(glob_scale), float(clip_thresh), bool(antialiased), bool(render_depth))
    return ops, tf_ids.to(torch.int32), statics, S


def render(means3d: torch.Tensor, scales: torch.Tensor, quats: torch.Tensor,
           colors: torch.Tensor, opacities: torch.Tensor, *, viewmat: torch.Tensor,
           background: torch.Tensor, img_shape: tuple[int, int], f: tuple[float, float],
           c: tuple[float, float] | None = None, glob_scale: float = 1.0,
           clip_thresh: float = 0.01, antialiased: bool = False, render_depth: bool = False,
           gaussian_transforms: torch.Tensor | None = None,
           gaussian_slices: Sequence[tuple[int, int]] | None = None):
    """Render a splat; returns (image, depth-or-None) like splax.render (splax/_render.py:29-115)."""
    ops, tf_ids, statics, S = _prepare(means3d, scales, quats, colors, opacities, viewmat,
                                       background, img_shape, f, c, glob_scale, clip_thresh,
                                       antialiased, render_depth, gaussian_transforms,
                                       gaussian_slices)
    H, W = img_shape
    if torch.is_grad_enabled() and any(t.requires_grad for t in ops):
        img, depth = _RenderFn.apply(*ops[:7], ops[7], tf_ids, statics)
    else:  # no backward can follow: the forward alone, keeping no emission positions
        img, _, _, _, depth = _fused_forward(*ops, tf_ids, statics, backward=False)
    img = img.reshape(*S, H, W, 3)
    return img, (depth.reshape(*S, H, W) if render_depth else None)


_LOSS_KINDS = {"l1": _ops.LOSS_L1, "mse": _ops.LOSS_MSE}


def render_loss(means3d: torch.Tensor, scales: torch.Tensor, quats: torch.Tensor,
                colors: torch.Tensor, opacities: torch.Tensor, *, target: torch.Tensor,
                loss: str = "mse", viewmat: torch.Tensor, background: torch.Tensor,
                img_shape: tuple[int, int], f: tuple[float, float],
                c: tuple[float, float] | None = None, glob_scale: float = 1.0,
                clip_thresh: float = 0.01, antialiased: bool = False,
                gaussian_transforms: torch.Tensor | None = None,
                gaussian_slices: Sequence[tuple[int, int]] | None = None):
    """The mean of |img - target| (loss="l1") or (img - target)^2 ("mse") over render()'s image,
    with the loss fused into the blends. Returns (loss, image): the loss is differentiable like
    the loss of render()'s image (the same value up to the order of its double additions, the
    same gradients), the image carries no gradient. target has the image's shape and receives no
    gradient. The reference has no such call: its trainers apply the loss to render()'s image."""
    if loss not in _LOSS_KINDS:
        raise ValueError(f"loss must be one of {sorted(_LOSS_KINDS)}, got {loss!r}")
    ops, tf_ids, statics, S = _prepare(means3d, scales, quats, colors, opacities, viewmat,
                                       background, img_shape, f, c, glob_scale, clip_thresh,
                                       antialiased, False, gaussian_transforms, gaussian_slices)
    H, W = img_shape
    if tuple(target.shape) != (*S, H, W, 3) or target.dtype != torch.float32:
        raise ValueError(f"target must be float32 of the image's shape {(*S, H, W, 3)}, got "
                         f"{tuple(target.shape)} {target.dtype}")
    tgt = target.detach().reshape(-1, W, 3).contiguous()
    if torch.is_grad_enabled() and any(t.requires_grad for t in ops):
        value, img = _RenderLossFn.apply(*ops[:7], ops[7], tf_ids, tgt, statics,
                                         _LOSS_KINDS[loss])
    else:  # no backward can follow: the forward alone, keeping no emission positions
        value = torch.empty((), device=means3d.device, dtype=torch.float32)
        img = _fused_forward(*ops, tf_ids, statics, backward=False,
                             loss=(_LOSS_KINDS[loss], tgt, value))[0]
    return value, img.reshape(*S, H, W, 3)


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


def render_log_loss(means3d: torch.Tensor, log_scales: torch.Tensor, quats: torch.Tensor,
                    logit_colors: torch.Tensor, logit_opacities: torch.Tensor, *,
                    target: torch.Tensor, loss: str = "l1", viewmat: torch.Tensor,
                    background: torch.Tensor, img_shape: tuple[int, int],
                    f: tuple[float, float], c: tuple[float, float] | None = None,
                    glob_scale: float = 1.0, clip_thresh: float = 0.01,
                    antialiased: bool = False):
    """render_loss from log scales / logits (the parameter map of render_log)."""
    scales, quats, colors, opacities = _LogParamsFn.apply(log_scales, quats, logit_colors,
                                                          logit_opacities)
    return render_loss(means3d, scales, quats, colors, opacities, target=target, loss=loss,
                       viewmat=viewmat, background=background, img_shape=img_shape, f=f, c=c,
                       glob_scale=glob_scale, clip_thresh=clip_thresh, antialiased=antialiased)
