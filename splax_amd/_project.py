"""Differentiable projection stage (torch).

Mirrors splax/_project/_project.py: ``project`` (:25-92) is the public entry, ``_ProjectFn`` plays
the role of the ``jax.custom_vjp`` ``_project`` (:142-278) with one backward launch computing
every gradient; ``opacity_compensation`` (:95-117) and ``transform_ids`` (:120-136) are restated
as plain tensor code.

Batching. The reference folds ``jax.vmap`` over cameras into one launch (splax/_batching.py). Here
the same launch is reached by passing leading batch dimensions: ``viewmat`` of shape (..., 4, 4)
and/or gaussian parameters of shape (..., N, ...), any number of them, aligned from the right as in
broadcasting; they fold into one flat batch, outer axis major (``_batching``). Unbatched operands
are shared across the batch (read at the gaussian index), batched ones at the flat index;
gradients of shared operands are summed over the batch, as jax does for broadcast vmap inputs.
"""

from __future__ import annotations

from collections.abc import Sequence

import math

import torch

from splax_amd import _ops
from splax_amd._batching import batch_shape, fold


def _flat(t: torch.Tensor, width: int) -> torch.Tensor:
    return t.reshape(-1, width) if width > 1 else t.reshape(-1)


class _ProjectFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, means, scales, quats_wxyz, viewmat, opac, transforms, tf_ids, statics):
        n, B, K, has_tf, img_shape, f, c, glob_scale, clip_thresh = statics
        xys, depths, radii, conics, nth, cum = _ops.project_fwd(
            _flat(means, 3), _flat(scales, 3), _flat(quats_wxyz, 4), viewmat.reshape(-1, 4),
            opac.reshape(-1), transforms.reshape(-1, 4, 4), tf_ids.reshape(-1), n=n, total=B * n,
            num_transforms=K, has_transforms=has_tf, img_shape=img_shape, f=f, c=c,
            glob_scale=glob_scale, clip_thresh=clip_thresh, quats_wxyz=True)
        ctx.save_for_backward(means, scales, quats_wxyz, viewmat, transforms, tf_ids, radii,
                              conics)
        ctx.statics = statics
        ctx.mark_non_differentiable(radii, nth, cum)
        ctx.set_materialize_grads(False)  # unused outputs arrive as None, not zero tensors
        return xys, depths, radii, conics, nth, cum

    @staticmethod
    def backward(ctx, v_xys, v_depths, _v_radii, v_conics, _v_nth, _v_cum):
        means, scales, quats, viewmat, transforms, tf_ids, radii, conics = ctx.saved_tensors
        n, B, K, has_tf, img_shape, f, c, glob_scale, clip_thresh = ctx.statics
        z = torch.zeros_like
        v_xys = z(radii, dtype=torch.float32).unsqueeze(-1).expand(-1, 2) if v_xys is None \
            else v_xys
        v_conics = z(radii, dtype=torch.float32).unsqueeze(-1).expand(-1, 3) if v_conics is None \
            else v_conics
        # shared gaussian parameters: the library sums their per-image rows itself
        fold_here = B > 1 and all(t.numel() == n * w for t, w in ((means, 3), (scales, 3),
                                                                   (quats, 4)))
        v_mean, v_scale, v_quat, v_view, v_tf = _ops.project_bwd(
            _flat(means, 3), _flat(scales, 3), _flat(quats, 4), viewmat.reshape(-1, 4), radii,
            conics, v_xys.reshape(-1, 2), None if v_depths is None else v_depths.reshape(-1),
            v_conics.reshape(-1, 3),
            transforms.reshape(-1, 4, 4), tf_ids.reshape(-1), n=n, B=B, num_transforms=K,
            has_transforms=has_tf, f=f, glob_scale=glob_scale, quats_wxyz=True, fold=fold_here,
            want_viewmat=ctx.needs_input_grad[3])

        def fold(g: torch.Tensor, like: torch.Tensor, width: int) -> torch.Tensor:
            if g.numel() == like.numel():  # one image, or a batched operand
                return g.reshape(like.shape)
            g = g.reshape(B, n, width) if width > 1 else g.reshape(B, n)
            return g.sum(0).reshape(like.shape)  # shared operand: sum over the batch

        g_means = fold(v_mean, means, 3) if ctx.needs_input_grad[0] else None
        g_scales = fold(v_scale, scales, 3) if ctx.needs_input_grad[1] else None
        g_quats = fold(v_quat, quats, 4) if ctx.needs_input_grad[2] else None
        g_view = None
        if ctx.needs_input_grad[3]:
            g_view = v_view.reshape(B, 4, 4)
            g_view = g_view.reshape(viewmat.shape) if viewmat.ndim == 3 else g_view.sum(0)
        g_tf = None
        if has_tf and ctx.needs_input_grad[5]:
            g_tf = v_tf.reshape(B, K, 4, 4)
            g_tf = g_tf.reshape(transforms.shape) if transforms.ndim == 4 else g_tf.sum(0)
        return g_means, g_scales, g_quats, g_view, None, g_tf, None, None


_NO_TF: dict = {}


def _no_transforms(dev: torch.device):
    """The reference's dummy (1, 4, 4) transforms and (1,) ids of -1 (splax/_project/_project.py:71-73),
    made once per device."""
    key = str(dev)
    if key not in _NO_TF:
        _NO_TF[key] = (torch.zeros((1, 4, 4), device=dev, dtype=torch.float32),
                       torch.full((1,), -1, device=dev, dtype=torch.int32))
    return _NO_TF[key]


def project(mean3ds: torch.Tensor, scales: torch.Tensor, quats: torch.Tensor,
            viewmat: torch.Tensor, *, opacities: torch.Tensor, img_shape: tuple[int, int],
            f: tuple[float, float], c: tuple[float, float] | None = None,
            glob_scale: float = 1.0, clip_thresh: float = 0.01,
            gaussian_transforms: torch.Tensor | None = None,
            transform_ids: torch.Tensor | None = None):
    """Project gaussians to screen space with the opacity-aware tile intersection.

    Same arguments and outputs as splax.project (splax/_project/_project.py:25-92): quats are wxyz,
    outputs are xys (N, 2), depths (N, 1), radii (N, 1) int32, conics (N, 3), num_tiles_hit (N, 1)
    and the inclusive prefix sum cum_tiles_hit (N, 1) (int32; the reference returns uint32, which
    torch does not support as a general dtype). With leading batch dimensions on viewmat and/or
    the gaussian parameters (any number, broadcast against each other: the nested vmap of
    splax/_batching.py), every output gains the broadcast batch shape, and cum_tiles_hit is
    global over the flattened batch. Gradients flow to means, scales, quats, viewmat and
    gaussian_transforms.
    """
    n = int(mean3ds.shape[-2])
    if c is None:
        c = (img_shape[1] / 2, img_shape[0] / 2)
    has_tf = gaussian_transforms is not None
    if has_tf != (transform_ids is not None):
        raise ValueError("gaussian_transforms and transform_ids must be passed together")
    dev = mean3ds.device
    if not has_tf:
        gaussian_transforms, transform_ids = _no_transforms(dev)
        K = 1
    else:
        K = int(gaussian_transforms.shape[-3])
    opacities = opacities.reshape(*opacities.shape[:-2], n) if opacities.shape[-1] == 1 \
        and opacities.ndim >= 2 else opacities
    S = batch_shape(dict(means=(mean3ds, 2), scales=(scales, 2), quats=(quats, 2),
                         viewmat=(viewmat, 2), opacities=(opacities, 1),
                         gaussian_transforms=(gaussian_transforms, 3)))
    mean3ds, scales, quats = fold(mean3ds, 2, S), fold(scales, 2, S), fold(quats, 2, S)
    viewmat, opacities = fold(viewmat, 2, S), fold(opacities, 1, S)
    gaussian_transforms = fold(gaussian_transforms, 3, S)
    batched = len(S) > 0
    Bv = math.prod(S) if batched else 1
    # The reference rolls wxyz to its kernel's xyzw here (splax/_project/_project.py:74-76);
    # the library reads wxyz directly and returns the quaternion gradient in wxyz.
    statics = (n, Bv, K, has_tf, tuple(img_shape), tuple(map(float, f)), tuple(map(float, c)),
               float(glob_scale), float(clip_thresh))
    xys, depths, radii, conics, nth, cum = _ProjectFn.apply(
        mean3ds, scales, quats, viewmat, opacities, gaussian_transforms,
        transform_ids.to(torch.int32), statics)
    lead = (*S, n)
    return (xys.reshape(*lead, 2), depths.reshape(*lead, 1), radii.reshape(*lead, 1),
            conics.reshape(*lead, 3), nth.reshape(*lead, 1), cum.reshape(*lead, 1))


class _CompensationFn(torch.autograd.Function):
    """rho = sqrt(clip(rho2, 0, 1)) of the conics with the reverse-mode rules of the reference's
    jax expression (splax/_project/_project.py:113-116), not torch's: sqrt' = 0.5 / rho times the
    cotangent (so rho = 0 gives NaN or inf even for a zero cotangent), and each clip bound passes
    1 strictly inside, 1/2 at a tie and 0 outside, as multipliers (inf times 0 is NaN). The fused
    antialiased blend (grad_gather_kernel) and the oracle apply the same rules."""

    @staticmethod
    def forward(ctx, conics, eps):
        a, b, c = conics[..., 0], conics[..., 1], conics[..., 2]
        rho2 = 1.0 - eps * (a + c) + (eps * eps) * (a * c - b * b)
        rho = torch.sqrt(torch.clamp(rho2, 0.0, 1.0))
        ctx.save_for_backward(conics, rho2, rho)
        ctx.eps = eps
        return rho

    @staticmethod
    def backward(ctx, g):
        conics, rho2, rho = ctx.saved_tensors
        eps = ctx.eps
        a, b, c = conics[..., 0], conics[..., 1], conics[..., 2]
        one, half, zero = (torch.full_like(rho2, v) for v in (1.0, 0.5, 0.0))
        v_cl = g * (0.5 / rho)
        m_lo = torch.where(rho2 > 0, one, torch.where(rho2 == 0, half, zero))
        y = torch.where(rho2 > 0, rho2, zero)
        m_hi = torch.where(y < 1, one, torch.where(y == 1, half, zero))
        v_r2 = (v_cl * m_hi) * m_lo
        v_s, v_t = -(eps * v_r2), (eps * eps) * v_r2
        v_conics = torch.stack([v_s + v_t * c, -(v_t * b) - v_t * b, v_s + v_t * a], dim=-1)
        return v_conics, None


def opacity_compensation(conics: torch.Tensor, radii: torch.Tensor,
                         eps: float = 0.3) -> torch.Tensor:
    """Mip-Splatting opacity compensation rho per gaussian (splax/_project/_project.py:95-117),
    differentiated by the reference's rules (a visible item whose rho2 <= 0 gets NaN conic
    cotangents, as jax's sqrt and clip rules give there)."""
    lead = conics.shape[:-1]
    rho = _CompensationFn.apply(conics, eps)
    return torch.where(radii.reshape(lead) > 0, rho, torch.ones_like(rho))


def transform_ids(n: int, slices: Sequence[tuple[int, int]],
                  device: torch.device | str | None = None) -> torch.Tensor:
    """Map each gaussian to the transform it follows (splax/_project/_project.py:120-136)."""
    for k, (start, stop) in enumerate(slices):
        if not (0 <= start < stop <= n):
            raise ValueError(f"gaussian slice {k} = [{start}, {stop}) outside [0, {n})")
    ordered = sorted(slices)
    for (_, prev_stop), (start, _) in zip(ordered, ordered[1:]):
        if start < prev_stop:
            raise ValueError(f"gaussian slices overlap: {list(slices)}")
    ids = torch.full((n,), -1, dtype=torch.int32, device=device)
    for k, (start, stop) in enumerate(slices):
        ids[start:stop] = k
    return ids
