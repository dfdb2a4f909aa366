"""Tensor-level calls into the C ABI (no autograd).

Each function takes flattened operands in the reference's FFI convention (leading dimension =
rows; an operand is batched when its rows exceed ``n``), allocates the outputs with torch on the
operands' device and enqueues the library call on torch's current stream of that device.
"""

from __future__ import annotations

import ctypes
from typing import NamedTuple, Optional

import torch

from splax_amd import _lib


def _f32(t: torch.Tensor) -> torch.Tensor:
    if t.dtype != torch.float32:
        raise ValueError(f"expected float32, got {t.dtype}")
    return t.contiguous()


def _i32(t: torch.Tensor) -> torch.Tensor:
    if t.dtype != torch.int32:
        t = t.to(torch.int32)
    return t.contiguous()


def rows(t: torch.Tensor, width: int) -> int:
    return t.numel() // width


def project_fwd(means, scales, quats, viewmat, opac, transforms, transform_ids, *, n,
                total, num_transforms, has_transforms, img_shape, f, c, glob_scale, clip_thresh,
                quats_wxyz=False):
    """_project_warp (splax/_project/_kernels.py:31-107) over ``total`` flat items; quats are
    xyzw as the reference's kernel takes them, or wxyz with ``quats_wxyz``."""
    means, scales, quats, viewmat, opac = map(_f32, (means, scales, quats, viewmat, opac))
    transforms = _f32(transforms)
    transform_ids = _i32(transform_ids)
    dev = _lib.require_gpu(means, scales, quats, viewmat, opac, transforms, transform_ids)
    H, W = img_shape
    xys = torch.empty((total, 2), device=dev, dtype=torch.float32)
    depths = torch.empty((total,), device=dev, dtype=torch.float32)
    radii = torch.empty((total,), device=dev, dtype=torch.int32)
    conics = torch.empty((total, 3), device=dev, dtype=torch.float32)
    nth = torch.empty((total,), device=dev, dtype=torch.int32)
    cum = torch.empty((total,), device=dev, dtype=torch.int32)
    if total == 0:
        return xys, depths, radii, conics, nth, cum
    p = _lib.ptr
    with torch.cuda.device(dev):
        st = _lib.lib().splat_project_fwd(
            _lib.stream_handle(dev), p(means), rows(means, 3), p(scales), rows(scales, 3),
            p(quats), rows(quats, 4), p(viewmat), rows(viewmat, 4), p(opac), opac.numel(),
            p(transforms), rows(transforms, 16), p(transform_ids), n, num_transforms,
            int(has_transforms), total, H, W, f[0], f[1], c[0], c[1], glob_scale, clip_thresh,
            p(xys), p(depths), p(radii), p(conics), p(nth), p(cum), int(quats_wxyz))
    _lib.check(st, "project")
    return xys, depths, radii, conics, nth, cum


def project_bwd(means, scales, quats, viewmat, radii, conics, v_xy, v_depth, v_conic,
                transforms, transform_ids, *, n, B, num_transforms, has_transforms, f,
                glob_scale, quats_wxyz=False, fold=False, want_viewmat=True):
    """_project_bwd_warp (splax/_project/_kernels.py:257-341).

    v_depth may be None (a zero depth cotangent); v_tf is None without transforms. v_quat comes
    in the layout of quats (xyzw, or wxyz with ``quats_wxyz``). With ``fold`` (shared means,
    scales and quats) v_mean, v_scale and v_quat have n rows, summed over the B images. Without
    ``want_viewmat`` no viewmat gradient is formed and v_view is None."""
    means, scales, quats, viewmat, conics = map(_f32, (means, scales, quats, viewmat,
                                                       conics))
    v_xy, v_conic, transforms = map(_f32, (v_xy, v_conic, transforms))
    v_depth = None if v_depth is None else _f32(v_depth)
    radii, transform_ids = _i32(radii), _i32(transform_ids)
    dev = _lib.require_gpu(means, scales, quats, viewmat, conics, v_xy, v_conic)
    total = n if fold else B * n
    v_mean = torch.empty((total, 3), device=dev, dtype=torch.float32)
    v_scale = torch.empty((total, 3), device=dev, dtype=torch.float32)
    v_quat = torch.empty((total, 4), device=dev, dtype=torch.float32)
    v_view = torch.empty((B * 4, 4), device=dev, dtype=torch.float32) if want_viewmat else None
    v_tf = None
    if has_transforms:
        v_tf = torch.empty((B * num_transforms, 4, 4), device=dev, dtype=torch.float32)
    p = _lib.ptr
    with torch.cuda.device(dev):
        st = _lib.lib().splat_project_bwd(
            _lib.stream_handle(dev), p(means), rows(means, 3), p(scales), rows(scales, 3),
            p(quats), rows(quats, 4), p(viewmat), rows(viewmat, 4), p(radii), radii.numel(),
            p(conics), rows(conics, 3), p(v_xy), rows(v_xy, 2), p(v_depth),
            0 if v_depth is None else v_depth.numel(), p(v_conic), rows(v_conic, 3),
            p(transforms), rows(transforms, 16), p(transform_ids), n, num_transforms,
            int(has_transforms), B, f[0], f[1], glob_scale, p(v_mean), p(v_scale), p(v_quat),
            p(v_view), p(v_tf), int(quats_wxyz), int(fold))
    _lib.check(st, "project_bwd")
    return v_mean, v_scale, v_quat, v_view, v_tf


def rasterize_fwd(colors, opac, map_opac, background, xys, depths, radii, conics, cum, *, n, B,
                  img_shape, render_depth=False):
    """_rasterize_warp (splax/_rasterize/_kernels.py:37-87): sort_and_bin + forward blend; with
    render_depth, _rasterize_depth_warp (:208-262), whose expected depth (B*H, W) comes last."""
    colors, opac, map_opac, background, xys, depths, conics = map(
        _f32, (colors, opac, map_opac, background, xys, depths, conics))
    radii, cum = _i32(radii), _i32(cum)
    dev = _lib.require_gpu(colors, opac, map_opac, background, xys, depths, radii, conics, cum)
    H, W = img_shape
    Ts = torch.empty((B * H, W), device=dev, dtype=torch.float32)
    fidx = torch.empty((B * H, W), device=dev, dtype=torch.int32)
    img = torch.empty((B * H, W, 3), device=dev, dtype=torch.float32)
    depth = torch.empty((B * H, W), device=dev, dtype=torch.float32) if render_depth else None
    m = ctypes.c_int64(0)
    p = _lib.ptr
    args = (_lib.stream_handle(dev), p(colors), rows(colors, 3), p(opac), opac.numel(),
            p(map_opac), map_opac.numel(), p(background), rows(background, 3), p(xys), p(depths),
            p(radii), p(conics), p(cum), n, B, H, W, p(Ts), p(fidx), p(img))
    with torch.cuda.device(dev):
        if render_depth:
            st = _lib.lib().splat_rasterize_depth_fwd(*args, p(depth), ctypes.byref(m))
        else:
            st = _lib.lib().splat_rasterize_fwd(*args, ctypes.byref(m))
    _lib.check(st, "rasterize")
    if render_depth:
        return img, Ts, fidx, int(m.value), depth
    return img, Ts, fidx, int(m.value)


# Per device: the capacity estimate for the kept sorted lists (1.25x the largest count seen) and
# the workload signature (B, n, tiles per image) it was seen on. A call with another signature
# starts again from no estimate, as the library drops its own scratch then (the reference drops
# its scratch entry on a signature change, splax/_cache.py:61-75); clear_cache() forgets both.
_KEEP_CAPACITY: dict = {}
_KEEP_SIG: dict = {}


def _keep_capacity(key: str, sig: tuple) -> int:
    if _KEEP_SIG.get(key) != sig:
        _KEEP_SIG[key] = sig
        _KEEP_CAPACITY[key] = 0
    return _KEEP_CAPACITY.get(key, 0)


def clear_cache() -> None:
    """Release the library's persistent per-device scratch and forget the kept-list capacity
    estimates (splax/_cache.py:158-164)."""
    _KEEP_CAPACITY.clear()
    _KEEP_SIG.clear()
    _lib.clear_cache()


class KeptSort(NamedTuple):
    """What rasterize_fwd_keep leaves for rasterize_bwd_sorted: the sorted gaussian ids, their
    emission positions, the tile bins, the intersection count, the packed blend records
    ([B*n, 16], or None to have the backward pack them again) and the blend's tile order
    ([B*num_tiles], or None to have the backward order the tiles again)."""
    ids: torch.Tensor
    pos: torch.Tensor
    bins: torch.Tensor
    M: int
    records: Optional[torch.Tensor]
    order: Optional[torch.Tensor] = None


def rasterize_fwd_keep(colors, opac, map_opac, background, xys, depths, radii, conics, cum, *, n,
                       B, img_shape, render_depth=False, compensate=False):
    """Forward that also keeps the sorted lists and packed records for the backward; returns
    (img, Ts, fidx, KeptSort, depth or None).

    The buffers are sized from a per-device estimate (1.25x the largest count seen), so the host
    does not wait for the intersection count before launching: the library reads it itself while
    its first kernels run, and reports status 6 with the count when the buffers are too small, in
    which case they are reallocated and the call repeated.
    """
    colors, opac, map_opac, background, xys, depths, conics = map(
        _f32, (colors, opac, map_opac, background, xys, depths, conics))
    radii, cum = _i32(radii), _i32(cum)
    dev = _lib.require_gpu(colors, opac, map_opac, background, xys, depths, radii, conics, cum)
    H, W = img_shape
    tiles = ((W + 15) // 16) * ((H + 15) // 16)
    Ts = torch.empty((B * H, W), device=dev, dtype=torch.float32)
    fidx = torch.empty((B * H, W), device=dev, dtype=torch.int32)
    img = torch.empty((B * H, W, 3), device=dev, dtype=torch.float32)
    depth = torch.empty((B * H, W), device=dev, dtype=torch.float32) if render_depth else None
    bins = torch.empty((B * tiles, 2), device=dev, dtype=torch.int32)
    recs = torch.empty((xys.shape[0], 16), device=dev, dtype=torch.float32)
    order = torch.empty((B * tiles,), device=dev, dtype=torch.int32)
    key = str(dev)
    cap = _keep_capacity(key, (B, n, tiles))
    m = ctypes.c_int64(0)
    p = _lib.ptr
    for _ in range(2):
        ids = torch.empty((max(cap, 1),), device=dev, dtype=torch.int32)
        pos = torch.empty((max(cap, 1),), device=dev, dtype=torch.int32)
        with torch.cuda.device(dev):
            st = _lib.lib().splat_rasterize_fwd_keep(
                _lib.stream_handle(dev), p(colors), rows(colors, 3), p(opac), opac.numel(),
                p(map_opac), map_opac.numel(), p(background), rows(background, 3), p(xys),
                p(depths), p(radii), p(conics), p(cum), n, B, H, W, cap, p(Ts), p(fidx), p(img),
                p(depth), p(ids), p(pos), p(bins), p(recs), p(order), ctypes.byref(m),
                int(compensate))
        if st == _lib.ERR_TOO_MANY and m.value > cap:
            cap = int(m.value * 1.25) + 1
            _KEEP_CAPACITY[key] = cap
            continue
        break
    _lib.check(st, "rasterize")
    M = int(m.value)
    if M > _KEEP_CAPACITY.get(key, 0):
        _KEEP_CAPACITY[key] = int(M * 1.25) + 1
    return img, Ts, fidx, KeptSort(ids, pos, bins, M, recs, order), depth


class RenderKept(NamedTuple):
    """What splat_render_fwd keeps for splat_render_bwd: the projection outputs and the
    rasterizer's kept lists."""
    xys: torch.Tensor
    depths: torch.Tensor
    radii: torch.Tensor
    conics: torch.Tensor
    cum: torch.Tensor
    sort: KeptSort


def render_fwd(means, scales, quats_wxyz, colors, opac, viewmat, background, transforms,
               transform_ids, *, n, B, num_transforms, has_transforms, img_shape, f, c,
               glob_scale, clip_thresh, compensate=False, render_depth=False, backward=True,
               loss_kind=0, loss_target=None, loss_out=None):
    """The fused render forward (splat_render_fwd): projection, sort and blend in one call over
    B images of n gaussians; quaternions wxyz. Returns (img, Ts, fidx, RenderKept, depth or None).
    Kept-list capacity as rasterize_fwd_keep. backward=False (no render_bwd will follow) sorts no
    emission positions and writes no final_Ts / final_idx: Ts, fidx and the kept lists' pos are
    then None. loss_kind LOSS_L1 / LOSS_MSE fuses the mean pixel loss against loss_target
    ([B * H, W, 3] values) into the blend, its value written into loss_out (a float32 scalar)."""
    means, scales, quats_wxyz, colors, opac, viewmat, background, transforms = map(
        _f32, (means, scales, quats_wxyz, colors, opac, viewmat, background, transforms))
    transform_ids = _i32(transform_ids)
    dev = _lib.require_gpu(means, scales, quats_wxyz, colors, opac, viewmat, background)
    H, W = img_shape
    total = B * n
    if loss_kind:
        _check_loss_operands(loss_kind, loss_target, B, H, W, dev, loss_out)
        loss_target = _f32(loss_target)
    tiles = ((W + 15) // 16) * ((H + 15) // 16)
    e = lambda *shape, dt=torch.float32: torch.empty(shape, device=dev, dtype=dt)  # noqa: E731
    xys, depths, conics = e(total, 2), e(total), e(total, 3)
    radii, nth, cum = e(total, dt=torch.int32), e(total, dt=torch.int32), e(total, dt=torch.int32)
    img = e(B * H, W, 3)
    Ts, fidx = (e(B * H, W), e(B * H, W, dt=torch.int32)) if backward else (None, None)
    depth = e(B * H, W) if render_depth else None
    bins, recs, order = e(B * tiles, 2, dt=torch.int32), e(total, 16), e(B * tiles, dt=torch.int32)
    key = str(dev)
    cap = _keep_capacity(key, (B, n, tiles))
    m = ctypes.c_int64(0)
    p = _lib.ptr
    for _ in range(2):
        ids = e(max(cap, 1), dt=torch.int32)
        pos = e(max(cap, 1), dt=torch.int32) if backward else None
        with torch.cuda.device(dev):
            st = _lib.lib().splat_render_fwd(
                _lib.stream_handle(dev), p(means), rows(means, 3), p(scales), rows(scales, 3),
                p(quats_wxyz), rows(quats_wxyz, 4), p(viewmat), rows(viewmat, 4), p(opac),
                opac.numel(), p(colors), rows(colors, 3), p(background), rows(background, 3),
                p(transforms), rows(transforms, 16), p(transform_ids), n, num_transforms,
                int(has_transforms), B, H, W, f[0], f[1], c[0], c[1], glob_scale, clip_thresh, 1,
                int(compensate), p(xys), p(depths), p(radii), p(conics), p(nth), p(cum), cap,
                p(ids), p(pos), p(bins), p(recs), p(order), p(Ts), p(fidx), p(img), p(depth),
                ctypes.byref(m), p(loss_target) if loss_kind else None, int(loss_kind),
                p(loss_out) if loss_kind else None)
        if st == _lib.ERR_TOO_MANY and m.value > cap:
            cap = int(m.value * 1.25) + 1
            _KEEP_CAPACITY[key] = cap
            continue
        break
    _lib.check(st, "render")
    M = int(m.value)
    if M > _KEEP_CAPACITY.get(key, 0):
        _KEEP_CAPACITY[key] = int(M * 1.25) + 1
    kept = RenderKept(xys, depths, radii, conics, cum, KeptSort(ids, pos, bins, M, recs, order))
    return img, Ts, fidx, kept, depth


def render_bwd(means, scales, quats_wxyz, colors, opac, viewmat, background, transforms,
               transform_ids, kept: RenderKept, final_Ts, final_idx, v_out, *, n, B,
               num_transforms, has_transforms, img_shape, f, glob_scale, compensate=False,
               v_out_depth=None, fold=False, want_viewmat=True, loss_kind=0, loss_target=None,
               out_img=None, v_loss=None):
    """The fused render backward (splat_render_bwd). Returns (v_means, v_scales, v_quats (wxyz),
    v_colors, v_opac, v_viewmat or None, v_transforms or None), n rows each with ``fold`` (every
    gaussian operand shared), else B * n. With loss_kind (the forward's fused loss) the image
    cotangent comes from out_img (the forward's image), loss_target and the loss cotangent v_loss
    (a float32 scalar); v_out is then unused (may be None)."""
    means, scales, quats_wxyz, colors, opac, viewmat, background, transforms = map(
        _f32, (means, scales, quats_wxyz, colors, opac, viewmat, background, transforms))
    H, W = img_shape
    if loss_kind:
        _check_loss_operands(loss_kind, loss_target, B, H, W, means.device, v_loss)
        if out_img is None or out_img.shape != loss_target.shape:
            raise ValueError("render_bwd: a fused loss needs the forward's image, of the "
                             "target's shape")
        loss_target, out_img, v_loss = _f32(loss_target), _f32(out_img), _f32(v_loss.reshape(()))
        v_out = None
    else:
        v_out = _f32(v_out)
    vd = None if v_out_depth is None else _f32(v_out_depth)
    dev = _lib.require_gpu(means, *(t for t in (v_out, loss_target) if t is not None))
    rows_out = n if fold else B * n
    e = lambda *shape: torch.empty(shape, device=dev, dtype=torch.float32)  # noqa: E731
    v_means, v_scales, v_quats = e(rows_out, 3), e(rows_out, 3), e(rows_out, 4)
    v_colors, v_opac = e(rows_out, 3), e(rows_out)
    v_view = e(B * 4, 4) if want_viewmat else None
    v_tf = e(B * num_transforms, 4, 4) if has_transforms else None
    ks = kept.sort
    p = _lib.ptr
    with torch.cuda.device(dev):
        st = _lib.lib().splat_render_bwd(
            _lib.stream_handle(dev), p(means), rows(means, 3), p(scales), rows(scales, 3),
            p(quats_wxyz), rows(quats_wxyz, 4), p(viewmat), rows(viewmat, 4), p(opac),
            opac.numel(), p(colors), rows(colors, 3), p(background), rows(background, 3),
            p(transforms), rows(transforms, 16), p(_i32(transform_ids)), n, num_transforms,
            int(has_transforms), B, H, W, f[0], f[1], glob_scale, 1, int(compensate),
            p(kept.xys), p(kept.depths), p(kept.radii), p(kept.conics), p(kept.cum), p(ks.ids),
            p(ks.pos), p(ks.bins), p(ks.records), p(ks.order), ks.M, p(final_Ts), p(final_idx),
            p(v_out), 0 if v_out is None else v_out.numel() // (3 * W), p(vd),
            0 if vd is None else vd.numel() // W, p(v_means), p(v_scales), p(v_quats),
            p(v_colors), p(v_opac), p(v_view), p(v_tf), int(fold),
            p(loss_target) if loss_kind else None, int(loss_kind),
            p(out_img) if loss_kind else None, p(v_loss) if loss_kind else None)
    _lib.check(st, "render_bwd")
    return v_means, v_scales, v_quats, v_colors, v_opac, v_view, v_tf


LOSS_L1, LOSS_MSE = 1, 2  # loss_kind of the fused render loss


def _check_loss_operands(kind, target, B, H, W, dev, scalar):
    if kind not in (LOSS_L1, LOSS_MSE):
        raise ValueError(f"loss_kind must be {LOSS_L1} (L1) or {LOSS_MSE} (MSE), got {kind}")
    if target is None or target.numel() != B * H * W * 3 or target.device != dev or \
            target.dtype != torch.float32:
        raise ValueError(f"the loss target must hold {B} x {H} x {W} x 3 float32 values on {dev}")
    if scalar is None or scalar.numel() != 1 or scalar.dtype != torch.float32 or \
            scalar.device != dev:
        raise ValueError(f"the loss value / cotangent must be one float32 on {dev}")


def _bwd_outputs(nout, dev, with_depth):
    f = lambda *shape: torch.empty(shape, device=dev, dtype=torch.float32)  # noqa: E731
    return f(nout, 3), f(nout), f(nout, 2), f(nout, 3), (f(nout) if with_depth else None)


def rasterize_bwd_sorted(colors, opac, background, xys, depths, conics, cum, kept: KeptSort,
                         final_Ts, final_idx, v_out, *, n, B_out, B_geom, img_shape,
                         v_out_depth=None, compensate=False, fold=False):
    """Backward over the sorted lists (and records) of rasterize_fwd_keep for the same inputs
    (no re-sort); with v_out_depth also the depth channel's v_depths (last)."""
    colors, opac, background, xys, depths, conics, final_Ts, v_out = map(
        _f32, (colors, opac, background, xys, depths, conics, final_Ts, v_out))
    ids, pos, bins, M = _i32(kept.ids), _i32(kept.pos), _i32(kept.bins), kept.M
    recs = None if kept.records is None else _f32(kept.records)
    if recs is not None and recs.shape != (xys.shape[0], 16):
        raise ValueError(f"records must be [{xys.shape[0]}, 16], got {tuple(recs.shape)}")
    order = None if kept.order is None else _i32(kept.order)
    if order is not None and order.numel() != bins.shape[0]:
        raise ValueError(f"tile order must have {bins.shape[0]} entries, got {order.numel()}")
    cum, final_idx = _i32(cum), _i32(final_idx)
    vd = None if v_out_depth is None else _f32(v_out_depth)
    dev = _lib.require_gpu(colors, opac, xys, conics, cum, ids, pos, bins, final_Ts, final_idx,
                           v_out)
    H, W = img_shape
    v_colors, v_opac, v_xy, v_conic, v_depths = _bwd_outputs(B_out * n, dev, vd is not None)
    if fold:  # shared colours and opacities: the library sums their per-image rows
        v_colors, v_opac = v_colors[:n], v_opac[:n]
    p = _lib.ptr
    with torch.cuda.device(dev):
        st = _lib.lib().splat_rasterize_bwd_sorted(
            _lib.stream_handle(dev), p(colors), rows(colors, 3), p(opac), opac.numel(),
            p(background), rows(background, 3), p(xys), p(depths), p(conics), p(cum), p(ids),
            p(pos), p(bins), p(recs), p(order), M, p(final_Ts), p(final_idx), p(v_out),
            v_out.numel() // (3 * W),
            p(vd), 0 if vd is None else vd.numel() // W, n, B_out, B_geom, H, W, p(v_colors),
            p(v_opac), p(v_xy), p(v_conic), p(v_depths), int(compensate), int(fold))
    _lib.check(st, "rasterize_bwd")
    if vd is None:
        return v_colors, v_opac, v_xy, v_conic
    return v_colors, v_opac, v_xy, v_conic, v_depths


def rasterize_bwd(colors, opac, map_opac, background, xys, depths, radii, conics, cum, final_Ts,
                  final_idx, v_out, *, n, B_out, B_geom, img_shape, v_out_depth=None):
    """_rasterize_bwd_warp (splax/_rasterize/_kernels.py:386-500); with v_out_depth,
    _rasterize_bwd_depth_warp (:797-914), whose v_depths comes last."""
    colors, opac, map_opac, background, xys, depths, conics, final_Ts, v_out = map(
        _f32, (colors, opac, map_opac, background, xys, depths, conics, final_Ts, v_out))
    radii, cum, final_idx = _i32(radii), _i32(cum), _i32(final_idx)
    vd = None if v_out_depth is None else _f32(v_out_depth)
    dev = _lib.require_gpu(colors, opac, xys, conics, final_Ts, final_idx, v_out)
    H, W = img_shape
    v_colors, v_opac, v_xy, v_conic, v_depths = _bwd_outputs(B_out * n, dev, vd is not None)
    p = _lib.ptr
    args = (_lib.stream_handle(dev), p(colors), rows(colors, 3), p(opac), opac.numel(),
            p(map_opac), map_opac.numel(), p(background), rows(background, 3), p(xys), p(depths),
            p(radii), p(conics), p(cum), p(final_Ts), p(final_idx), p(v_out),
            v_out.numel() // (3 * W))
    with torch.cuda.device(dev):
        if vd is None:
            st = _lib.lib().splat_rasterize_bwd(*args, n, B_out, B_geom, H, W, p(v_colors),
                                                p(v_opac), p(v_xy), p(v_conic))
        else:
            st = _lib.lib().splat_rasterize_depth_bwd(*args, p(vd), vd.numel() // W, n, B_out,
                                                      B_geom, H, W, p(v_colors), p(v_opac),
                                                      p(v_xy), p(v_conic), p(v_depths))
    _lib.check(st, "rasterize_bwd")
    if vd is None:
        return v_colors, v_opac, v_xy, v_conic
    return v_colors, v_opac, v_xy, v_conic, v_depths


def sort_and_bin(xys, depths, radii, conics, map_opac, cum, *, n, B, img_shape, capacity=None):
    """splax/_rasterize/_sort/_sort.py:29-171: sorted keys (int64; packed keys widened), sorted
    gaussian ids, tile bins."""
    xys, depths, conics, map_opac = map(_f32, (xys, depths, conics, map_opac))
    radii, cum = _i32(radii), _i32(cum)
    dev = _lib.require_gpu(xys, depths, radii, conics, map_opac, cum)
    H, W = img_shape
    tiles = ((W + 15) // 16) * ((H + 15) // 16)
    if capacity is None:
        capacity = int(cum.reshape(-1)[-1].item()) if cum.numel() else 0
    keys = torch.empty((max(capacity, 1),), device=dev, dtype=torch.int64)
    ids = torch.empty((max(capacity, 1),), device=dev, dtype=torch.int32)
    bins = torch.empty((B * tiles, 2), device=dev, dtype=torch.int32)
    m = torch.zeros(1, dtype=torch.int64)
    p = _lib.ptr
    with torch.cuda.device(dev):
        st = _lib.lib().splat_sort_and_bin(
            _lib.stream_handle(dev), p(xys), p(depths), p(radii), p(conics), p(map_opac),
            map_opac.numel(), p(cum), n, B, H, W, p(keys), p(ids), capacity, p(bins),
            m.data_ptr())
    _lib.check(st, "sort_and_bin")
    M = int(m.item())
    return keys[:M], ids[:M], bins
