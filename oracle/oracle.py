"""numpy front end of the CPU oracle (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import this
module, as the checker of the GPU library or as the timed CPU baseline. The product package
(``splax_amd``) never imports it.

Each wrapper mirrors one reference entry point of amacati/splax:
- ``project_fwd``: ``_project_warp`` + ``_project_kernel``, splax/_project/_kernels.py:31-248
- ``sort_and_bin``: splax/_rasterize/_sort/_sort.py:29-171
- ``rasterize_fwd``: ``_rasterize_warp`` + ``_rasterize_kernel``, splax/_rasterize/_kernels.py:37-205
- ``rasterize_bwd``: ``_rasterize_bwd_warp``, splax/_rasterize/_kernels.py:386-665,1212-1254
- ``project_bwd``: ``_project_bwd_warp``, splax/_project/_kernels.py:257-664
Arrays follow the reference's flattened batch convention (rows > n means batched).
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int32)
_i64p = ctypes.POINTER(ctypes.c_int64)
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_f32 = ctypes.c_float


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            from oracle.build import build

            build()
        _lib = ctypes.CDLL(str(LIB_PATH))
        _lib.oracle_logf.restype = ctypes.c_float
        _lib.oracle_logf.argtypes = [ctypes.c_float]
        _lib.oracle_expf.restype = ctypes.c_float
        _lib.oracle_expf.argtypes = [ctypes.c_float]
        for name in ("oracle_emit_keys", "oracle_sort_and_bin", "oracle_rasterize_fwd",
                     "oracle_rasterize_bwd", "oracle_emit_keys_wide", "oracle_sort_and_bin_wide"):
            getattr(_lib, name).restype = ctypes.c_int64
    return _lib


def _f(a: np.ndarray) -> ctypes.Array:
    assert a.dtype == np.float32 and a.flags.c_contiguous, (a.dtype, a.flags)
    return a.ctypes.data_as(_f32p)


def _i(a: np.ndarray) -> ctypes.Array:
    assert a.dtype == np.int32 and a.flags.c_contiguous, (a.dtype, a.flags)
    return a.ctypes.data_as(_i32p)


def _c32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def _ci32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.int32))


def _rows(a: np.ndarray, width: int) -> int:
    return a.size // width


def logf(x) -> np.ndarray:
    x = _c32(x).ravel()
    y = np.empty_like(x)
    lib().oracle_logf_n(_f(x), _f(y), _i64(x.size))
    return y


def expf(x) -> np.ndarray:
    x = _c32(x).ravel()
    y = np.empty_like(x)
    lib().oracle_expf_n(_f(x), _f(y), _i64(x.size))
    return y


def blend_expf(x) -> np.ndarray:
    """The blends' exp(-sigma) sequence (x <= 0)."""
    x = _c32(x).ravel()
    y = np.empty_like(x)
    lib().oracle_blend_expf_n(_f(x), _f(y), _i64(x.size))
    return y


def key_layout(B: int, H: int, W: int) -> tuple[dict, bool]:
    out = np.zeros(6, np.int32)
    ok = lib().oracle_key_layout(_i32(B), _i32(H), _i32(W), _i(out))
    names = ("tile_bounds_x", "tile_bounds_y", "num_tiles", "tile_n_bits", "image_n_bits",
             "depth_bits")
    return dict(zip(names, (int(v) for v in out))), bool(ok)


def set_wide_keys(force: bool) -> None:
    """Force the 64-bit key for every layout (as the reference's tests patch _use_32bit_keys)."""
    lib().oracle_set_wide_keys(ctypes.c_int(int(bool(force))))


def key_mode(B: int, H: int, W: int) -> int:
    """0: packed 32-bit key, 1: 64-bit key, -2: even the 64-bit key overflows."""
    return int(lib().oracle_key_mode(_i32(B), _i32(H), _i32(W)))


def project_fwd(means, scales, quats_xyzw, viewmat, opacities, *, n, total, img_shape, f, c,
                glob_scale=1.0, clip_thresh=0.01, transforms=None, transform_ids=None,
                num_transforms=None):
    """Projection forward over ``total = B*n`` flat items; returns the six reference outputs.

    ``transforms`` is (K, 4, 4) shared or (B*K, 4, 4) per image; ``num_transforms`` is K.
    """
    means, scales, quats, viewmat, opac = map(_c32, (means, scales, quats_xyzw, viewmat,
                                                     opacities))
    has_tf = transforms is not None
    tf = _c32(transforms if has_tf else np.zeros((1, 4, 4)))
    ids = _ci32(transform_ids if has_tf else np.full((1,), -1))
    num_tf = int(num_transforms if num_transforms is not None else tf.size // 16)
    H, W = img_shape
    xys = np.empty((total, 2), np.float32)
    depths = np.empty(total, np.float32)
    radii = np.empty(total, np.int32)
    conics = np.empty((total, 3), np.float32)
    nth = np.empty(total, np.int32)
    cum = np.empty(total, np.int32)
    lib().oracle_project_fwd(
        _f(means), _i64(_rows(means, 3)), _f(scales), _i64(_rows(scales, 3)), _f(quats),
        _i64(_rows(quats, 4)), _f(viewmat), _i64(_rows(viewmat, 4)), _f(opac),
        _i64(opac.size), _f(tf), _i64(_rows(tf, 16)), _i(ids), _i32(n), _i32(num_tf),
        _i32(int(has_tf)), _i64(total), _i32(H), _i32(W), _f32(f[0]), _f32(f[1]), _f32(c[0]),
        _f32(c[1]), _f32(glob_scale), _f32(clip_thresh), _f(xys), _f(depths), _i(radii),
        _f(conics), _i(nth), _i(cum))
    return xys, depths, radii, conics, nth, cum


def emit_keys(xys, depths, radii, conics, map_opac, cum, *, n, B, img_shape):
    """Unsorted keys/ids in emission order and the per-image depth range (packed key), or
    int64 keys and ids (64-bit key; the depth range is then unused and returned as zeros)."""
    xys, depths, conics, map_opac = map(_c32, (xys, depths, conics, map_opac))
    radii, cum = _ci32(radii).ravel(), _ci32(cum).ravel()
    M = int(cum[-1]) if cum.size else 0
    ids = np.full(max(M, 1), -1, np.int32)
    mm = np.zeros(2 * B, np.float32)
    H, W = img_shape
    if key_mode(B, H, W) == 1:
        keys = np.full(max(M, 1), -999, np.int64)
        m = lib().oracle_emit_keys_wide(_f(xys), _f(depths), _i(radii), _f(conics), _f(map_opac),
                                        _i64(map_opac.size), _i(cum), _i32(n), _i32(B), _i32(H),
                                        _i32(W), keys.ctypes.data_as(_i64p), _i(ids),
                                        _i64(keys.size))
    else:
        keys = np.full(max(M, 1), -999, np.int32)
        m = lib().oracle_emit_keys(_f(xys), _f(depths), _i(radii), _f(conics), _f(map_opac),
                                   _i64(map_opac.size), _i(cum), _i32(n), _i32(B), _i32(H),
                                   _i32(W), _i(keys), _i(ids), _i64(keys.size), _f(mm))
    if m < 0:
        raise ValueError(f"oracle emit_keys failed with code {m}")
    return keys[:m], ids[:m], mm


def sort_and_bin(xys, depths, radii, conics, map_opac, cum, *, n, B, img_shape):
    """Sorted keys, sorted gaussian ids and (B*num_tiles, 2) tile bins."""
    xys, depths, conics, map_opac = map(_c32, (xys, depths, conics, map_opac))
    radii, cum = _ci32(radii).ravel(), _ci32(cum).ravel()
    M = int(cum[-1]) if cum.size else 0
    H, W = img_shape
    lay, _ = key_layout(B, H, W)
    wide = key_mode(B, H, W) == 1
    keys = np.zeros(max(M, 1), np.int64 if wide else np.int32)
    ids = np.zeros(max(M, 1), np.int32)
    bins = np.zeros((B * lay["num_tiles"], 2), np.int32)
    fn = lib().oracle_sort_and_bin_wide if wide else lib().oracle_sort_and_bin
    kp = keys.ctypes.data_as(_i64p) if wide else _i(keys)
    m = fn(_f(xys), _f(depths), _i(radii), _f(conics), _f(map_opac), _i64(map_opac.size),
           _i(cum), _i32(n), _i32(B), _i32(H), _i32(W), kp, _i(ids), _i64(keys.size), _i(bins))
    if m < 0:
        raise ValueError(f"oracle sort_and_bin failed with code {m}")
    return keys[:m], ids[:m], bins


def blend_fwd(colors, opacities, background, xys, conics, sorted_ids, tile_bins, *, B,
              img_shape, depths=None):
    """Returns (img, Ts, fidx, stats) and, when depths is given, the expected depth (B*H, W)."""
    colors, opac, bg, xys, conics = map(_c32, (colors, opacities, background, xys, conics))
    ids, bins = _ci32(sorted_ids), _ci32(tile_bins)
    if ids.size == 0:
        ids = np.zeros(1, np.int32)
    H, W = img_shape
    Ts = np.empty((B * H, W), np.float32)
    fidx = np.empty((B * H, W), np.int32)
    img = np.empty((B * H, W, 3), np.float32)
    stats = np.zeros(2, np.int64)
    dep = None if depths is None else _c32(depths)
    out_depth = None if depths is None else np.empty((B * H, W), np.float32)
    lib().oracle_blend_fwd(_f(colors), _i64(_rows(colors, 3)), _f(opac), _i64(opac.size), _f(bg),
                           _i64(_rows(bg, 3)), _f(xys), _f(conics), _i(ids), _i(bins), _i32(B),
                           _i32(H), _i32(W), _f(Ts), _i(fidx), _f(img),
                           stats.ctypes.data_as(_i64p), None if dep is None else _f(dep),
                           None if out_depth is None else _f(out_depth))
    if depths is None:
        return img, Ts, fidx, stats
    return img, Ts, fidx, stats, out_depth


def rasterize_fwd(colors, opacities, map_opac, background, xys, depths, radii, conics, cum, *,
                  n, B, img_shape, render_depth=False):
    """Returns (out_img (B*H, W, 3), final_Ts, final_idx, stats=[Pc, Pr], M), plus the expected
    depth (B*H, W) last when render_depth."""
    colors, opac, mopac, bg, xys, depths, conics = map(
        _c32, (colors, opacities, map_opac, background, xys, depths, conics))
    radii, cum = _ci32(radii).ravel(), _ci32(cum).ravel()
    H, W = img_shape
    Ts = np.empty((B * H, W), np.float32)
    fidx = np.empty((B * H, W), np.int32)
    img = np.empty((B * H, W, 3), np.float32)
    stats = np.zeros(2, np.int64)
    out_depth = np.empty((B * H, W), np.float32) if render_depth else None
    m = lib().oracle_rasterize_fwd(
        _f(colors), _i64(_rows(colors, 3)), _f(opac), _i64(opac.size), _f(mopac),
        _i64(mopac.size), _f(bg), _i64(_rows(bg, 3)), _f(xys), _f(depths), _i(radii),
        _f(conics), _i(cum), _i32(n), _i32(B), _i32(H), _i32(W), _f(Ts), _i(fidx), _f(img),
        stats.ctypes.data_as(_i64p), None if out_depth is None else _f(out_depth))
    if m < 0:
        raise ValueError(f"oracle rasterize_fwd failed with code {m}")
    if render_depth:
        return img, Ts, fidx, stats, int(m), out_depth
    return img, Ts, fidx, stats, int(m)


def rasterize_bwd(colors, opacities, map_opac, background, xys, depths, radii, conics, cum,
                  final_Ts, final_idx, v_out, *, n, B_out, B_geom, img_shape, v_out_depth=None):
    """Returns (v_colors, v_opacity, v_xy, v_conic, stats=[Qc, Qr]) sized B_out*n; with
    v_out_depth (the depth channel's cotangent) also v_depths, last."""
    colors, opac, mopac, bg, xys, depths, conics, Ts, vout = map(
        _c32, (colors, opacities, map_opac, background, xys, depths, conics, final_Ts, v_out))
    radii, cum, fidx = _ci32(radii).ravel(), _ci32(cum).ravel(), _ci32(final_idx)
    H, W = img_shape
    nout = B_out * n
    v_colors = np.empty((nout, 3), np.float32)
    v_opac = np.empty(nout, np.float32)
    v_xy = np.empty((nout, 2), np.float32)
    v_conic = np.empty((nout, 3), np.float32)
    stats = np.zeros(2, np.int64)
    vd = None if v_out_depth is None else _c32(v_out_depth)
    v_depths = None if vd is None else np.empty(nout, np.float32)
    m = lib().oracle_rasterize_bwd(
        _f(colors), _i64(_rows(colors, 3)), _f(opac), _i64(opac.size), _f(mopac),
        _i64(mopac.size), _f(bg), _i64(_rows(bg, 3)), _f(xys), _f(depths), _i(radii),
        _f(conics), _i(cum), _f(Ts), _i(fidx), _f(vout), _i64(vout.size // (3 * W)), _i32(n),
        _i32(B_out), _i32(B_geom), _i32(H), _i32(W), _f(v_colors), _f(v_opac), _f(v_xy),
        _f(v_conic), stats.ctypes.data_as(_i64p), None if vd is None else _f(vd),
        _i64(0 if vd is None else vd.size // W), None if v_depths is None else _f(v_depths))
    if m < 0:
        raise ValueError(f"oracle rasterize_bwd failed with code {m}")
    if vd is None:
        return v_colors, v_opac, v_xy, v_conic, stats
    return v_colors, v_opac, v_xy, v_conic, stats, v_depths


def rasterize_bwd_f64(colors, opacities, map_opac, background, xys, depths, radii, conics, cum,
                      final_Ts, final_idx, v_out, *, n, B_out, B_geom, img_shape,
                      v_out_depth=None):
    """The float64 truth of rasterize_bwd: the float walk's pairs and accept decisions, every
    value after them in double (oracle_rasterize_bwd_f64). Returns float64 (v_colors,
    v_opacity, v_xy, v_conic) sized B_out*n, and v_depths last when v_out_depth is given."""
    colors, opac, mopac, bg, xys, depths, conics, Ts, vout = map(
        _c32, (colors, opacities, map_opac, background, xys, depths, conics, final_Ts, v_out))
    radii, cum, fidx = _ci32(radii).ravel(), _ci32(cum).ravel(), _ci32(final_idx)
    H, W = img_shape
    vd = None if v_out_depth is None else _c32(v_out_depth)
    NG = 9 if vd is None else 10
    out = np.empty((B_out * n, NG), np.float64)
    fn = lib().oracle_rasterize_bwd_f64
    fn.restype = ctypes.c_int64
    m = fn(_f(colors), _i64(_rows(colors, 3)), _f(opac), _i64(opac.size), _f(mopac),
           _i64(mopac.size), _f(bg), _i64(_rows(bg, 3)), _f(xys), _f(depths), _i(radii),
           _f(conics), _i(cum), _f(Ts), _i(fidx), _f(vout), _i64(vout.size // (3 * W)), _i32(n),
           _i32(B_out), _i32(B_geom), _i32(H), _i32(W), None if vd is None else _f(vd),
           _i64(0 if vd is None else vd.size // W),
           out.ctypes.data_as(ctypes.POINTER(ctypes.c_double)))
    if m < 0:
        raise ValueError(f"oracle rasterize_bwd_f64 failed with code {m}")
    res = (out[:, 0:3], out[:, 8].copy(), out[:, 6:8], out[:, 3:6])
    return res if vd is None else res + (out[:, 9].copy(),)


def project_bwd(means, scales, quats_xyzw, viewmat, radii, conics, v_xy, v_depth, v_conic, *, n,
                B, f, glob_scale=1.0, transforms=None, transform_ids=None, num_transforms=None):
    """Returns (v_mean3d, v_scale, v_quat (xyzw), v_viewmat (B*4, 4), v_transforms)."""
    means, scales, quats, viewmat, conics, v_xy, v_depth, v_conic = map(
        _c32, (means, scales, quats_xyzw, viewmat, conics, v_xy, v_depth, v_conic))
    radii = _ci32(radii).ravel()
    has_tf = transforms is not None
    tf = _c32(transforms if has_tf else np.zeros((1, 4, 4)))
    ids = _ci32(transform_ids if has_tf else np.full((1,), -1))
    K = int(num_transforms if num_transforms is not None else (tf.size // 16 if has_tf else 1))
    total = B * n
    v_mean = np.empty((total, 3), np.float32)
    v_scale = np.empty((total, 3), np.float32)
    v_quat = np.empty((total, 4), np.float32)
    v_view = np.zeros((B * 4, 4), np.float32)
    v_tf = np.zeros((B * K, 4, 4), np.float32)
    lib().oracle_project_bwd(
        _f(means), _i64(_rows(means, 3)), _f(scales), _i64(_rows(scales, 3)), _f(quats),
        _i64(_rows(quats, 4)), _f(viewmat), _i64(_rows(viewmat, 4)), _i(radii), _i64(radii.size),
        _f(conics), _i64(_rows(conics, 3)), _f(v_xy), _i64(_rows(v_xy, 2)), _f(v_depth),
        _i64(v_depth.size), _f(v_conic), _i64(_rows(v_conic, 3)), _f(tf), _i64(_rows(tf, 16)),
        _i(ids), _i32(n), _i32(K), _i32(int(has_tf)), _i32(B), _f32(f[0]), _f32(f[1]),
        _f32(glob_scale), _f(v_mean), _f(v_scale), _f(v_quat), _f(v_view), _f(v_tf))
    return v_mean, v_scale, v_quat, v_view, v_tf


def set_threads(n: int) -> int:
    """Set the oracle's OpenMP thread count; returns the count in effect."""
    return int(lib().oracle_set_threads(ctypes.c_int(int(n))))


# ---------------------------------------------------------------- antialiasing compensation

_EPS = np.float32(0.3)        # splax/_project/_project.py:95 (eps), as float32
_EPS2 = np.float32(0.3 * 0.3)  # the reference's (eps * eps), formed in Python, as float32


def compensation_rho(conics):
    """opacity_compensation's rho (splax/_project/_project.py:113-117) in float32, in the
    expression's order; returns (rho, rho2) with rho2 the unclipped argument. Items with
    radii <= 0 take 1 in the reference; the fused blend never reads them."""
    cn = np.asarray(conics, np.float32).reshape(-1, 3)
    a, b, c = cn[:, 0], cn[:, 1], cn[:, 2]
    with np.errstate(invalid="ignore"):
        rho2 = (np.float32(1.0) - _EPS * (a + c)) + _EPS2 * (a * c - b * b)
        cl = np.where(rho2 < 0, np.float32(0), rho2)
        cl = np.where(cl > 1, np.float32(1), cl)
        return np.sqrt(cl).astype(np.float32), rho2.astype(np.float32)


def compensation_vjp(v_blend_opac, opac, conics):
    """Cotangents of blend_opac = opac * rho(conics) for a blend-opacity cotangent, by the
    reverse-mode rules of the reference's expression (sqrt' = 0.5 / rho; maximum / minimum pass
    1 inside, 1/2 at a tie, 0 outside); returns (v_opac, v_conics) in float32, per item."""
    f = np.float32
    vbo = np.asarray(v_blend_opac, np.float32).reshape(-1)
    o = np.asarray(opac, np.float32).reshape(-1)
    cn = np.asarray(conics, np.float32).reshape(-1, 3)
    a, b, c = cn[:, 0], cn[:, 1], cn[:, 2]
    rho, rho2 = compensation_rho(cn)
    with np.errstate(divide="ignore", invalid="ignore"):
        v_o = vbo * rho
        v_rho = vbo * o
        v_cl = v_rho * (f(0.5) / rho)
        m_lo = np.where(rho2 > 0, f(1), np.where(rho2 == 0, f(0.5), f(0)))
        y = np.where(rho2 > 0, rho2, f(0))
        m_hi = np.where(y < 1, f(1), np.where(y == 1, f(0.5), f(0)))
        v_r2 = (v_cl * m_hi) * m_lo
        v_s = -(_EPS * v_r2)
        v_t = _EPS2 * v_r2
        vc = np.stack([v_s + v_t * c, -(v_t * b) - v_t * b, v_s + v_t * a], axis=1)
    return v_o.astype(np.float32), vc.astype(np.float32)
