"""Pins the tightness of the oracle's tile walk and the depth quantization of its keys (CPU only).

Tile walk. The reference's AccuTile walk (splax/_intersect.py:146-183) marches the ellipse
A dx^2 + 2B dx dy + C dy^2 <= t column strip by column strip, takes the exact cross-axis extent
of the ellipse inside each strip (the rolling intersect lines plus the bbox extremum when it lies
inside the strip) and emits the tiles floor(min/16) .. floor(max/16) of that strip, clipped to
the ellipse's tile rectangle (:82-85, :166-168). The ellipse meets strip u in a convex set, so a
tile row lies in that range exactly when the ellipse meets the tile: the emitted set is the set of
image tiles whose square meets the ellipse, whichever axis the walk takes. The checker below
decides that set independently, in float64, by minimizing the quadratic form over each tile
square (the minimum of a convex quadratic over a box is 0 inside it, else on one of its four
edges, each a clamped 1-D minimum), and requires equality with the emitted set except for tiles
whose square is within DELTA pixels of meeting / missing the ellipse (where the float32 walk's
rounding decides).

depth_q. `_map_intersects_32bit` quantizes depth_q = int32((d - dmin) / drange * maxq), clamped
(splax/_rasterize/_sort/_kernels.py:116-124). The checker forms x = (d - dmin) / drange * maxq
exactly (float64 of the float32 operands) and requires depth_q == floor(x) except where an
integer lies within the float32 evaluation's error bound (four roundings, 4.1 * 2^-24 * x) of x.

Each checker is shown to reject a planted mistake: a walk that emits the whole tile rectangle or
one extra tile row in a column, and a depth_q that rounds instead of truncating.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import random_scene
from oracle import oracle as O

# Pixels: a tile whose square comes this close to the ellipse boundary may go either way.
DELTA = 1e-4
EXTEND_SQ = 3.33 * 3.33


def _project(sc, B=1, vms=None):
    H, W = sc["img_shape"]
    n = sc["means"].shape[0]
    q = np.roll(sc["quats"], -1, axis=-1)
    vm = sc["vm"] if vms is None else vms.reshape(-1, 4)
    return O.project_fwd(sc["means"], sc["scales"], q, vm, sc["opac"], n=n, total=B * n,
                         img_shape=(H, W), f=sc["f"], c=sc["c"])


def _box_qmin(A, B, C, x0, x1, y0, y1):
    """min over [x0, x1] x [y0, y1] (offsets from the centre) of A x^2 + 2B xy + C y^2, for a
    positive definite form; arrays of boxes, float64."""
    inside = (x0 <= 0) & (0 <= x1) & (y0 <= 0) & (0 <= y1)
    best = np.full(np.shape(x0), np.inf)
    for X in (x0, x1):  # vertical edges: minimize over y
        y = np.clip(-B * X / C, y0, y1)
        best = np.minimum(best, A * X * X + 2 * B * X * y + C * y * y)
    for Y in (y0, y1):  # horizontal edges: minimize over x
        x = np.clip(-B * Y / A, x0, x1)
        best = np.minimum(best, A * x * x + 2 * B * x * Y + C * Y * Y)
    return np.where(inside, 0.0, best)


def tile_set_violations(xys, conics, opac, radii, tiles, ids, *, img_shape, delta=DELTA):
    """Compares the emitted (gaussian, tile) pairs with the tiles whose squares meet each visible
    gaussian's ellipse. Returns (missing, extra, ambiguous, checked): emitted sets lacking a tile
    that surely meets the ellipse, emitted tiles that surely miss it, tiles within `delta` of
    either, and the number of gaussians checked."""
    H, W = img_shape
    tx_n, ty_n = (W + 15) // 16, (H + 15) // 16
    order = np.argsort(ids, kind="stable")
    ids_s, tiles_s = ids[order], tiles[order]
    starts = np.searchsorted(ids_s, np.arange(len(radii) + 1))
    missing = extra = ambiguous = checked = 0
    for g in np.nonzero(np.asarray(radii).ravel() > 0)[0]:
        A, Bc, C = np.asarray(conics[g], np.float64)
        px, py = np.asarray(xys[g], np.float64)
        t = min(EXTEND_SQ, 2.0 * np.log(float(np.asarray(opac).ravel()[g]) * 255.0))
        det = A * C - Bc * Bc
        ex, ey = np.sqrt(t * C / det), np.sqrt(t * A / det)
        u0 = max(0, int(np.floor((px - ex) / 16)) - 1)
        u1 = min(tx_n - 1, int(np.floor((px + ex) / 16)) + 1)
        v0 = max(0, int(np.floor((py - ey) / 16)) - 1)
        v1 = min(ty_n - 1, int(np.floor((py + ey) / 16)) + 1)
        got = set(tiles_s[starts[g]:starts[g + 1]].tolist())
        if u1 < u0 or v1 < v0:
            extra += len(got)
            checked += 1
            continue
        uu, vv = np.meshgrid(np.arange(u0, u1 + 1), np.arange(v0, v1 + 1), indexing="ij")
        x0, y0 = uu * 16.0 - px, vv * 16.0 - py
        q_in = _box_qmin(A, Bc, C, x0 + delta, x0 + 16 - delta, y0 + delta, y0 + 16 - delta)
        q_out = _box_qmin(A, Bc, C, x0 - delta, x0 + 16 + delta, y0 - delta, y0 + 16 + delta)
        sure_in = q_in <= t
        sure_out = q_out > t
        ids_win = (vv * tx_n + uu)
        need = set(ids_win[sure_in].tolist())
        never = set(ids_win[sure_out].tolist())
        window = set(ids_win.ravel().tolist())
        missing += len(need - got)
        extra += len(got & never) + len(got - window)
        ambiguous += int((~sure_in & ~sure_out).sum())
        checked += 1
    return missing, extra, ambiguous, checked


def _emitted(sc, n):
    H, W = sc["img_shape"]
    xys, depths, radii, conics, nth, cum = _project(sc)
    keys, ids, mm = O.emit_keys(xys, depths, radii, conics, sc["opac"], cum, n=n, B=1,
                                img_shape=(H, W))
    lay, _ = O.key_layout(1, H, W)
    tiles = (keys >> lay["depth_bits"]) & ((1 << lay["tile_n_bits"]) - 1)
    return (xys, depths, radii, conics), keys, ids, tiles, lay, mm


SCENES = [
    # many multi-tile ellipses, some cut by the image border (mean_scale 1.2 reaches past it)
    dict(n=500, H=160, W=208, seed=0, scale_range=(0.01, 0.12), mean_scale=1.0),
    dict(n=500, H=144, W=144, seed=1, scale_range=(0.02, 0.2), mean_scale=1.2),
    # ragged image (neither side a multiple of 16), small and large splats
    dict(n=800, H=125, W=171, seed=2, scale_range=(0.005, 0.15), mean_scale=0.8),
]


@pytest.mark.parametrize("cfg", SCENES, ids=lambda c: f"seed{c['seed']}")
def test_tile_walk_emits_exactly_the_tiles_the_ellipse_meets(cfg):
    cfg = dict(cfg)
    n = cfg.pop("n")
    H, W = cfg.pop("H"), cfg.pop("W")
    sc = random_scene(n, H, W, **cfg)
    (xys, depths, radii, conics), keys, ids, tiles, lay, _ = _emitted(sc, n)
    missing, extra, ambiguous, checked = tile_set_violations(
        xys, conics, sc["opac"], radii, tiles, ids, img_shape=(H, W))
    assert checked > 200
    assert len(tiles) > 3 * checked  # mostly multi-tile ellipses
    assert missing == 0, f"{missing} tiles the ellipse meets were not emitted"
    assert extra == 0, f"{extra} emitted tiles miss the ellipse"
    # the undecided band is a sliver: a handful of tiles at most
    assert ambiguous <= max(3, len(tiles) // 2000), ambiguous


def test_tile_checker_rejects_bbox_and_widened_walks():
    """Planted mistakes: emitting each ellipse's whole tile rectangle, or one tile row past the
    walk's max_v in one column, both show up as extra tiles."""
    cfg = dict(SCENES[0])
    n = cfg.pop("n")
    H, W = cfg.pop("H"), cfg.pop("W")
    sc = random_scene(n, H, W, **cfg)
    (xys, depths, radii, conics), keys, ids, tiles, lay, _ = _emitted(sc, n)
    tx_n, ty_n = (W + 15) // 16, (H + 15) // 16
    # (1) the tile rectangle of every emitted set
    bb_ids, bb_tiles = [], []
    for g in np.unique(ids):
        tg = tiles[ids == g]
        ty, tx = np.divmod(tg, tx_n)
        for v in range(ty.min(), ty.max() + 1):
            for u in range(tx.min(), tx.max() + 1):
                bb_ids.append(g)
                bb_tiles.append(v * tx_n + u)
    _, extra, _, _ = tile_set_violations(xys, conics, sc["opac"], radii, np.array(bb_tiles),
                                         np.array(bb_ids), img_shape=(H, W))
    assert extra > 100, "whole-rectangle emission was not detected"
    # (2) one extra row below the lowest emitted tile of the first column of each gaussian
    caught = tried = 0
    for g in np.unique(ids):
        tg = tiles[ids == g]
        ty, tx = np.divmod(tg, tx_n)
        u = tx.min()
        vmax = ty[tx == u].max()
        if vmax + 1 >= ty_n:
            continue
        mut_tiles = np.concatenate([tg, [(vmax + 1) * tx_n + u]])
        mut_ids = np.full(mut_tiles.size, g)
        r = np.zeros_like(radii)
        r[g] = 1
        _, extra, _, _ = tile_set_violations(xys, conics, sc["opac"], r, mut_tiles, mut_ids,
                                             img_shape=(H, W))
        tried += 1
        caught += extra > 0
    assert tried > 200 and caught >= tried - 2, (caught, tried)


# ---------------------------------------------------------------- depth_q


def depth_q_violations(keys, ids, depths, radii, *, n, B, lay):
    """Keys whose depth field differs from floor((d - dmin) / drange * maxq) (exact), outside the
    float32 evaluation's error band around an integer; plus the number of keys checked away
    from such a band."""
    db, tb = lay["depth_bits"], lay["tile_n_bits"]
    maxq = (1 << db) - 1
    img = keys.astype(np.int64) >> (db + tb)
    dq = keys.astype(np.int64) & maxq
    d = np.asarray(depths, np.float64).ravel()
    vis = np.asarray(radii).ravel() > 0
    bad = clear = 0
    for b in range(B):
        sel = img == b
        if not sel.any():
            continue
        dv = d[b * n:(b + 1) * n][vis[b * n:(b + 1) * n]]
        dmin, dmax = dv.min(), dv.max()
        x = (d[ids[sel]] - dmin) / (dmax - dmin) * maxq if dmax > dmin else np.zeros(sel.sum())
        want = np.clip(np.floor(x), 0, maxq).astype(np.int64)
        band = 4.1 * 2.0 ** -24 * np.abs(x) + 1e-12
        near = np.abs(x - np.rint(x)) <= band
        bad += int(((dq[sel] != want) & ~near).sum())
        bad += int((np.abs(dq[sel] - want) > 1).sum())
        clear += int((~near).sum())
    return bad, clear


# Depth-bit widths of the benchmark layouts: 19 (800^2), 18 (1080p), 17 (B=16 at 512^2), 16 (B=4
# at 1600x1060). Above about 21 bits the float32 evaluation's error band reaches a whole unit of
# x, so truncation is only decidable at these widths.
@pytest.mark.parametrize("B,H,W", [(1, 800, 800), (1, 1080, 1920), (16, 512, 512),
                                   (4, 1060, 1600)])
def test_depth_q_is_the_truncated_fraction(B, H, W):
    n = 3000
    sc = random_scene(n, H, W, seed=B + H)
    vms = np.stack([sc["vm"]] * B)
    for b in range(B):
        vms[b, 2, 3] += 0.3 * b
    xys, depths, radii, conics, nth, cum = _project(sc, B=B, vms=vms)
    keys, ids, mm = O.emit_keys(xys, depths, radii, conics, sc["opac"], cum, n=n, B=B,
                                img_shape=(H, W))
    lay, packed = O.key_layout(B, H, W)
    assert lay["depth_bits"] >= 16
    bad, clear = depth_q_violations(keys, ids, depths, radii, n=n, B=B, lay=lay)
    assert bad == 0
    assert clear > 0.8 * keys.size  # the band covers about 2 * 4.1 * 2^-24 * x of each unit


def test_depth_q_checker_rejects_rounding():
    """A planted depth_q that rounds to nearest instead of truncating is caught."""
    n, H, W = 4000, 800, 800
    sc = random_scene(n, H, W, seed=3)
    xys, depths, radii, conics, nth, cum = _project(sc)
    keys, ids, mm = O.emit_keys(xys, depths, radii, conics, sc["opac"], cum, n=n, B=1,
                                img_shape=(H, W))
    lay, _ = O.key_layout(1, H, W)
    db = lay["depth_bits"]
    maxq = (1 << db) - 1
    dmin, dmax = np.float32(mm[0]), np.float32(mm[1])
    f = (depths[ids].astype(np.float32) - dmin) / np.float32(dmax - dmin)
    rounded = np.clip(np.rint(f * np.float32(maxq)), 0, maxq).astype(np.int64)
    planted = (keys.astype(np.int64) & ~np.int64(maxq)) | rounded
    bad, _ = depth_q_violations(planted, ids, depths, radii, n=n, B=1, lay=lay)
    assert bad > 0.3 * keys.size


def test_depth_q_single_depth_is_zero():
    """drange <= 0 (one visible depth) gives depth_q = 0 (splax/_rasterize/_sort/_kernels.py:
    116-124)."""
    means = np.array([[0.0, 0.0, 0.0], [0.05, 0.0, 0.0]], np.float32)
    scales = np.full((2, 3), 0.05, np.float32)
    quats = np.tile(np.array([[0.0, 0.0, 0.0, 1.0]], np.float32), (2, 1))
    opac = np.array([[0.9], [0.8]], np.float32)
    vm = np.eye(4, dtype=np.float32)
    vm[2, 3] = 5.0
    xys, depths, radii, conics, nth, cum = O.project_fwd(
        means, scales, quats, vm, opac, n=2, total=2, img_shape=(64, 64), f=(64.0, 64.0),
        c=(32.0, 32.0))
    assert (radii > 0).all() and depths[0] == depths[1]
    keys, ids, mm = O.emit_keys(xys, depths, radii, conics, opac, cum, n=2, B=1,
                                img_shape=(64, 64))
    lay, _ = O.key_layout(1, 64, 64)
    assert keys.size > 0 and ((keys & ((1 << lay["depth_bits"]) - 1)) == 0).all()


@pytest.mark.parametrize("cfg,n", [(0, None), (2, 20_000)])
def test_tile_walk_tight_on_benchmark_scenes(cfg, n):
    """Config 0 (the reference's CPU-runnable case) whole, and 20k gaussians of config 2 (planes,
    1920x1080: large pixel coordinates and thin, steep ellipses)."""
    from splax_amd.scenes import make_scene

    s = make_scene(cfg) if n is None else make_scene(cfg, n=n)
    q = np.roll(s.quats, -1, axis=-1)
    xys, depths, radii, conics, nth, cum = O.project_fwd(
        s.means, s.scales, q, s.viewmats[0], s.opacities, n=s.n, total=s.n,
        img_shape=s.img_shape, f=s.f, c=s.c)
    keys, ids, _ = O.emit_keys(xys, depths, radii, conics, s.opacities, cum, n=s.n, B=1,
                               img_shape=s.img_shape)
    lay, _ = O.key_layout(1, *s.img_shape)
    tiles = (keys >> lay["depth_bits"]) & ((1 << lay["tile_n_bits"]) - 1)
    missing, extra, ambiguous, checked = tile_set_violations(
        xys, conics, s.opacities, radii, tiles, ids, img_shape=s.img_shape)
    assert checked > 1000
    assert missing == 0 and extra == 0, (missing, extra)
    assert ambiguous <= max(3, len(tiles) // 2000), ambiguous
