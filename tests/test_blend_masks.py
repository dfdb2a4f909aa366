"""The forward blend's sub-block masks keep every sub-block a record can reach (CPU only).

blend_fwd_kernel walks, per 4x4 sub-block, only the records whose 16-bit mask has that
sub-block's bit; a record is dropped from a sub-block only when no pixel centre there can pass the
blend's `0 <= sigma <= sigma_max` test, so the blended sequence and the image stay the
reference's. `subblock_mask_tight` (csrc/blend.hip) forms the mask from the exact x-extent of the
ellipse Q <= 1.0201 sigma_max over each 4-row band, from tile-independent parts the record pack
forms (1 / a, the scaled ellipse's half-widths, its rightmost point's height); this test restates
both step by step in float32 (the hardware square root as a correctly rounded one: the function's
margins are orders of magnitude above its error) and checks, against a brute force of the blend's own
sigma expression (two FMAs, float32) over all 256 pixel centres of each tile, that
- no pixel centre with sigma in [0, sigma_max] lies in a sub-block the mask drops, on records
  from the benchmark scenes' projections and on synthetic extremes (thin ellipses up to the box
  mode's conditioning limit, sub-pixel and very large ones), in every tile a record's box meets;
- the mask is tighter than the bounding-box mask (it drops more than 5% of the sub-blocks the
  box keeps).
Planted mistakes (a band's extent from its end rows only; the extreme point's height mirrored) are
shown to break the first property.
"""

from __future__ import annotations

import numpy as np

from splax_amd.scenes import make_scene

f32 = np.float32
SCALE2 = f32(1.0201)
BW = 16


def _fma(a, b, c):
    """float32 fma: the product of two float32 values is exact in float64."""
    return (np.asarray(a, np.float64) * np.asarray(b, np.float64)
            + np.asarray(c, np.float64)).astype(f32)


def pack(x, y, a, b, c, o):
    """The packed record fields the masks read (pack_record, csrc/splat_common.hpp): a/2, c/2,
    sigma_max, the box half-widths and the cull mode (0 box, 1 keep, 2 none)."""
    x, y, a, b, c, o = (np.asarray(v, f32) for v in (x, y, a, b, c, o))
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        smax = np.minimum(np.log(o.astype(np.float64) * 255.0).astype(f32) + f32(1e-3), f32(87))
        smax = np.where(o > 0, smax, -np.inf).astype(f32)
        det = (a * c - b * b).astype(f32)
        tr = (a + c).astype(f32)
        ex2 = (f32(2) * smax * c / det).astype(f32)
        ey2 = (f32(2) * smax * a / det).astype(f32)
        box = (a > 0) & (c > 0) & (det > 0) & (tr * tr < f32(1e4) * det) & (ex2 < f32(1e30)) & \
            (ey2 < f32(1e30))
        sx = (np.sqrt(ex2).astype(f32) * f32(1.01)).astype(f32)
        sy = (np.sqrt(ey2).astype(f32) * f32(1.01)).astype(f32)
        ex = np.where(box, sx + f32(0.01), 0).astype(f32)
        ey = np.where(box, sy + f32(0.01), 0).astype(f32)
        inv_a = np.where(box, f32(1) / a, 0).astype(f32)
        dy_r = np.where(box, (-(b * sx).astype(f32) / c).astype(f32), 0).astype(f32)
    mode = np.where(~(smax >= 0), 2, np.where(box, 0, 1))
    return dict(x=x, y=y, ha=(f32(0.5) * a).astype(f32), b=b, hc=(f32(0.5) * c).astype(f32),
                smax=smax, ex=ex, ey=ey, inv_a=inv_a, dy_r=dy_r, mode=mode)


def mask_tight(R, tx, ty, peaks=True, peak_sign=1):
    """subblock_mask_tight, element-wise over records R (dict of arrays) at tiles (tx, ty).
    peaks=False or peak_sign=-1 plant mistakes (no extreme point inside a band; its height
    mirrored) for the checker to catch."""
    scale2, margin = SCALE2, True
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        a = (f32(2) * R["ha"]).astype(f32)
        b = R["b"]
        c = (f32(2) * R["hc"]).astype(f32)
        s2 = (f32(2) * (scale2 * R["smax"]).astype(f32)).astype(f32)
        det = (a * c - b * b).astype(f32)
        inv_a = R["inv_a"]
        ex = (R["ex"] - f32(0.01)).astype(f32)
        ey = (R["ey"] - f32(0.01)).astype(f32)
        dy_r = (f32(peak_sign) * R["dy_r"]).astype(f32)
        m = (f32(0.01) + f32(1e-3) * ex).astype(f32) if margin else np.zeros_like(ex)
        two_a_s = (a * s2).astype(f32)
        nb_a = (-b * inv_a).astype(f32)
        bx = ((np.asarray(tx) * BW).astype(f32) + f32(0.5) - R["x"]).astype(f32)
        by = ((np.asarray(ty) * BW).astype(f32) + f32(0.5) - R["y"]).astype(f32)
        mask = np.zeros(np.broadcast(bx, by).shape, np.uint32)
        for j in range(4):
            y0 = (by + f32(4 * j)).astype(f32)
            d0 = np.maximum(y0, -ey - m).astype(f32)
            d1 = np.minimum((y0 + f32(3)).astype(f32), (ey + m).astype(f32)).astype(f32)
            w0 = (np.sqrt(np.maximum(two_a_s - det * (d0 * d0), 0).astype(f32)) * inv_a).astype(f32)
            w1 = (np.sqrt(np.maximum(two_a_s - det * (d1 * d1), 0).astype(f32)) * inv_a).astype(f32)
            c0, c1 = (nb_a * d0).astype(f32), (nb_a * d1).astype(f32)
            hi = np.maximum(c0 + w0, c1 + w1).astype(f32)
            lo = np.minimum(c0 - w0, c1 - w1).astype(f32)
            if peaks:
                hi = np.where((dy_r >= d0) & (dy_r <= d1), ex, hi)
                lo = np.where((-dy_r >= d0) & (-dy_r <= d1), -ex, lo)
            hi, lo = (hi + m).astype(f32), (lo - m).astype(f32)
            band = d0 <= d1
            for i in range(4):
                x0 = (bx + f32(4 * i)).astype(f32)
                keep = band & (x0 <= hi) & ((x0 + f32(3)).astype(f32) >= lo)
                mask |= np.where(keep, np.uint32(1 << (4 * j + i)), np.uint32(0))
    mode = R["mode"]
    return np.where(mode == 2, np.uint32(0), np.where(mode == 1, np.uint32(0xFFFF), mask))


def mask_box(R, tx, ty):
    """subblock_mask (the box test) element-wise."""
    xm = np.zeros(np.broadcast(R["x"], tx).shape, np.uint32)
    ym = np.zeros_like(xm)
    for k in range(4):
        x0 = ((np.asarray(tx) * BW + 4 * k).astype(f32) + f32(0.5)).astype(f32)
        y0 = ((np.asarray(ty) * BW + 4 * k).astype(f32) + f32(0.5)).astype(f32)
        xm |= np.where((R["x"] + R["ex"] >= x0) & (R["x"] - R["ex"] <= x0 + f32(3)), 1 << k, 0
                       ).astype(np.uint32)
        ym |= np.where((R["y"] + R["ey"] >= y0) & (R["y"] - R["ey"] <= y0 + f32(3)), 1 << k, 0
                       ).astype(np.uint32)
    m = np.zeros_like(xm)
    for r in range(4):
        m |= np.where((ym >> r) & 1, xm << (4 * r), 0).astype(np.uint32)
    mode = R["mode"]
    return np.where(mode == 2, np.uint32(0), np.where(mode == 1, np.uint32(0xFFFF), m))


def reach(R, tx, ty):
    """Brute force: bit k set when a pixel centre of sub-block k passes 0 <= sigma <= sigma_max,
    sigma = dx (a/2 dx + b dy) + (c/2 dy) dy with two FMAs (blend_sigma)."""
    out = np.zeros(np.broadcast(R["x"], tx).shape, np.uint32)
    for py in range(BW):
        for px in range(BW):
            X = (np.asarray(tx) * BW + px).astype(f32) + f32(0.5)
            Y = (np.asarray(ty) * BW + py).astype(f32) + f32(0.5)
            dx = (R["x"] - X).astype(f32)
            dy = (R["y"] - Y).astype(f32)
            sig = _fma(dx, _fma(R["ha"], dx, (R["b"] * dy).astype(f32)),
                       ((R["hc"] * dy).astype(f32) * dy).astype(f32))
            hit = (sig >= 0) & (sig <= R["smax"])
            out |= np.where(hit, np.uint32(1 << (4 * (py // 4) + px // 4)), np.uint32(0))
    return out


def _scene_records(cfg, n, rng, count):
    from oracle import oracle as O
    s = make_scene(cfg, n=n)
    q = np.roll(s.quats, -1, axis=-1)
    xys, depths, radii, conics, nth, cum = O.project_fwd(
        s.means, s.scales, q, s.viewmats[0], s.opacities, n=s.n, total=s.n,
        img_shape=s.img_shape, f=s.f, c=s.c)
    vis = np.flatnonzero(radii > 0)
    pick = rng.choice(vis, size=min(count, len(vis)), replace=False)
    return pack(xys[pick, 0], xys[pick, 1], conics[pick, 0], conics[pick, 1], conics[pick, 2],
                s.opacities.reshape(-1)[pick])


def _synthetic_records(rng, count):
    """Thin (conditioning up to the box limit), tiny and huge ellipses at sub-pixel offsets."""
    x = rng.uniform(100, 140, count)
    y = rng.uniform(100, 140, count)
    ang = rng.uniform(0, np.pi, count)
    # eigenvalues of the conic: scale^-2 with scales from 0.05 px to 200 px, aspect up to ~95
    s1 = np.exp(rng.uniform(np.log(0.05), np.log(200), count))
    s2 = s1 * np.exp(rng.uniform(0, np.log(95), count))
    l1, l2 = 1 / s1 ** 2, 1 / s2 ** 2
    cs, sn = np.cos(ang), np.sin(ang)
    a = l1 * cs * cs + l2 * sn * sn
    c = l1 * sn * sn + l2 * cs * cs
    b = (l1 - l2) * cs * sn
    o = rng.uniform(0.005, 0.99, count)
    return pack(x, y, a, b, c, o)


def _tiles_of(R, k_extra=1):
    """(record index, tx, ty) for every tile a record's widened box meets, plus a ring."""
    rec, txs, tys = [], [], []
    for r in range(len(R["x"])):
        if R["mode"][r] != 0:
            continue
        x0 = int(np.floor((R["x"][r] - R["ex"][r]) / BW)) - k_extra
        x1 = int(np.floor((R["x"][r] + R["ex"][r]) / BW)) + k_extra
        y0 = int(np.floor((R["y"][r] - R["ey"][r]) / BW)) - k_extra
        y1 = int(np.floor((R["y"][r] + R["ey"][r]) / BW)) + k_extra
        if (x1 - x0 + 1) * (y1 - y0 + 1) > 64:  # huge ellipses: a sample of their tiles
            cx, cy = int(R["x"][r] // BW), int(R["y"][r] // BW)
            xs = [x0, x1, cx, cx - 1, cx + 1]
            ys = [y0, y1, cy, cy - 1, cy + 1]
            for tx in xs:
                for ty in ys:
                    rec.append(r); txs.append(tx); tys.append(ty)
            continue
        for tx in range(x0, x1 + 1):
            for ty in range(y0, y1 + 1):
                rec.append(r); txs.append(tx); tys.append(ty)
    return np.array(rec), np.array(txs), np.array(tys)


def _check(R, **kw):
    idx, tx, ty = _tiles_of(R)
    Rt = {k: v[idx] for k, v in R.items()}
    need = reach(Rt, tx, ty)
    got = mask_tight(Rt, tx, ty, **kw)
    box = mask_box(Rt, tx, ty)
    return need, got, box


def test_tight_mask_is_conservative_and_tighter_than_the_box():
    rng = np.random.default_rng(3)
    for R in (_scene_records(2, 60_000, rng, 1500), _scene_records(1, 30_000, rng, 800),
              _synthetic_records(rng, 1500)):
        need, got, box = _check(R)
        missed = need & ~got
        assert not missed.any(), f"{int((missed != 0).sum())} (record, tile) pairs lose a sub-block"
        # tighter than the box overall (its margin can reach 1e-3 ex past the box's edge)
        dropped = int(np.unpackbits((box & ~got).view(np.uint8)).sum())
        kept_box = int(np.unpackbits(box.view(np.uint8)).sum())
        assert dropped > 0.05 * kept_box, (dropped, kept_box)


def test_planted_mistakes_lose_sub_blocks():
    """Taking a band's extent from its end rows only (no extreme point inside the band), or the
    extreme point's height with the wrong sign, drops sub-blocks the ellipse reaches."""
    rng = np.random.default_rng(4)
    R = _synthetic_records(rng, 1500)
    for kw in (dict(peaks=False), dict(peak_sign=-1)):
        need, got, _ = _check(R, **kw)
        assert (need & ~got).any(), kw
