"""Walk statistics of the backward blend, counted on the CPU from the oracle's forward.

blend_bwd_kernel walks, per 16x16 tile and per 8x8 quadrant (one wave64), the list of staged
records whose 4x4 sub-block box mask meets the quadrant, back to front from the tile's largest
final index. An entry above the quadrant's largest final index is skipped on the scalar unit; an
entry whose ballot of "in range" lanes (idx <= final_idx, 0 <= sigma <= sigma_max) is empty costs
the sigma evaluation only; every other entry is an event that pays the full per-pair arithmetic
and the wave reduction. This script counts those entries and the lanes that contribute
(alpha >= 1/255) per event over every tile (or a seeded sample scaled to the whole image) of the
workload's first camera, and the lanes an event's ellipse reaches before the final-index test.

It also counts the forward blend's row walks: each 16-lane row of a wave walks the list of the
records that reach its 4x4 sub-block (the ellipse {sigma <= sigma_max} meets a pixel centre of
it), and a pixel stops at the record that brings its transmittance to 1e-4 or below, so in each
batch of 256 staged records a row takes as many steps as its slowest pixel and a wave as many as
its slowest row. Printed: the wave steps
as built, the steps if the four rows of each wave were balanced (every row a quarter of the
wave's total), and the steps if every pixel's own steps were packed 64 to a wave step.

The geometry evaluates in float64 (a pair at a threshold edge may count differently from the
float32 kernel; that moves the totals far below their printed precision). Run from the repository
root (test infrastructure: it uses the CPU oracle):

    python tests/blend_event_counts.py [--config 2] [--tiles N] [--threads 8]
"""

from __future__ import annotations

import argparse
import sys
import time
from pathlib import Path

import numpy as np

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))

from oracle import oracle as O  # noqa: E402
from splax_amd.scenes import make_scene  # noqa: E402

ALPHA_MAX, ALPHA_MIN, SIGMA_CAP = 0.999, 1.0 / 255.0, 87.0


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", type=int, default=2)
    ap.add_argument("--tiles", type=int, default=None, help="sample this many tiles (seeded)")
    ap.add_argument("--threads", type=int, default=8)
    args = ap.parse_args()
    O.set_threads(args.threads)
    s = make_scene(args.config)
    q = np.roll(s.quats, -1, axis=-1)
    xys, depths, radii, conics, nth, cum = O.project_fwd(
        s.means, s.scales, q, s.viewmats[0], s.opacities, n=s.n, total=s.n,
        img_shape=s.img_shape, f=s.f, c=s.c)
    # antialiased workloads blend o * rho(conic) and intersect tiles with the raw opacity
    blend_opac = s.opacities.reshape(-1)
    if s.antialiased:
        blend_opac = (blend_opac * O.compensation_rho(conics)[0]).astype(np.float32)
    _, _, fidx, _, M = O.rasterize_fwd(s.colors, blend_opac.reshape(-1, 1), s.opacities,
                                       s.background, xys, depths, radii, conics, cum, n=s.n,
                                       B=1, img_shape=s.img_shape)
    _, sid, bins = O.sort_and_bin(xys, depths, radii, conics, s.opacities, cum, n=s.n, B=1,
                                  img_shape=s.img_shape)
    H, W = s.img_shape
    tiles_x = (W + 15) // 16
    fidx = fidx.reshape(H, W)
    opac = blend_opac.astype(np.float64)
    ca, cb, cc = (conics[:, k].astype(np.float64) for k in range(3))
    # the packed record's sigma_max and cull box (pack_record in csrc/splat_common.hpp)
    with np.errstate(divide="ignore", invalid="ignore"):
        smax = np.minimum(np.log(opac * 255.0) + 1e-3, SIGMA_CAP)
        det = ca * cc - cb * cb
        ex = np.sqrt(2 * smax * cc / det) * 1.01 + 0.01
        ey = np.sqrt(2 * smax * ca / det) * 1.01 + 0.01
        boxed = (ca > 0) & (cc > 0) & (det > 0) & ((ca + cc) ** 2 < 1e4 * det)
    ex = np.where(boxed, ex, np.inf)
    ey = np.where(boxed, ey, np.inf)

    live = np.flatnonzero(bins[:, 1] > bins[:, 0])
    rng = np.random.default_rng(0)
    sample = live if args.tiles is None else rng.choice(live, size=min(args.tiles, len(live)),
                                                         replace=False)
    tot = dict(entries=0, past_wmax=0, reach=0, events=0, lanes=0, pairs_in_range=0,
               reach_lanes=0, fwd_wave_steps=0, fwd_row_balanced=0.0, fwd_packed=0.0)
    # sub-block (row-major over the tile's 4x4 grid of 4x4 pixel blocks) of each pixel
    sub = (np.arange(16)[:, None] // 4) * 4 + np.arange(16)[None, :] // 4
    hist = np.zeros(65, np.int64)
    t0 = time.time()
    for tile in sample:
        ty, tx = divmod(int(tile), tiles_x)
        rs, re = (int(v) for v in bins[tile])
        ii = np.arange(16)[:, None] + ty * 16
        jj = np.arange(16)[None, :] + tx * 16
        inside = (ii < H) & (jj < W)
        bf = np.where(inside, fidx[np.minimum(ii, H - 1), np.minimum(jj, W - 1)], rs - 1)
        start = min(int(bf.max()), re - 1)
        idx = np.arange(start, rs - 1, -1)
        if len(idx) == 0:
            continue
        g = sid[idx]
        dx = xys[g, 0][:, None, None] - (jj + 0.5)[None]
        dy = xys[g, 1][:, None, None] - (ii + 0.5)[None]
        sig = 0.5 * (ca[g][:, None, None] * dx * dx + cc[g][:, None, None] * dy * dy) + \
            cb[g][:, None, None] * dx * dy
        with np.errstate(over="ignore", invalid="ignore"):
            alpha = np.minimum(ALPHA_MAX, opac[g][:, None, None] * np.exp(-sig))
        reach = (sig >= 0) & (sig <= smax[g][:, None, None]) & inside[None]
        in_range = reach & (idx[:, None, None] <= bf[None])
        contrib = in_range & (alpha >= ALPHA_MIN)
        # forward row walks: the tile's whole range in sorted order
        gf = sid[rs:re]
        fdx = xys[gf, 0][:, None, None] - (jj + 0.5)[None]
        fdy = xys[gf, 1][:, None, None] - (ii + 0.5)[None]
        fsig = 0.5 * (ca[gf][:, None, None] * fdx * fdx + cc[gf][:, None, None] * fdy * fdy) + \
            cb[gf][:, None, None] * fdx * fdy
        with np.errstate(over="ignore", invalid="ignore"):
            falpha = np.minimum(ALPHA_MAX, opac[gf][:, None, None] * np.exp(-fsig))
        fr = (fsig >= 0) & (fsig <= smax[gf][:, None, None]) & inside[None]
        fa = np.where(fr & (falpha >= ALPHA_MIN), falpha, 0.0)
        below = np.cumprod(1.0 - fa, axis=0) <= 1e-4
        nf = len(gf)
        stop = np.where(below.any(0), below.argmax(0), nf)  # the record where a pixel stops
        on_list = np.stack([fr[:, sub == b].any(1) for b in range(16)], 1)  # [records, 16]
        pos = np.cumsum(on_list, axis=0)
        pos = np.vstack([np.zeros((1, 16), pos.dtype), pos])  # pos[k + 1]: entries in [0, k]
        last = np.minimum(stop, nf - 1)
        for a in range(0, nf, 256):  # the kernel's batches of 256 staged records
            e = min(a + 256, nf)
            # a pixel's steps in this batch: its list's entries from a to its stop (inclusive)
            upto = np.minimum(last, e - 1)
            steps = np.where(inside & (stop >= a), pos[upto + 1, sub] - pos[a, sub], 0)
            row_task = np.array([steps[sub == b].max() for b in range(16)])
            for w in range(4):
                rows = [(2 * (w >> 1) + (r >> 1)) * 4 + 2 * (w & 1) + (r & 1) for r in range(4)]
                tot["fwd_wave_steps"] += int(row_task[rows].max())
                tot["fwd_row_balanced"] += float(row_task[rows].mean())
            tot["fwd_packed"] += float(steps.sum()) / 64.0
        x0 = tx * 16 + np.arange(4) * 4 + 0.5
        y0 = ty * 16 + np.arange(4) * 4 + 0.5
        xm = (xys[g, 0][:, None] + ex[g][:, None] >= x0) & (xys[g, 0][:, None] - ex[g][:, None]
                                                           <= x0 + 3)
        ym = (xys[g, 1][:, None] + ey[g][:, None] >= y0) & (xys[g, 1][:, None] - ey[g][:, None]
                                                           <= y0 + 3)
        for qy in range(2):
            for qx in range(2):
                listed = xm[:, 2 * qx:2 * qx + 2].any(1) & ym[:, 2 * qy:2 * qy + 2].any(1)
                rows, cols = slice(qy * 8, qy * 8 + 8), slice(qx * 8, qx * 8 + 8)
                wmax = int(bf[rows, cols].max())
                walked = listed & (idx <= wmax)
                ir = in_range[:, rows, cols].reshape(len(idx), 64)
                ev = walked & ir.any(1)
                lanes = contrib[:, rows, cols].reshape(len(idx), 64).sum(1)
                tot["entries"] += int(listed.sum())
                tot["past_wmax"] += int(walked.sum())
                tot["reach"] += int((walked & reach[:, rows, cols].reshape(len(idx), 64)
                                     .any(1)).sum())
                tot["events"] += int(ev.sum())
                tot["lanes"] += int(lanes[ev].sum())
                tot["pairs_in_range"] += int(ir[ev].sum())
                tot["reach_lanes"] += int(reach[:, rows, cols].reshape(len(idx), 64)[ev].sum())
                hist += np.bincount(lanes[ev], minlength=65)
    scale = len(live) / len(sample)
    print(f"config {args.config}, first of {s.B} camera(s): {H}x{W}, M = {M}, "
          f"tiles with intersections {len(live)}, "
          f"sampled {len(sample)} (scale {scale:.3f}), {time.time() - t0:.0f} s")
    print(f"quadrant-list entries        {tot['entries'] * scale:.4g}")
    print(f"  walked (<= quadrant max)   {tot['past_wmax'] * scale:.4g}")
    print(f"  walked, ellipse reaches a pixel centre of the quadrant "
          f"{tot['reach'] * scale:.4g}")
    print(f"  events (a lane in range)   {tot['events'] * scale:.4g}")
    print(f"contributing pairs           {tot['lanes'] * scale:.4g}")
    print(f"contributing lanes per event {tot['lanes'] / max(tot['events'], 1):.2f} of 64")
    print(f"in-range lanes per event     {tot['pairs_in_range'] / max(tot['events'], 1):.2f}")
    print(f"lanes the ellipse reaches per event (before the final-index test) "
          f"{tot['reach_lanes'] / max(tot['events'], 1):.2f}")
    cdf = np.cumsum(hist) / max(hist.sum(), 1)
    print("events with <= k contributing lanes: " +
          ", ".join(f"k={k}: {cdf[k]:.2f}" for k in (1, 4, 8, 16, 32, 48)))
    ws = tot["fwd_wave_steps"]
    print(f"forward row walks: wave steps {ws * scale:.4g}; rows balanced within each wave "
          f"{tot['fwd_row_balanced'] * scale:.4g} ({tot['fwd_row_balanced'] / max(ws, 1):.3f}); "
          f"every pixel's steps packed 64 per wave step {tot['fwd_packed'] * scale:.4g} "
          f"({tot['fwd_packed'] / max(ws, 1):.3f})")


if __name__ == "__main__":
    main()
