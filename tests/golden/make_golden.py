"""Writes tests/golden/tiny_render.npz: a tiny seeded scene with the CPU oracle's outputs.

The reference ships no golden vectors for this path (its tests compare against gsplat live), so
this fixture records the oracle's projection, sort/bin, forward blend and both VJPs on a 64-gaussian
40x40 scene. The CPU suite checks the oracle still reproduces it bit for bit (regression); the GPU
suite checks the gfx950 library against it. Run: python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))

from conftest import random_scene  # noqa: E402
from oracle import oracle as O  # noqa: E402

OUT = Path(__file__).resolve().parent / "tiny_render.npz"


def make():
    n, H, W = 64, 40, 40
    sc = random_scene(n, H, W, seed=2024, scale_range=(0.03, 0.12), mean_scale=0.5,
                      opac_range=(0.2, 0.95))
    q = np.roll(sc["quats"], -1, axis=-1)
    xys, depths, radii, conics, nth, cum = O.project_fwd(
        sc["means"], sc["scales"], q, sc["vm"], sc["opac"], n=n, total=n, img_shape=(H, W),
        f=sc["f"], c=sc["c"])
    keys, ids, bins = O.sort_and_bin(xys, depths, radii, conics, sc["opac"], cum, n=n, B=1,
                                     img_shape=(H, W))
    img, Ts, fidx, stats, M = O.rasterize_fwd(sc["colors"], sc["opac"], sc["opac"], sc["bg"], xys,
                                              depths, radii, conics, cum, n=n, B=1,
                                              img_shape=(H, W))
    v_out = np.random.default_rng(7).uniform(-1, 1, (H, W, 3)).astype(np.float32)
    v_colors, v_opac, v_xy, v_conic, _ = O.rasterize_bwd(
        sc["colors"], sc["opac"], sc["opac"], sc["bg"], xys, depths, radii, conics, cum, Ts, fidx,
        v_out, n=n, B_out=1, B_geom=1, img_shape=(H, W))
    v_depth = np.random.default_rng(8).uniform(-1, 1, n).astype(np.float32)
    v_mean, v_scale, v_quat, v_view, _ = O.project_bwd(
        sc["means"], sc["scales"], q, sc["vm"], radii, conics, v_xy, v_depth, v_conic, n=n, B=1,
        f=sc["f"])
    return dict(
        means=sc["means"], scales=sc["scales"], quats_wxyz=sc["quats"], colors=sc["colors"],
        opac=sc["opac"], bg=sc["bg"], viewmat=sc["vm"], img_shape=np.array([H, W]),
        f=np.array(sc["f"], np.float32), c=np.array(sc["c"], np.float32),
        xys=xys, depths=depths, radii=radii, conics=conics, num_tiles_hit=nth, cum=cum,
        keys=keys, ids=ids, bins=bins, img=img, final_Ts=Ts, final_idx=fidx, v_out=v_out,
        v_colors=v_colors, v_opac=v_opac, v_xy=v_xy, v_conic=v_conic, v_depth=v_depth,
        v_mean=v_mean, v_scale=v_scale, v_quat_xyzw=v_quat, v_viewmat=v_view)


if __name__ == "__main__":
    np.savez_compressed(OUT, **make())
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")
