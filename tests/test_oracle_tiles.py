"""Pins the oracle's tile intersection, key emission, sort and bin edges (CPU only).

- Conservativeness by brute force: every tile holding a pixel centre inside the opacity-aware
  ellipse (A dx^2 + 2B dx dy + C dy^2 <= t, i.e. alpha >= 1/255 when t is not capped) is emitted
  (splax/_intersect.py:46-183).
- emit == count: each visible item owns exactly num_tiles_hit contiguous slots at cum[idx-1]
  (tests/test_warp_rasterize.py:433-487).
- Key layout decode and depth monotonicity (splax/_rasterize/_sort/_kernels.py:116-125).
- Sort: equals numpy's stable argsort of the emission-order keys (radix_sort_pairs contract).
- Bins: closed form from the sorted keys, including the M == 1 behaviour
  (splax/_rasterize/_sort/_kernels.py:214-241).
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import random_scene
from oracle import oracle as O


def _project(sc, B=1, vms=None):
    H, W = sc["img_shape"]
    n = sc["means"].shape[0]
    q = np.roll(sc["quats"], -1, axis=-1)
    vm = sc["vm"] if vms is None else vms.reshape(-1, 4)
    return O.project_fwd(sc["means"], sc["scales"], q, vm, sc["opac"], n=n, total=B * n,
                         img_shape=(H, W), f=sc["f"], c=sc["c"])


@pytest.mark.parametrize("seed", [0, 1])
def test_tiles_conservative_brute_force(seed):
    sc = random_scene(400, 96, 112, seed=seed, scale_range=(0.01, 0.08))
    H, W = sc["img_shape"]
    xys, depths, radii, conics, nth, cum = _project(sc)
    keys, ids, _ = O.emit_keys(xys, depths, radii, conics, sc["opac"], cum, n=400, B=1,
                               img_shape=(H, W))
    lay, _ = O.key_layout(1, H, W)
    tiles = (keys >> lay["depth_bits"]) & ((1 << lay["tile_n_bits"]) - 1)
    tbx = lay["tile_bounds_x"]
    jj, ii = np.meshgrid(np.arange(W) + 0.5, np.arange(H) + 0.5)
    pix_tile = (np.arange(H)[:, None] // 16) * tbx + np.arange(W)[None, :] // 16
    checked = 0
    for g in np.nonzero(radii > 0)[0]:
        A, Bc, C = conics[g].astype(np.float64)
        t = min(3.33 ** 2, 2 * np.log(sc["opac"][g, 0] * 255.0))
        dx = jj - xys[g, 0]
        dy = ii - xys[g, 1]
        q = A * dx * dx + 2 * Bc * dx * dy + C * dy * dy
        inside = q <= t * (1 - 1e-4)
        need = set(np.unique(pix_tile[inside]).tolist())
        got = set(tiles[ids == g].tolist())
        assert need <= got, f"gaussian {g}: missing tiles {sorted(need - got)[:5]}"
        # emitted tiles lie inside the ellipse's bounding box (in tiles)
        ex, ey = np.sqrt(t * C / (A * C - Bc * Bc)), np.sqrt(t * A / (A * C - Bc * Bc))
        for tile in got:
            ty, tx = divmod(tile, tbx)
            assert tx * 16 <= xys[g, 0] + ex + 1e-3 and (tx + 1) * 16 >= xys[g, 0] - ex - 1e-3
            assert ty * 16 <= xys[g, 1] + ey + 1e-3 and (ty + 1) * 16 >= xys[g, 1] - ey - 1e-3
        checked += 1
    assert checked > 100


@pytest.mark.parametrize("n,H,W", [(20_000, 256, 256), (30_000, 300, 420)])
def test_emit_matches_count(n, H, W):
    sc = random_scene(n, H, W, seed=n)
    xys, depths, radii, conics, nth, cum = _project(sc)
    np.testing.assert_array_equal(cum, np.cumsum(nth))
    keys, ids, _ = O.emit_keys(xys, depths, radii, conics, sc["opac"], cum, n=n, B=1,
                               img_shape=(H, W))
    M = int(cum[-1])
    assert keys.shape == (M,) and (ids >= 0).all() and (keys >= 0).all()
    starts = np.concatenate([[0], cum[:-1]])
    owner = np.repeat(np.arange(n), nth)
    np.testing.assert_array_equal(ids, owner)
    lay, _ = O.key_layout(1, H, W)
    tiles = keys >> lay["depth_bits"]
    for g in np.nonzero(nth > 1)[0][:3000]:
        s, e = starts[g], cum[g]
        assert len(np.unique(tiles[s:e])) == e - s, "a gaussian emitted a tile twice"


def test_key_fields_and_depth_monotone():
    sc = random_scene(5000, 128, 128, seed=9)
    B = 3
    vms = np.stack([sc["vm"]] * B)
    vms[1, 0, 3] += 0.2
    vms[2, 2, 3] += 0.5
    n = 5000
    xys, depths, radii, conics, nth, cum = _project(sc, B=B, vms=vms)
    keys, ids, mm = O.emit_keys(xys, depths, radii, conics, sc["opac"], cum, n=n, B=B,
                                img_shape=(128, 128))
    lay, _ = O.key_layout(B, 128, 128)
    db, tb = lay["depth_bits"], lay["tile_n_bits"]
    img = keys >> (db + tb)
    np.testing.assert_array_equal(img, ids // n)
    assert ((keys >> db) & ((1 << tb) - 1)).max() < lay["num_tiles"]
    dq = keys & ((1 << db) - 1)
    for b in range(B):
        vis = (radii > 0) & (np.arange(B * n) // n == b)
        assert mm[2 * b] == depths[vis].min() and mm[2 * b + 1] == depths[vis].max()
        sel = img == b
        d = depths[ids[sel]]
        o = np.argsort(d, kind="stable")
        assert np.all(np.diff(dq[sel][o]) >= 0), "depth_q not monotone in depth"
        assert dq[sel].min() == 0 and dq[sel].max() == (1 << db) - 1


def _bins_closed_form(sorted_keys, B, num_tiles, db, tb):
    bins = np.zeros((B * num_tiles, 2), np.int32)
    if sorted_keys.size == 0:
        return bins
    k = sorted_keys >> db
    flat = (k >> tb) * num_tiles + (k & ((1 << tb) - 1))
    uniq, first = np.unique(flat, return_index=True)
    last = np.r_[first[1:], flat.size]
    bins[uniq, 0] = first
    bins[uniq, 1] = last
    if flat.size == 1:  # index 0 writes only the start
        bins[uniq, 1] = 0
    return bins


@pytest.mark.parametrize("B", [1, 4])
def test_sort_and_bins_closed_form(B):
    sc = random_scene(8000, 144, 176, seed=B)
    n = 8000
    vms = np.stack([sc["vm"]] * B)
    for b in range(B):
        vms[b, 0, 3] += 0.1 * b
    xys, depths, radii, conics, nth, cum = _project(sc, B=B, vms=vms)
    H, W = sc["img_shape"]
    ek, eid, _ = O.emit_keys(xys, depths, radii, conics, sc["opac"], cum, n=n, B=B,
                             img_shape=(H, W))
    sk, sid, bins = O.sort_and_bin(xys, depths, radii, conics, sc["opac"], cum, n=n, B=B,
                                   img_shape=(H, W))
    order = np.argsort(ek, kind="stable")  # ascending key, ties in emission order
    np.testing.assert_array_equal(sk, ek[order])
    np.testing.assert_array_equal(sid, eid[order])
    # the same order is the closed form (key, flat gaussian index)
    np.testing.assert_array_equal(order, np.lexsort((eid, ek)))
    lay, _ = O.key_layout(B, H, W)
    ref = _bins_closed_form(sk, B, lay["num_tiles"], lay["depth_bits"], lay["tile_n_bits"])
    np.testing.assert_array_equal(bins, ref)


def test_single_intersection_bin_quirk():
    """M == 1: the reference's bin-edge kernel writes only the start, so the bin stays [0, 0)."""
    H = W = 64
    means = np.array([[0.0, 0.0, 5.0]], np.float32)
    scales = np.full((1, 3), 0.01, np.float32)
    quats = np.array([[0.0, 0.0, 0.0, 1.0]], np.float32)  # xyzw identity
    opac = np.array([[0.9]], np.float32)
    vm = np.eye(4, dtype=np.float32)
    xys, depths, radii, conics, nth, cum = O.project_fwd(
        means, scales, quats, vm, opac, n=1, total=1, img_shape=(H, W), f=(50.0, 50.0),
        c=(40.0, 40.0))
    assert cum[-1] == 1
    sk, sid, bins = O.sort_and_bin(xys, depths, radii, conics, opac, cum, n=1, B=1,
                                   img_shape=(H, W))
    assert (bins == 0).all()


# ---------------------------------------------------------------- 64-bit key path
# splax/_rasterize/_sort/_sort.py:23-26,56-66,143-170 and _sort/_kernels.py:156-211,244-269.


@pytest.fixture
def wide_keys():
    O.set_wide_keys(True)
    yield
    O.set_wide_keys(False)


def test_key_mode_fallback_and_overflow():
    """B=1 at 1080p packs (18 depth bits); B=8 leaves 15 < 16 and falls back to the 64-bit key
    (the reference's tests/test_warp_rasterize.py:321-359); image + tile bits above 32 overflow."""
    assert O.key_mode(1, 1080, 1920) == 0
    assert O.key_mode(8, 1080, 1920) == 1
    assert O.key_mode(16, 512, 512) == 0  # config 3: 17 depth bits
    assert O.key_mode(1 << 20, 1080, 1920) == -2  # 20 image + 13 tile bits
    O.set_wide_keys(True)
    try:
        assert O.key_mode(1, 1080, 1920) == 1
    finally:
        O.set_wide_keys(False)


@pytest.mark.parametrize("B", [1, 3])
def test_wide_keys_fields_sort_and_bins(B, wide_keys):
    sc = random_scene(6000, 144, 176, seed=10 + B)
    n = 6000
    vms = np.stack([sc["vm"]] * B)
    for b in range(B):
        vms[b, 0, 3] += 0.1 * b
    xys, depths, radii, conics, nth, cum = _project(sc, B=B, vms=vms)
    H, W = sc["img_shape"]
    lay, _ = O.key_layout(B, H, W)
    ek, eid, _ = O.emit_keys(xys, depths, radii, conics, sc["opac"], cum, n=n, B=B,
                             img_shape=(H, W))
    assert ek.dtype == np.int64 and ek.size == int(cum[-1])
    # fields: image and tile above bit 32, the float depth's bits below
    hi = (ek.view(np.uint64) >> np.uint64(32)).astype(np.int64)
    tb = lay["tile_n_bits"]
    np.testing.assert_array_equal(hi >> tb, eid // n)
    np.testing.assert_array_equal((ek & 0xFFFFFFFF).astype(np.uint32),
                                  depths.ravel()[eid].view(np.uint32))
    sk, sid, bins = O.sort_and_bin(xys, depths, radii, conics, sc["opac"], cum, n=n, B=B,
                                   img_shape=(H, W))
    order = np.lexsort((eid, ek.view(np.uint64)))  # (key as unsigned, flat index)
    np.testing.assert_array_equal(sk, ek[order])
    np.testing.assert_array_equal(sid, eid[order])
    # within a tile, the order is by exact depth
    ref = _bins_closed_form(hi[order], B, lay["num_tiles"], 0, tb)
    np.testing.assert_array_equal(bins, ref)


def test_wide_and_packed_renders_agree():
    """The 64-bit key orders by exact depth, the packed key by quantized depth; the images
    agree within the reference's bound (tests/test_warp_rasterize.py:280-318: max abs < 0.05,
    PSNR > 65 dB)."""
    sc = random_scene(20000, 128, 128, seed=21, scale_range=(0.01, 0.05))
    n = 20000
    xys, depths, radii, conics, nth, cum = _project(sc)
    H, W = sc["img_shape"]
    args = (sc["colors"], sc["opac"], sc["opac"], np.ones(3, np.float32), xys, depths, radii,
            conics, cum)
    packed = O.rasterize_fwd(*args, n=n, B=1, img_shape=(H, W))[0]
    O.set_wide_keys(True)
    try:
        wide = O.rasterize_fwd(*args, n=n, B=1, img_shape=(H, W))[0]
    finally:
        O.set_wide_keys(False)
    d = np.abs(packed.astype(np.float64) - wide)
    mse = float((d ** 2).mean())
    psnr = 99.0 if mse == 0 else -10 * np.log10(mse)
    assert d.max() < 0.05 and psnr > 65, (d.max(), psnr)


def test_wide_batch_equals_stack_bit_exact(wide_keys):
    """With the 64-bit key each image's (tile, depth) order does not depend on B, so a batched
    render equals the per-image renders bit for bit (tests/test_warp_batch.py:45-56)."""
    sc = random_scene(3000, 96, 96, seed=5)
    n, B = 3000, 3
    vms = np.stack([sc["vm"]] * B)
    vms[1, 0, 3] += 0.2
    vms[2, 1, 3] -= 0.15
    H, W = sc["img_shape"]
    xys, depths, radii, conics, nth, cum = _project(sc, B=B, vms=vms)
    bimg = O.rasterize_fwd(sc["colors"], sc["opac"], sc["opac"], sc["bg"], xys, depths, radii,
                           conics, cum, n=n, B=B, img_shape=(H, W))[0].reshape(B, H, W, 3)
    for b in range(B):
        p = _project(sc, B=1, vms=vms[b:b + 1])
        img = O.rasterize_fwd(sc["colors"], sc["opac"], sc["opac"], sc["bg"], *p[:4], p[5],
                              n=n, B=1, img_shape=(H, W))[0].reshape(H, W, 3)
        np.testing.assert_array_equal(bimg[b], img)
