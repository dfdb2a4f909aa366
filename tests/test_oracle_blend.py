"""Pins the oracle's forward blend (splax/_rasterize/_kernels.py:102-205) on the CPU.

- A float64 dense brute-force blend (tests/torch_ref.py) over the same tile assignment and
  front-to-back order reproduces the image, final_Ts and final_idx.
- Closed form for a single gaussian: img = bg + alpha (c - bg) where alpha >= 1/255, else bg.
- Closed form for two fully overlapping gaussians (front occludes back).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import random_scene
from oracle import oracle as O
from torch_ref import blend_ref, tile_members


def _pipeline(sc, n):
    H, W = sc["img_shape"]
    q = np.roll(sc["quats"], -1, axis=-1)
    proj = O.project_fwd(sc["means"], sc["scales"], q, sc["vm"], sc["opac"], n=n, total=n,
                         img_shape=(H, W), f=sc["f"], c=sc["c"])
    xys, depths, radii, conics, nth, cum = proj
    img, Ts, fidx, stats, M = O.rasterize_fwd(sc["colors"], sc["opac"], sc["opac"], sc["bg"],
                                              xys, depths, radii, conics, cum, n=n, B=1,
                                              img_shape=(H, W))
    sk, sid, bins = O.sort_and_bin(xys, depths, radii, conics, sc["opac"], cum, n=n, B=1,
                                   img_shape=(H, W))
    return proj, (img, Ts, fidx, stats, M), (sk, sid, bins)


def _front_to_back(sk, sid, depth_bits):
    dq = sk & ((1 << depth_bits) - 1)
    first = {}
    for d, g in zip(dq, sid):
        first.setdefault(int(g), int(d))
    gs = np.array(sorted(first, key=lambda g: (first[g], g)), np.int64)
    return gs


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_blend_matches_float64_brute_force(seed):
    n, H, W = 300, 48, 64
    sc = random_scene(n, H, W, seed=seed, scale_range=(0.02, 0.1), mean_scale=0.6,
                      opac_range=(0.2, 0.95))
    proj, (img, Ts, fidx, stats, M), (sk, sid, bins) = _pipeline(sc, n)
    xys, depths, radii, conics, nth, cum = proj
    lay, _ = O.key_layout(1, H, W)
    order = _front_to_back(sk, sid, lay["depth_bits"])
    mem = tile_members(sk, sid, order, img_shape=(H, W), depth_bits=lay["depth_bits"],
                       tile_bits=lay["tile_n_bits"])
    t = lambda a: torch.from_numpy(np.asarray(a, np.float64))  # noqa: E731
    rimg, rT, acc = blend_ref(t(xys), t(conics), t(sc["opac"][:, 0]), t(sc["colors"]),
                              t(sc["bg"]), order, torch.from_numpy(mem), img_shape=(H, W))
    err = np.abs(img.reshape(H, W, 3) - rimg.numpy())
    assert err.max() < 1e-5, f"max abs image error {err.max()}"
    np.testing.assert_allclose(Ts.reshape(H, W), rT.numpy(), atol=1e-6, rtol=1e-5)
    # final_idx: sorted-array index of each pixel's last blended gaussian (0 when none)
    acc = acc.numpy()
    tbx = lay["tile_bounds_x"]
    ref_idx = np.zeros((H, W), np.int64)
    for i in range(H):
        for j in range(W):
            ks = np.nonzero(acc[:, i, j])[0]
            if ks.size == 0:
                continue
            g = order[ks[-1]]
            tile = (i // 16) * tbx + j // 16
            s, e = bins[tile]
            ref_idx[i, j] = s + int(np.nonzero(sid[s:e] == g)[0][0])
    np.testing.assert_array_equal(fidx.reshape(H, W), ref_idx)
    assert stats[0] == int(acc.sum())


def test_single_gaussian_closed_form():
    H = W = 32
    means = np.array([[0.05, -0.03, 3.0]], np.float32)
    scales = np.full((1, 3), 0.04, np.float32)
    quats = np.array([[0.0, 0.0, 0.0, 1.0]], np.float32)
    opac = np.array([[0.7]], np.float32)
    color = np.array([[0.2, 0.9, 0.4]], np.float32)
    bg = np.array([1.0, 0.5, 0.0], np.float32)
    vm = np.eye(4, dtype=np.float32)
    f, c = (120.0, 120.0), (16.0, 16.0)
    xys, depths, radii, conics, nth, cum = O.project_fwd(means, scales, quats, vm, opac, n=1,
                                                         total=1, img_shape=(H, W), f=f, c=c)
    img, Ts, fidx, stats, M = O.rasterize_fwd(color, opac, opac, bg, xys, depths, radii, conics,
                                              cum, n=1, B=1, img_shape=(H, W))
    jj, ii = np.meshgrid(np.arange(W) + 0.5, np.arange(H) + 0.5)
    dx, dy = xys[0, 0] - jj, xys[0, 1] - ii
    a, b, cc = conics[0].astype(np.float64)
    sigma = 0.5 * (a * dx * dx + cc * dy * dy) + b * dx * dy
    alpha = np.minimum(0.999, 0.7 * np.exp(-sigma))
    alpha = np.where(alpha >= 1 / 255, alpha, 0.0)
    tile_ok = np.zeros((H, W), bool)
    sk, sid, bins = O.sort_and_bin(xys, depths, radii, conics, opac, cum, n=1, B=1,
                                   img_shape=(H, W))
    for tile in np.nonzero(bins[:, 1] > bins[:, 0])[0]:
        ty, tx = divmod(int(tile), 2)
        tile_ok[ty * 16:(ty + 1) * 16, tx * 16:(tx + 1) * 16] = True
    if M == 1:  # the lone-bin behaviour renders nothing
        tile_ok[:] = False
    alpha = np.where(tile_ok, alpha, 0.0)
    ref = bg + alpha[..., None] * (color[0] - bg)
    np.testing.assert_allclose(img.reshape(H, W, 3), ref, atol=2e-6)
    np.testing.assert_allclose(Ts.reshape(H, W), 1.0 - alpha, atol=2e-6)


def test_front_gaussian_occludes():
    """Two coincident-footprint gaussians: the nearer one is blended first."""
    H = W = 16
    means = np.array([[0.0, 0.0, 2.0], [0.0, 0.0, 3.0]], np.float32)
    scales = np.array([[0.3, 0.3, 0.3], [0.45, 0.45, 0.45]], np.float32)
    quats = np.tile(np.array([[0.0, 0.0, 0.0, 1.0]], np.float32), (2, 1))
    opac = np.array([[0.99], [0.99]], np.float32)
    colors = np.array([[1.0, 0.0, 0.0], [0.0, 0.0, 1.0]], np.float32)
    bg = np.zeros(3, np.float32)
    vm = np.eye(4, dtype=np.float32)
    proj = O.project_fwd(means, scales, quats, vm, opac, n=2, total=2, img_shape=(H, W),
                         f=(20.0, 20.0), c=(8.0, 8.0))
    img, Ts, fidx, stats, M = O.rasterize_fwd(colors, opac, opac, bg, *proj[:3], proj[3],
                                              proj[5], n=2, B=1, img_shape=(H, W))
    xys, conics = proj[0].astype(np.float64), proj[3].astype(np.float64)

    def alpha(g, px, py):
        dx, dy = xys[g, 0] - px, xys[g, 1] - py
        a, b, c = conics[g]
        return min(0.999, 0.99 * np.exp(-(0.5 * (a * dx * dx + c * dy * dy) + b * dx * dy)))

    a0, a1 = alpha(0, 8.5, 8.5), alpha(1, 8.5, 8.5)
    expect = np.array([a0, 0.0, (1 - a0) * a1])  # red in front of blue, black background
    np.testing.assert_allclose(img.reshape(H, W, 3)[8, 8], expect, atol=1e-6)
    np.testing.assert_allclose(Ts.reshape(H, W)[8, 8], (1 - a0) * (1 - a1), atol=1e-6)


# ---------------------------------------------------------------- depth channel
# _rasterize_depth_kernel (splax/_rasterize/_kernels.py:277-383): the expected depth uses the
# colour blend's weights and adds no background term.


def test_depth_single_gaussian_equals_z_times_coverage():
    """One gaussian: depth = z * A exactly, A the accumulated alpha (unit colour over black), as
    the reference's tests/test_depth_reg.py:75-107; empty pixels are 0."""
    H = W = 64
    means = np.array([[0.1, -0.05, 0.0]], np.float32)
    scales = np.full((1, 3), 0.12, np.float32)
    quats = np.array([[0.0, 0.0, 0.0, 1.0]], np.float32)
    opac = np.array([[0.9]], np.float32)
    vm = np.array([[1, 0, 0, 0], [0, 1, 0, 0], [0, 0, 1, 4.0], [0, 0, 0, 1]], np.float32)
    f, c = (float(H), float(H)), (W // 2, H // 2)
    xys, depths, radii, conics, nth, cum = O.project_fwd(means, scales, quats, vm, opac, n=1,
                                                         total=1, img_shape=(H, W), f=f, c=c)
    black = np.zeros(3, np.float32)
    A = O.rasterize_fwd(np.ones((1, 3), np.float32), opac, opac, black, xys, depths, radii,
                        conics, cum, n=1, B=1, img_shape=(H, W))[0][..., 0]
    out = O.rasterize_fwd(np.full((1, 3), 0.5, np.float32), opac, opac, black, xys, depths,
                          radii, conics, cum, n=1, B=1, img_shape=(H, W), render_depth=True)
    D = out[5]
    z = np.float32(4.0)
    assert depths[0] == z
    np.testing.assert_array_equal(D, z * A)  # the same weight times z, in float32
    assert D[0, 0] == 0.0 and A[0, 0] == 0.0
    assert D.max() > 0.5 * z


@pytest.mark.parametrize("seed", [0, 1])
def test_depth_path_keeps_image_and_matches_brute_force(seed):
    """The depth path's image is bit-for-bit the plain one (tests/test_depth_reg.py:110-118),
    and its depth equals a float64 brute-force blend of the depths."""
    n, H, W = 300, 48, 64
    sc = random_scene(n, H, W, seed=seed, scale_range=(0.02, 0.1), mean_scale=0.6,
                      opac_range=(0.2, 0.95))
    proj, (img, Ts, fidx, stats, M), (sk, sid, bins) = _pipeline(sc, n)
    xys, depths, radii, conics, nth, cum = proj
    dimg_out = O.rasterize_fwd(sc["colors"], sc["opac"], sc["opac"], sc["bg"], xys, depths, radii,
                               conics, cum, n=n, B=1, img_shape=(H, W), render_depth=True)
    np.testing.assert_array_equal(dimg_out[0], img)
    np.testing.assert_array_equal(dimg_out[1], Ts)
    np.testing.assert_array_equal(dimg_out[2], fidx)
    lay, _ = O.key_layout(1, H, W)
    order = _front_to_back(sk, sid, lay["depth_bits"])
    mem = tile_members(sk, sid, order, img_shape=(H, W), depth_bits=lay["depth_bits"],
                       tile_bits=lay["tile_n_bits"])
    t = lambda a: torch.from_numpy(np.asarray(a, np.float64))  # noqa: E731
    _, _, _, rdep = blend_ref(t(xys), t(conics), t(sc["opac"][:, 0]), t(sc["colors"]),
                              t(sc["bg"]), order, torch.from_numpy(mem), img_shape=(H, W),
                              depths=t(depths).reshape(-1))
    err = np.abs(dimg_out[5].reshape(H, W) - rdep.numpy())
    assert err.max() < 1e-5 * max(1.0, float(np.abs(depths).max())), err.max()
    assert float(np.abs(dimg_out[5]).max()) > 0.0
