"""Pins the oracle's projection (splax/_project/_kernels.py:122-248) on the CPU.

Checks: closed forms for gaussians on the optical axis; a float64 torch restatement in matrix form
for random scenes; the culls; radii > 0 <=> num_tiles_hit > 0; cum == cumsum (global over a batch,
tests/test_warp_batch.py:123-126); batch == stack.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import random_scene
from oracle import oracle as O
from torch_ref import project_ref


def _proj(means, scales, quats_wxyz, vm, opac, H, W, f, c, **kw):
    n = means.shape[0]
    q = np.roll(np.asarray(quats_wxyz, np.float32), -1, axis=-1)
    B = vm.size // 16
    return O.project_fwd(means, scales, q, vm, opac, n=n, total=B * n, img_shape=(H, W), f=f,
                         c=c, **kw)


def test_closed_form_on_axis():
    """Isotropic gaussian at (0, 0, z): xy = c, depth = z, conic = 1/(f^2 s^2/z^2 + 0.3) I."""
    H = W = 64
    f = (80.0, 80.0)
    c = (32.0, 32.0)
    zs = np.array([2.0, 3.5, 5.0], np.float32)
    s = np.array([0.05, 0.02, 0.1], np.float32)
    means = np.stack([np.zeros(3), np.zeros(3), zs], -1).astype(np.float32)
    scales = np.repeat(s[:, None], 3, axis=1)
    quats = np.tile(np.array([[1.0, 0, 0, 0]], np.float32), (3, 1))
    opac = np.full((3, 1), 0.9, np.float32)
    vm = np.eye(4, dtype=np.float32)
    xys, depths, radii, conics, nth, cum = _proj(means, scales, quats, vm, opac, H, W, f, c)
    np.testing.assert_allclose(xys, np.tile(c, (3, 1)), atol=1e-4)
    np.testing.assert_allclose(depths, zs, rtol=1e-6)
    expect = 1.0 / (f[0] ** 2 * s.astype(np.float64) ** 2 / zs.astype(np.float64) ** 2 + 0.3)
    np.testing.assert_allclose(conics[:, 0], expect, rtol=2e-6)
    np.testing.assert_allclose(conics[:, 2], expect, rtol=2e-6)
    np.testing.assert_allclose(conics[:, 1], 0.0, atol=1e-9)
    # radius = ceil(sqrt(t) sqrt(cov_xx)), t = min(3.33^2, 2 log(255 o))
    t = min(3.33 ** 2, 2 * np.log(255 * 0.9))
    np.testing.assert_array_equal(radii, np.ceil(np.sqrt(t) * np.sqrt(1.0 / expect)).astype(int))
    assert (nth > 0).all()


def test_closed_form_off_axis_center():
    """Pixel centre uses the unclamped position: xy = f p / (z + 1e-6) + c."""
    means = np.array([[0.3, -0.2, 4.0], [-1.0, 0.5, 6.0]], np.float32)
    scales = np.full((2, 3), 0.05, np.float32)
    quats = np.tile(np.array([[1.0, 0, 0, 0]], np.float32), (2, 1))
    opac = np.full((2, 1), 0.8, np.float32)
    vm = np.eye(4, dtype=np.float32)
    xys, depths, *_ = _proj(means, scales, quats, vm, opac, 128, 96, (100.0, 110.0), (48.0, 64.0))
    z = means[:, 2].astype(np.float64) + 1e-6
    np.testing.assert_allclose(xys[:, 0], 100.0 * means[:, 0] / z + 48.0, rtol=1e-6)
    np.testing.assert_allclose(xys[:, 1], 110.0 * means[:, 1] / z + 64.0, rtol=1e-6)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_matches_float64_matrix_form(seed):
    sc = random_scene(3000, 128, 160, seed=seed)
    H, W = sc["img_shape"]
    xys, depths, radii, conics, nth, cum = _proj(sc["means"], sc["scales"], sc["quats"], sc["vm"],
                                                 sc["opac"], H, W, sc["f"], sc["c"])
    vis = radii > 0
    assert vis.sum() > 500
    t64 = lambda a: torch.from_numpy(np.asarray(a, np.float64))  # noqa: E731
    rx, rd, rc, _ = project_ref(t64(sc["means"]), t64(sc["scales"]), t64(sc["quats"]),
                                t64(sc["vm"]), f=sc["f"], c=sc["c"], img_shape=(H, W))
    np.testing.assert_allclose(xys[vis], rx.numpy()[vis], rtol=1e-5, atol=1e-3)
    np.testing.assert_allclose(depths[vis], rd.numpy()[vis], rtol=1e-6)
    ref_c = rc.numpy()[vis]
    scale = np.abs(ref_c).max(axis=1, keepdims=True)
    np.testing.assert_allclose(conics[vis] / scale, ref_c / scale, atol=2e-4)


def test_culls_and_invariants():
    sc = random_scene(4000, 96, 96, seed=11)
    H, W = sc["img_shape"]
    means = sc["means"].copy()
    means[:10, 2] = -6.0  # behind the camera (z <= clip_thresh)
    opac = sc["opac"].copy()
    opac[10:20] = 1.0 / 256.0  # below the 1/255 alpha floor
    means[20:30, 0] = 50.0  # far off screen
    xys, depths, radii, conics, nth, cum = _proj(means, sc["scales"], sc["quats"], sc["vm"], opac,
                                                 H, W, sc["f"], sc["c"])
    assert (radii[:30] == 0).all() and (nth[:30] == 0).all()
    np.testing.assert_array_equal(radii > 0, nth > 0)
    np.testing.assert_array_equal(cum, np.cumsum(nth))
    culled = radii == 0
    assert (xys[culled] == 0).all() and (conics[culled] == 0).all() and (depths[culled] == 0).all()


def test_batch_equals_stack_with_global_cum():
    sc = random_scene(2000, 64, 80, seed=5)
    H, W = sc["img_shape"]
    vms = np.stack([sc["vm"], sc["vm"] @ np.diag([1.0, 1.0, 1.0, 1.0]).astype(np.float32),
                    sc["vm"].copy()])
    vms[1, 0, 3] += 0.3
    vms[2, 2, 3] += 1.0
    batched = _proj(sc["means"], sc["scales"], sc["quats"], vms.reshape(-1, 4), sc["opac"], H, W,
                    sc["f"], sc["c"])
    singles = [_proj(sc["means"], sc["scales"], sc["quats"], vms[b], sc["opac"], H, W, sc["f"],
                     sc["c"]) for b in range(3)]
    n = 2000
    for k in range(5):
        np.testing.assert_array_equal(batched[k], np.concatenate([s[k] for s in singles]))
    nth_all = np.concatenate([s[4] for s in singles])
    np.testing.assert_array_equal(batched[5], np.cumsum(nth_all))
    assert batched[5].shape == (3 * n,)


def test_rigid_transform_matches_manual():
    """A transform applied in projection equals projecting the moved gaussians
    (tests/test_transforms.py:104-150)."""
    sc = random_scene(500, 64, 64, seed=3)
    H, W = sc["img_shape"]
    ang = 0.3
    Rz = np.array([[np.cos(ang), -np.sin(ang), 0], [np.sin(ang), np.cos(ang), 0], [0, 0, 1]])
    tf = np.eye(4)
    tf[:3, :3] = Rz
    tf[:3, 3] = [0.1, -0.2, 0.05]
    tf = tf.astype(np.float32)[None]
    ids = np.full(500, -1, np.int32)
    ids[100:300] = 0
    got = _proj(sc["means"], sc["scales"], sc["quats"], sc["vm"], sc["opac"], H, W, sc["f"],
                sc["c"], transforms=tf, transform_ids=ids, num_transforms=1)
    moved = sc["means"].copy().astype(np.float64)
    moved[100:300] = moved[100:300] @ Rz.T + tf[0, :3, 3]
    # rotate the moved gaussians' orientation too: q' = q_tf * q
    def qmul(a, b):
        w1, x1, y1, z1 = a
        w2, x2, y2, z2 = b.T
        return np.stack([w1 * w2 - x1 * x2 - y1 * y2 - z1 * z2, w1 * x2 + x1 * w2 + y1 * z2 - z1 * y2,
                         w1 * y2 - x1 * z2 + y1 * w2 + z1 * x2, w1 * z2 + x1 * y2 - y1 * x2 + z1 * w2],
                        -1)
    q_tf = np.array([np.cos(ang / 2), 0, 0, np.sin(ang / 2)])
    quats = sc["quats"].astype(np.float64).copy()
    quats[100:300] = qmul(q_tf, quats[100:300])
    ref = _proj(moved.astype(np.float32), sc["scales"], quats.astype(np.float32), sc["vm"],
                sc["opac"], H, W, sc["f"], sc["c"])
    np.testing.assert_allclose(got[0], ref[0], atol=2e-3)
    np.testing.assert_allclose(got[1], ref[1], rtol=1e-5)
    np.testing.assert_allclose(got[3], ref[3], rtol=2e-3, atol=1e-4)
    same = np.r_[0:100, 300:500]
    for k in range(5):
        np.testing.assert_array_equal(got[k][same], _proj(sc["means"], sc["scales"], sc["quats"],
                                                          sc["vm"], sc["opac"], H, W, sc["f"],
                                                          sc["c"])[k][same])
