"""Pins the oracle's per-object rigid transforms, forward and VJP (CPU only).

The reference moves each gaussian of a slice by its transform before the camera
(`_apply_transform`, splax/_project/_kernels.py:627-644; the covariance factor is rotated too,
:647-664) and differentiates through it with `_transform_vjp` (:536-557), accumulating the
transform gradient per (image, transform) (:461-484). Here:
- forward: the oracle's projection with transforms equals the plain projection of the moved means
  and rotated covariance factors (float64 torch restatement, tests/torch_ref.py), and ids that are
  negative or at least num_transforms leave a gaussian static;
- VJP: the oracle's v_means / v_scales / v_quats / v_viewmat / v_transforms equal float64
  autograd of that restatement for arbitrary cotangents of xys, depths and conics, with shared
  (K, 4, 4) and per-image (B*K, 4, 4) transforms; a dropped term, a transposed R_tf or a wrong
  sign is O(1) there;
- a directional finite difference of the oracle's own forward along its transform gradient.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import rel_fro
from oracle import oracle as O
from torch_ref import project_ref

F = (120.0, 120.0)
C = (64.0, 56.0)
HW = (112, 128)


def _rot(rng, max_angle):
    axis = rng.normal(size=3)
    axis /= np.linalg.norm(axis)
    ang = rng.uniform(-max_angle, max_angle)
    K = np.array([[0, -axis[2], axis[1]], [axis[2], 0, -axis[0]], [-axis[1], axis[0], 0]])
    return np.eye(3) + np.sin(ang) * K + (1 - np.cos(ang)) * K @ K


def _transforms(rng, count):
    tf = np.zeros((count, 4, 4), np.float32)
    for k in range(count):
        tf[k, :3, :3] = _rot(rng, 0.4)
        tf[k, :3, 3] = rng.uniform(-0.15, 0.15, 3)
        tf[k, 3, 3] = 1.0
    return tf


def _scene(seed, n=150):
    rng = np.random.default_rng(seed)
    means = (rng.normal(size=(n, 3)) * 0.35).astype(np.float32)
    scales = rng.uniform(0.03, 0.1, (n, 3)).astype(np.float32)
    q = rng.normal(size=(n, 4))
    quats = (q / np.linalg.norm(q, axis=-1, keepdims=True)).astype(np.float32)  # wxyz
    opac = rng.uniform(0.2, 0.9, (n, 1)).astype(np.float32)
    return rng, means, scales, quats, opac


def _viewmats(B):
    vms = np.tile(np.eye(4, dtype=np.float32), (B, 1, 1))
    for b in range(B):
        vms[b, :3, 3] = [0.1 * b, -0.05, 5.0 + 0.2 * b]
    return vms


def _ids(n, slices):
    ids = np.full(n, -1, np.int32)
    for k, (a, b) in enumerate(slices):
        ids[a:b] = k
    return ids


def _oracle(means, scales, quats, opac, vms, tf, ids, K, B, n):
    q = np.roll(quats, -1, axis=-1)
    return O.project_fwd(means, scales, q, vms.reshape(-1, 4), opac, n=n, total=B * n,
                         img_shape=HW, f=F, c=C, transforms=tf, transform_ids=ids,
                         num_transforms=K)


def _per_item_tf(tf, ids, K, b, n, batched):
    """(n, 3, 3) rotations and (n, 3) translations of image b (identity where static)."""
    R = torch.eye(3, dtype=torch.float64).repeat(n, 1, 1)
    t = torch.zeros((n, 3), dtype=torch.float64)
    moved = (ids >= 0) & (ids < K)
    sel = torch.from_numpy(np.nonzero(moved)[0])
    rows = torch.from_numpy(ids[moved].astype(np.int64)) + (b * K if batched else 0)
    R = R.index_put((sel,), tf[rows, :3, :3])
    t = t.index_put((sel,), tf[rows, :3, 3])
    return R, t


@pytest.mark.parametrize("B,batched_tf", [(1, False), (2, False), (2, True)])
def test_transform_forward_and_vjp_match_autograd(B, batched_tf):
    n, K = 150, 3
    rng, means, scales, quats, opac = _scene(B + 7 * batched_tf, n)
    slices = [(0, 40), (40, 70), (95, 150)]  # 70..95 static
    ids = _ids(n, slices)
    tf = _transforms(rng, B * K if batched_tf else K)
    vms = _viewmats(B)
    xys, depths, radii, conics, nth, cum = _oracle(means, scales, quats, opac, vms, tf, ids, K,
                                                   B, n)
    vis = radii.reshape(B, n) > 0
    assert vis.sum() > 0.8 * B * n
    w_xy = rng.uniform(-1, 1, (B * n, 2)).astype(np.float32)
    w_d = rng.uniform(-1, 1, (B * n,)).astype(np.float32)
    w_c = rng.uniform(-1, 1, (B * n, 3)).astype(np.float32)
    q = np.roll(quats, -1, axis=-1)
    v_mean, v_scale, v_quat, v_view, v_tf = O.project_bwd(
        means, scales, q, vms.reshape(-1, 4), radii, conics, w_xy, w_d, w_c, n=n, B=B, f=F,
        transforms=tf, transform_ids=ids, num_transforms=K)

    t = lambda a: torch.from_numpy(np.asarray(a, np.float64)).requires_grad_(True)  # noqa: E731
    m_t, s_t, q_t, vm_t, tf_t = t(means), t(scales), t(quats), t(vms), t(tf)
    loss = 0
    for b in range(B):
        R, tr = _per_item_tf(tf_t, ids, K, b, n, batched_tf)
        x, d, cn, _ = project_ref(m_t, s_t, q_t, vm_t[b], f=F, c=C, img_shape=HW, clamp=False,
                                  tf_R=R, tf_t=tr)
        sl = slice(b * n, (b + 1) * n)
        # forward parity (float32 oracle against float64)
        vb = vis[b]
        assert np.abs(x.detach().numpy()[vb] - xys[sl][vb]).max() < 2e-3
        assert np.abs(d.detach().numpy()[vb] - depths[sl][vb]).max() < 1e-4
        assert np.abs(cn.detach().numpy()[vb] - conics[sl][vb]).max() < 2e-3
        mask = torch.from_numpy(vb.astype(np.float64))
        loss = loss + ((torch.from_numpy(w_xy[sl].astype(np.float64)) * x).sum(-1) * mask).sum()
        loss = loss + (torch.from_numpy(w_d[sl].astype(np.float64)) * d * mask).sum()
        loss = loss + ((torch.from_numpy(w_c[sl].astype(np.float64)) * cn).sum(-1) * mask).sum()
    loss.backward()
    sum_b = lambda a, w: a.reshape(B, n, w).sum(0)  # noqa: E731 (shared parameters)
    assert rel_fro(sum_b(v_mean, 3), m_t.grad.numpy()) < 2e-4
    assert rel_fro(sum_b(v_scale, 3), s_t.grad.numpy()) < 2e-4
    assert rel_fro(np.roll(sum_b(v_quat, 4), 1, axis=-1), q_t.grad.numpy()) < 2e-4
    g_view = vm_t.grad.numpy()
    assert rel_fro(v_view.reshape(B, 4, 4)[:, :3], g_view[:, :3]) < 2e-4
    g_tf = tf_t.grad.numpy()
    got_tf = v_tf.reshape(B, K, 4, 4)
    got_tf = got_tf.reshape(B * K, 4, 4) if batched_tf else got_tf.sum(0)
    assert rel_fro(got_tf[:, :3], g_tf[:, :3]) < 2e-4
    assert (got_tf[:, 3] == 0).all()  # the bottom row carries no gradient
    assert np.abs(got_tf[:, :3]).min(axis=(1, 2)).max() > 0


def test_out_of_range_ids_are_static():
    """ids of -1 or >= num_transforms leave the gaussian where it is and add nothing to
    v_transforms (both sides of the C ABI treat them alike)."""
    n, K = 150, 2
    rng, means, scales, quats, opac = _scene(3, n)
    tf = _transforms(rng, K)
    vms = _viewmats(1)
    ids = np.full(n, -1, np.int32)
    ids[:50] = 0
    ids[50:100] = K  # one past the last transform
    ids[100:120] = K + 5
    ref = _oracle(means, scales, quats, opac, vms, None, None, 1, 1, n)
    got = _oracle(means, scales, quats, opac, vms, tf, ids, K, 1, n)
    for a, b in zip(got[:5], ref[:5]):  # cum_tiles_hit also counts the moved items 0..49
        np.testing.assert_array_equal(a[50:], b[50:])
    xys, depths, radii, conics, nth, cum = got
    ones2 = np.ones((n, 2), np.float32)
    q = np.roll(quats, -1, axis=-1)
    out = O.project_bwd(means, scales, q, vms.reshape(-1, 4), radii, conics, ones2,
                        np.ones(n, np.float32), np.ones((n, 3), np.float32), n=n, B=1, f=F,
                        transforms=tf, transform_ids=ids, num_transforms=K)
    ids0 = ids.copy()
    ids0[50:] = -1
    out0 = O.project_bwd(means, scales, q, vms.reshape(-1, 4), radii, conics, ones2,
                         np.ones(n, np.float32), np.ones((n, 3), np.float32), n=n, B=1, f=F,
                         transforms=tf, transform_ids=ids0, num_transforms=K)
    for a, b in zip(out, out0):
        np.testing.assert_array_equal(a, b)
    assert (out[4][1] == 0).all()


def test_transform_gradient_finite_difference():
    """Directional FD of sum(w * outputs) of the oracle's forward along its v_transforms."""
    n, K, B = 150, 3, 1
    rng, means, scales, quats, opac = _scene(11, n)
    ids = _ids(n, [(0, 50), (50, 100), (100, 150)])
    tf = _transforms(rng, K)
    vms = _viewmats(B)
    w_xy = rng.uniform(-1, 1, (n, 2)).astype(np.float32)
    w_c = rng.uniform(-1, 1, (n, 3)).astype(np.float32)
    w_d = rng.uniform(-1, 1, n).astype(np.float32)
    xys, depths, radii, conics, nth, cum = _oracle(means, scales, quats, opac, vms, tf, ids, K,
                                                   B, n)
    vis = radii > 0
    q = np.roll(quats, -1, axis=-1)
    wx, wd, wc = (w_xy * vis[:, None], w_d * vis, w_c * vis[:, None])
    v_tf = O.project_bwd(means, scales, q, vms.reshape(-1, 4), radii, conics, wx, wd, wc, n=n,
                         B=B, f=F, transforms=tf, transform_ids=ids, num_transforms=K)[4]
    direction = v_tf.astype(np.float64)
    direction[:, 3] = 0
    direction /= np.linalg.norm(direction)

    def L(tfx):
        o = _oracle(means, scales, quats, opac, vms, tfx.astype(np.float32), ids, K, B, n)
        return float((wx * o[0]).sum() + (wd * o[1]).sum() + (wc * o[3]).sum())

    eps = 1e-3
    numeric = (L(tf + eps * direction) - L(tf - eps * direction)) / (2 * eps)
    analytic = float((v_tf.astype(np.float64) * direction).sum())
    assert abs(numeric - analytic) / abs(analytic) < 1e-2, (numeric, analytic)
