"""Independent float64 restatement of the render path in torch (test infrastructure).

Matrix-form projection (EWA) and a dense brute-force blend, differentiable with autograd. It is
written from the mathematics of the reference (splax/_project/_kernels.py:181-248 for the
projection, splax/_rasterize/_kernels.py:159-198 for the blend) rather than from the oracle's
scalar expressions, so a dropped term, a sign or a transposed operand in the oracle shows up as a
mismatch. Used only by tests.
"""

from __future__ import annotations

import numpy as np
import torch

F64 = torch.float64


def quat_rotation_wxyz(q: torch.Tensor) -> torch.Tensor:
    """Textbook rotation of (un-normalized) wxyz quaternions, (N, 3, 3)."""
    w, x, y, z = q.unbind(-1)
    R = torch.stack([
        1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y),
        2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x),
        2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y),
    ], dim=-1)
    return R.reshape(*q.shape[:-1], 3, 3)


def project_ref(means, scales, quats_wxyz, viewmat, *, f, c, img_shape, glob_scale=1.0,
                clamp=True, tf_R=None, tf_t=None):
    """Returns xys (N,2), depths (N,), conics (N,3), cov2d (N,2,2) in float64.

    tf_R (N,3,3) / tf_t (N,3), when given, move each gaussian rigidly before the camera: the mean
    becomes tf_R mean + tf_t and the covariance factor tf_R R(q) S (splax/_project/_kernels.py:
    627-664)."""
    H, W = img_shape
    Rv = viewmat[:3, :3]
    tv = viewmat[:3, 3]
    R = quat_rotation_wxyz(quats_wxyz)
    M = R * (glob_scale * scales)[:, None, :]
    if tf_R is not None:
        means = (tf_R @ means[..., None])[..., 0] + tf_t
        M = tf_R @ M
    p = means @ Rv.T + tv
    V = M @ M.transpose(-1, -2)
    tz = p[:, 2]
    lim_x = 1.3 * 0.5 * W / f[0]
    lim_y = 1.3 * 0.5 * H / f[1]
    if clamp:
        tx = tz * torch.clamp(p[:, 0] / tz, -lim_x, lim_x)
        ty = tz * torch.clamp(p[:, 1] / tz, -lim_y, lim_y)
    else:
        tx, ty = p[:, 0], p[:, 1]
    zero = torch.zeros_like(tz)
    J = torch.stack([
        torch.stack([f[0] / tz, zero, -f[0] * tx / tz ** 2], -1),
        torch.stack([zero, f[1] / tz, -f[1] * ty / tz ** 2], -1),
    ], dim=-2)  # (N, 2, 3)
    T = J @ Rv
    cov = T @ V @ T.transpose(-1, -2) + 0.3 * torch.eye(2, dtype=F64)
    det = cov[:, 0, 0] * cov[:, 1, 1] - cov[:, 0, 1] ** 2
    conics = torch.stack([cov[:, 1, 1], -cov[:, 0, 1], cov[:, 0, 0]], -1) / det[:, None]
    rw = 1.0 / (tz + 1e-6)
    xys = torch.stack([p[:, 0] * rw * f[0] + c[0], p[:, 1] * rw * f[1] + c[1]], -1)
    return xys, tz, conics, cov


def blend_ref(xys, conics, opac, colors, bg, order, members, *, img_shape, keep=None,
              depths=None):
    """Dense front-to-back blend of the gaussians `order` (front first) into (H, W, 3).

    members[k] is a (H, W) bool mask of the pixels whose tile lists gaussian order[k] (the tile
    assignment, fixed by the sort). keep (optional, (K, H, W) bool) overrides the per-pair
    accept decision (e.g. the oracle's float32 decisions) so gradients follow the same pairs.
    Returns (img, T_final, accepted (K, H, W)); with depths (per gaussian) also the expected
    depth (H, W): depth times the same blend weights, no background term
    (splax/_rasterize/_kernels.py:370-372).
    """
    H, W = img_shape
    jj, ii = torch.meshgrid(torch.arange(W, dtype=F64), torch.arange(H, dtype=F64),
                            indexing="xy")
    px, py = jj + 0.5, ii + 0.5
    T = torch.ones((H, W), dtype=F64)
    out = torch.zeros((H, W, 3), dtype=F64)
    dout = torch.zeros((H, W), dtype=F64)
    done = torch.zeros((H, W), dtype=torch.bool)
    acc = []
    for k, g in enumerate(order):
        dx = xys[g, 0] - px
        dy = xys[g, 1] - py
        a, b, cc = conics[g, 0], conics[g, 1], conics[g, 2]
        sigma = 0.5 * (a * dx * dx + cc * dy * dy) + b * dx * dy
        alpha = torch.minimum(torch.tensor(0.999, dtype=F64), opac[g] * torch.exp(-sigma))
        if keep is None:
            ok = members[k] & ~done & (sigma >= 0) & (alpha >= 1.0 / 255.0)
            nxt = T * (1 - alpha)
            stop = ok & (nxt <= 1e-4)
            done = done | stop
            ok = ok & ~stop
        else:
            ok = keep[k]
        acc.append(ok)
        okf = ok.to(F64)
        out = out + (colors[g] * (alpha * T * okf)[..., None])
        if depths is not None:
            dout = dout + depths[g] * (alpha * T * okf)
        T = T * (1 - alpha * okf)
    img = out + T[..., None] * bg
    accepted = torch.stack(acc) if acc else torch.zeros((0, H, W), dtype=torch.bool)
    if depths is not None:
        return img, T, accepted, dout
    return img, T, accepted


def tile_members(keys: np.ndarray, ids: np.ndarray, order: np.ndarray, *, img_shape,
                 depth_bits: int, tile_bits: int) -> np.ndarray:
    """(K, H, W) masks: pixel tiles that list each gaussian of `order` in the sorted keys."""
    H, W = img_shape
    tx = (W + 15) // 16
    tiles = (keys >> depth_bits) & ((1 << tile_bits) - 1)
    pos = {int(g): k for k, g in enumerate(order)}
    mem = np.zeros((len(order), H, W), bool)
    for t, g in zip(tiles, ids):
        ty_, tx_ = divmod(int(t), tx)
        mem[pos[int(g)], ty_ * 16:(ty_ + 1) * 16, tx_ * 16:(tx_ + 1) * 16] = True
    return mem
