"""float64 truth of the render path's backward (test infrastructure only).

The float32 oracle and the GPU library evaluate the reference's backward formulas in float32, so
both round; on ill-conditioned items (needle-thin conics) the projection VJP amplifies that
rounding. To measure either against the same exact-as-possible value, this module restates the
projection VJP of the reference in float64, vectorized over items:
``_project_bwd_kernel`` with ``_proj_vjp``, ``_scale_vjp``, ``_quat_vjp`` and ``_view_vjp``
(splax/_project/_kernels.py:356-484,487-533,560-606), J from the unclamped camera-space position
(:428-432), v_cov2d = -X G X with the stored conic X (:434-439). Its blend counterpart is
``oracle.rasterize_bwd_f64`` (the oracle's walk evaluated in double). Rigid transforms are not
covered (the tests that use this module have none).

Only ``tests/`` imports this module.
"""

from __future__ import annotations

import numpy as np

F64 = np.float64


def quat_to_rot_xyzw(q: np.ndarray) -> np.ndarray:
    """warp-lang's quat_to_matrix for q = (x, y, z, w), any norm:
    R = (2 w^2 - 1) I + 2 v v^T + 2 w [v]_x, (G, 3, 3)."""
    x, y, z, w = (q[:, k] for k in range(4))
    c = 2.0 * w * w - 1.0
    R = np.empty((q.shape[0], 3, 3), F64)
    R[:, 0, 0] = c + 2 * x * x
    R[:, 0, 1] = 2 * x * y - 2 * z * w
    R[:, 0, 2] = 2 * x * z + 2 * y * w
    R[:, 1, 0] = 2 * y * x + 2 * z * w
    R[:, 1, 1] = c + 2 * y * y
    R[:, 1, 2] = 2 * y * z - 2 * x * w
    R[:, 2, 0] = 2 * z * x - 2 * y * w
    R[:, 2, 1] = 2 * z * y + 2 * x * w
    R[:, 2, 2] = c + 2 * z * z
    return R


def _rows_for(a: np.ndarray, width: int, n: int, total: int) -> np.ndarray:
    """(total, width) float64 rows: a shared (n rows) operand repeated per image."""
    a = np.asarray(a, F64).reshape(-1, width)
    if a.shape[0] == total:
        return a
    assert a.shape[0] == n, (a.shape, n, total)
    return np.tile(a, (total // n, 1))


def project_bwd_f64(means, scales, quats_xyzw, viewmat, radii, conics, v_xy, v_depth, v_conic,
                    *, n, B, f, glob_scale=1.0):
    """Returns float64 (v_mean3d, v_scale, v_quat (xyzw), v_viewmat (B, 4, 4)) for B images of n
    items, with the operands' shared-or-batched rows rule (rows == n: shared)."""
    total = B * n
    mean = _rows_for(means, 3, n, total)
    sc = _rows_for(scales, 3, n, total)
    q = _rows_for(quats_xyzw, 4, n, total)
    vm = np.asarray(viewmat, F64).reshape(-1, 4, 4)
    vm = np.repeat(vm, n, axis=0) if vm.shape[0] == B else np.broadcast_to(vm, (total, 4, 4))
    cn = _rows_for(conics, 3, n, total)
    vxy = _rows_for(v_xy, 2, n, total)
    vd = _rows_for(v_depth, 1, n, total)[:, 0]
    vc = _rows_for(v_conic, 3, n, total)
    vis = np.asarray(radii).reshape(-1) > 0
    if vis.size == n and total != n:
        vis = np.tile(vis, B)
    fx, fy = float(f[0]), float(f[1])

    W = vm[:, :3, :3]
    t = vm[:, :3, 3]
    p = np.einsum("gij,gj->gi", W, mean) + t
    R = quat_to_rot_xyzw(q)
    s = glob_scale * sc
    M = R * s[:, None, :]
    V = M @ np.swapaxes(M, 1, 2)
    x, y, z = p[:, 0], p[:, 1], p[:, 2]
    with np.errstate(divide="ignore", invalid="ignore"):
        rz = 1.0 / z
        rz2 = rz * rz
        j00, j02 = fx * rz, -fx * x * rz2
        j11, j12 = fy * rz, -fy * y * rz2
        T0 = j00[:, None] * W[:, 0] + j02[:, None] * W[:, 2]
        T1 = j11[:, None] * W[:, 1] + j12[:, None] * W[:, 2]
        # v_cov2d = -X G X, G the conic cotangent as a symmetric matrix (off-diagonal halved)
        X = np.stack([np.stack([cn[:, 0], cn[:, 1]], -1), np.stack([cn[:, 1], cn[:, 2]], -1)], 1)
        G = np.stack([np.stack([vc[:, 0], 0.5 * vc[:, 1]], -1),
                      np.stack([0.5 * vc[:, 1], vc[:, 2]], -1)], 1)
        S = X @ G @ X
        c0, c1, c2 = -S[:, 0, 0], 0.5 * -(S[:, 0, 1] + S[:, 1, 0]), -S[:, 1, 1]
        # _proj_vjp: the image-plane position, the 2D covariance through T = J W
        rw = 1.0 / (z + 1e-6)
        vpx, vpy = fx * vxy[:, 0], fy * vxy[:, 1]
        vvx, vvy = vpx * rw, vpy * rw
        vvz = -(vpx * x + vpy * y) * rw * rw + vd
        T = np.stack([T0, T1], 1)  # (G, 2, 3)
        C = np.stack([np.stack([c0, c1], -1), np.stack([c1, c2], -1)], 1)  # (G, 2, 2)
        v_V = np.swapaxes(T, 1, 2) @ C @ T  # (G, 3, 3)
        v_T = 2.0 * C @ T @ V  # (G, 2, 3)
        v_J = v_T @ np.swapaxes(W, 1, 2)  # (G, 2, 3)
        rz3 = rz2 * rz
        v_tx = -fx * rz2 * v_J[:, 0, 2]
        v_ty = -fy * rz2 * v_J[:, 1, 2]
        v_tz = (-fx * rz2 * v_J[:, 0, 0] + 2.0 * fx * x * rz3 * v_J[:, 0, 2]
                - fy * rz2 * v_J[:, 1, 1] + 2.0 * fy * y * rz3 * v_J[:, 1, 2])
        v_p = np.stack([vvx + v_tx, vvy + v_ty, vvz + v_tz], -1)
        v_mean = np.einsum("gji,gj->gi", W, v_p)
        v_M = (v_V + np.swapaxes(v_V, 1, 2)) @ M
        v_scale = (R * v_M).sum(axis=1) * glob_scale
        vR = v_M * s[:, None, :]
        qx, qy, qz, qw = (q[:, k] for k in range(4))
        v_qw = 2.0 * (qx * (vR[:, 2, 1] - vR[:, 1, 2]) + qy * (vR[:, 0, 2] - vR[:, 2, 0])
                      + qz * (vR[:, 1, 0] - vR[:, 0, 1]))
        v_qx = 2.0 * (-2.0 * qx * (vR[:, 1, 1] + vR[:, 2, 2]) + qy * (vR[:, 1, 0] + vR[:, 0, 1])
                      + qz * (vR[:, 2, 0] + vR[:, 0, 2]) + qw * (vR[:, 2, 1] - vR[:, 1, 2]))
        v_qy = 2.0 * (qx * (vR[:, 1, 0] + vR[:, 0, 1]) - 2.0 * qy * (vR[:, 0, 0] + vR[:, 2, 2])
                      + qz * (vR[:, 2, 1] + vR[:, 1, 2]) + qw * (vR[:, 0, 2] - vR[:, 2, 0]))
        v_qz = 2.0 * (qx * (vR[:, 2, 0] + vR[:, 0, 2]) + qy * (vR[:, 2, 1] + vR[:, 1, 2])
                      - 2.0 * qz * (vR[:, 0, 0] + vR[:, 1, 1]) + qw * (vR[:, 1, 0] - vR[:, 0, 1]))
        v_quat = np.stack([v_qx, v_qy, v_qz, v_qw], -1)
        # _view_vjp: v_R = v_p (x) mean + J^T v_T, v_t = v_p, summed per image
        J = np.zeros((total, 2, 3), F64)
        J[:, 0, 0], J[:, 0, 2], J[:, 1, 1], J[:, 1, 2] = j00, j02, j11, j12
        v_R = v_p[:, :, None] * mean[:, None, :] + np.swapaxes(J, 1, 2) @ v_T
    zero = ~vis
    for a in (v_mean, v_scale, v_quat, v_p, v_R):
        a[zero] = 0.0
    v_view = np.zeros((B, 4, 4), F64)
    v_view[:, :3, :3] = v_R.reshape(B, n, 3, 3).sum(1)
    v_view[:, :3, 3] = v_p.reshape(B, n, 3).sum(1)
    return v_mean, v_scale, v_quat, v_view


def compensation_vjp_f64(v_blend_opac, opac, conics):
    """compensation_vjp (oracle.oracle) in float64: cotangents of opac * rho(conic),
    rho = sqrt(clip(1 - eps (a + c) + eps^2 (a c - b^2), 0, 1)), eps = 0.3
    (splax/_project/_project.py:95-117), by the reference's reverse-mode rules; returns
    (v_opac, v_conics)."""
    vbo = np.asarray(v_blend_opac, F64).reshape(-1)
    o = np.asarray(opac, F64).reshape(-1)
    cn = np.asarray(conics, F64).reshape(-1, 3)
    a, b, c = cn[:, 0], cn[:, 1], cn[:, 2]
    eps = float(np.float32(0.3))
    eps2 = float(np.float32(0.3 * 0.3))
    with np.errstate(divide="ignore", invalid="ignore"):
        rho2 = (1.0 - eps * (a + c)) + eps2 * (a * c - b * b)
        rho = np.sqrt(np.clip(rho2, 0.0, 1.0))
        v_o = vbo * rho
        v_cl = vbo * o * (0.5 / rho)
        m_lo = np.where(rho2 > 0, 1.0, np.where(rho2 == 0, 0.5, 0.0))
        y = np.where(rho2 > 0, rho2, 0.0)
        m_hi = np.where(y < 1, 1.0, np.where(y == 1, 0.5, 0.0))
        v_r2 = v_cl * m_hi * m_lo
        vc = np.stack([-eps * v_r2 + eps2 * v_r2 * c, -2.0 * eps2 * v_r2 * b,
                       -eps * v_r2 + eps2 * v_r2 * a], axis=1)
    return v_o, vc
