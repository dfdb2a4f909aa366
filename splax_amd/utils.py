"""Camera helpers (numpy).

``look_at`` and ``nerf_camera`` restate splax/utils.py:9-45. The reference inverts the
camera-to-world matrix with scipy's ``RigidTransform``; the inverse of a rigid transform
``[R t; 0 1]`` is ``[R^T -R^T t; 0 1]``, which is what is computed here.
"""

from __future__ import annotations

import numpy as np


def _rigid_inverse(c2w: np.ndarray) -> np.ndarray:
    R = c2w[..., :3, :3]
    t = c2w[..., :3, 3]
    out = np.zeros_like(c2w)
    Rt = np.swapaxes(R, -1, -2)
    out[..., :3, :3] = Rt
    out[..., :3, 3] = -np.einsum("...ij,...j->...i", Rt, t)
    out[..., 3, 3] = 1.0
    return out


def look_at(eye: np.ndarray, target: np.ndarray, up=(0, 1, 0)) -> np.ndarray:
    """World-to-camera OpenCV matrices looking from ``eye`` to ``target`` (splax/utils.py:9-30).

    x = right, y = down, z = forward; returns (..., 4, 4) float32.
    """
    eye = np.asarray(eye, np.float64)
    target = np.asarray(target, np.float64)
    z = target - eye
    norm = np.linalg.norm(z, axis=-1, keepdims=True)
    if not (norm > 0).all():
        raise ValueError("eye and target must differ")
    z = z / norm
    x = np.cross(z, np.asarray(up, np.float64))
    x = x / np.linalg.norm(x, axis=-1, keepdims=True)
    c2w = np.zeros((*z.shape[:-1], 4, 4))
    c2w[..., :3, :3] = np.stack([x, np.cross(z, x), z], axis=-1)
    c2w[..., :3, 3] = eye
    c2w[..., 3, 3] = 1.0
    return _rigid_inverse(c2w).astype(np.float32)


def nerf_camera(c2w) -> np.ndarray:
    """Blender camera-to-world to OpenCV world-to-camera (splax/utils.py:33-45)."""
    c2w = np.asarray(c2w, np.float64) @ np.diag([1.0, -1.0, -1.0, 1.0])
    return _rigid_inverse(c2w).astype(np.float32)
