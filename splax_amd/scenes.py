"""Synthetic workloads 0-4 of the render-path benchmark (numpy, seeded).

Each config draws from ``numpy.random.Generator(PCG64(seed))`` with ``seed`` = config index, in the
fixed order written in ``_gaussians``. Quaternions are returned wxyz (the public API convention,
splax/_project/_project.py:52), opacities as (N, 1).

Config 2-4 scenes place gaussians on 64 random planes: normal ``n = normalize(N(0, I3))``, offset
``d ~ U[-3, 3]``, point ``d n + u e1 + v e2`` with ``u, v ~ U[-3, 3]`` in the plane basis
``e1 = normalize(n x a)`` (``a`` = x axis, or y axis when ``|n_x| > 0.9``), ``e2 = n x e1``, plus
``N(0, 0.02^2)`` jitter.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from splax_amd.utils import look_at


@dataclass
class Scene:
    name: str
    means: np.ndarray  # (N, 3)
    scales: np.ndarray  # (N, 3)
    quats: np.ndarray  # (N, 4) wxyz
    colors: np.ndarray  # (N, 3)
    opacities: np.ndarray  # (N, 1)
    viewmats: np.ndarray  # (B, 4, 4) world-to-camera
    background: np.ndarray  # (3,)
    img_shape: tuple[int, int]  # (H, W)
    f: tuple[float, float]
    targets: np.ndarray  # (B, H, W, 3)
    antialiased: bool = False
    loss: str = "mse"
    extra: dict = field(default_factory=dict)

    @property
    def n(self) -> int:
        return int(self.means.shape[0])

    @property
    def B(self) -> int:
        return int(self.viewmats.shape[0])

    @property
    def c(self) -> tuple[float, float]:
        H, W = self.img_shape
        return (W / 2, H / 2)


def _sigmoid(x: np.ndarray) -> np.ndarray:
    return 1.0 / (1.0 + np.exp(-x))


def _planes(rng: np.random.Generator, n: int, n_planes: int = 64) -> np.ndarray:
    normals = rng.normal(size=(n_planes, 3))
    normals /= np.linalg.norm(normals, axis=-1, keepdims=True)
    offsets = rng.uniform(-3.0, 3.0, size=n_planes)
    assign = rng.integers(0, n_planes, size=n)
    uv = rng.uniform(-3.0, 3.0, size=(n, 2))
    jitter = rng.normal(0.0, 0.02, size=(n, 3))
    axis = np.where(np.abs(normals[:, :1]) > 0.9, [[0.0, 1.0, 0.0]], [[1.0, 0.0, 0.0]])
    e1 = np.cross(normals, axis)
    e1 /= np.linalg.norm(e1, axis=-1, keepdims=True)
    e2 = np.cross(normals, e1)
    nrm, off = normals[assign], offsets[assign]
    pts = off[:, None] * nrm + uv[:, :1] * e1[assign] + uv[:, 1:] * e2[assign]
    return pts + jitter


def _gaussians(rng, n, *, plane_layout, mean_half_width, log_scale, opac_logit):
    if plane_layout:
        means = _planes(rng, n)
    else:
        means = rng.uniform(-mean_half_width, mean_half_width, size=(n, 3))
    scales = np.exp(rng.normal(log_scale[0], log_scale[1], size=(n, 3)))
    quats = rng.normal(size=(n, 4))
    quats /= np.linalg.norm(quats, axis=-1, keepdims=True)
    colors = rng.uniform(0.0, 1.0, size=(n, 3))
    opac = _sigmoid(rng.normal(opac_logit[0], opac_logit[1], size=(n, 1)))
    f32 = lambda a: np.ascontiguousarray(a, np.float32)  # noqa: E731
    return f32(means), f32(scales), f32(quats), f32(colors), f32(opac)


def _orbit(B: int, radius: float, elevation_deg: float) -> np.ndarray:
    az = 2.0 * np.pi * np.arange(B) / B
    el = np.radians(elevation_deg)
    eyes = radius * np.stack(
        [np.cos(el) * np.cos(az), np.cos(el) * np.sin(az), np.full(B, np.sin(el))], axis=1)
    return look_at(eyes, np.zeros(3), up=(0, 0, 1))


def make_scene(config: int, n: int | None = None) -> Scene:
    """Build synthetic workload ``config`` (0-4); ``n`` overrides the gaussian count."""
    rng = np.random.Generator(np.random.PCG64(config))
    if config == 0:
        n = n or 10_000
        g = _gaussians(rng, n, plane_layout=False, mean_half_width=1.0, log_scale=(-4.0, 0.5),
                       opac_logit=(0.0, 1.0))
        vms = look_at(np.array([[0.0, 0.0, 4.0]]), np.zeros(3))
        H = W = 256
        f = (300.0, 300.0)
        aa, loss = False, "mse"
    elif config == 1:
        n = n or 100_000
        g = _gaussians(rng, n, plane_layout=False, mean_half_width=2.0, log_scale=(-4.0, 0.5),
                       opac_logit=(0.0, 1.0))
        vms = look_at(np.array([[0.0, 0.0, 6.0]]), np.zeros(3))
        H = W = 800
        f = (1100.0, 1100.0)
        aa, loss = False, "mse"
    elif config == 2:
        n = n or 1_000_000
        g = _gaussians(rng, n, plane_layout=True, mean_half_width=3.0, log_scale=(-5.0, 0.7),
                       opac_logit=(1.0, 1.5))
        vms = look_at(np.array([[0.0, 0.0, 8.0]]), np.zeros(3))
        H, W = 1080, 1920
        f = (1500.0, 1500.0)
        aa, loss = False, "mse"
    elif config == 3:
        n = n or 500_000
        g = _gaussians(rng, n, plane_layout=True, mean_half_width=3.0, log_scale=(-5.0, 0.7),
                       opac_logit=(1.0, 1.5))
        vms = _orbit(16, 7.0, 20.0)
        H = W = 512
        f = (600.0, 600.0)
        aa, loss = False, "mse"
    elif config == 4:
        n = n or 3_000_000
        g = _gaussians(rng, n, plane_layout=True, mean_half_width=3.0, log_scale=(-5.0, 0.7),
                       opac_logit=(1.0, 1.5))
        vms = _orbit(4, 7.0, 20.0)
        H, W = 1060, 1600
        f = (1400.0, 1400.0)
        aa, loss = True, "l1"
    else:
        raise ValueError(f"unknown config {config}")
    B = vms.shape[0]
    targets = rng.uniform(0.0, 1.0, size=(B, H, W, 3)).astype(np.float32)
    bg = np.ones(3, np.float32)
    return Scene(f"config{config}", *g, vms, bg, (H, W), f, targets, aa, loss)
