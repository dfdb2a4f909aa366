"""Test configuration: markers, import path, shared scene helpers.

Tests marked ``gpu`` need a ROCm GPU and compare the gfx950 library (through its C ABI) with the
CPU oracle; all other tests run on the CPU and pin the oracle itself.
"""

from __future__ import annotations

import functools
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X); parity vs the oracle")


@pytest.fixture(scope="session", autouse=True)
def _oracle_built():
    from oracle import oracle as O

    if not O.LIB_PATH.exists():
        from oracle.build import build

        build()
    yield


@functools.lru_cache(maxsize=2)
def cached_scene(config: int, n: int | None = None):
    """splax_amd.scenes.make_scene, kept for the session (the config-4 scene takes seconds to
    draw); callers must not modify its arrays."""
    from splax_amd.scenes import make_scene

    return make_scene(config, n=n)


def random_scene(n: int, H: int, W: int, seed: int = 0, scale_range=(0.005, 0.05),
                 mean_scale: float = 1.0, opac_range=(0.0, 1.0)):
    """Random scene in the style of the reference tests (tests/test_warp_rasterize.py:91-104):
    means N(0, 1), scales U[0.005, 0.05], unit quats (wxyz), colors U[0, 1], opacities U[0, 1],
    camera translated by (0.2, -0.1, 5), f = H, c = (W // 2, H // 2)."""
    rng = np.random.default_rng(seed)
    means = (rng.normal(size=(n, 3)) * mean_scale).astype(np.float32)
    scales = rng.uniform(*scale_range, size=(n, 3)).astype(np.float32)
    quats = rng.normal(size=(n, 4))
    quats = (quats / np.linalg.norm(quats, axis=-1, keepdims=True)).astype(np.float32)
    colors = rng.uniform(size=(n, 3)).astype(np.float32)
    opac = rng.uniform(*opac_range, size=(n, 1)).astype(np.float32)
    bg = rng.uniform(size=3).astype(np.float32)
    vm = np.array([[1, 0, 0, 0.2], [0, 1, 0, -0.1], [0, 0, 1, 5], [0, 0, 0, 1]], np.float32)
    cam = {"img_shape": (H, W), "f": (float(H), float(H)), "c": (float(W // 2), float(H // 2))}
    return dict(means=means, scales=scales, quats=quats, colors=colors, opac=opac, bg=bg, vm=vm,
                **cam)


def bits(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a)
    return a.view(np.uint32) if a.dtype == np.float32 else a


def assert_bit_exact(got: np.ndarray, ref: np.ndarray, what: str):
    got, ref = np.asarray(got), np.asarray(ref)
    assert got.shape == ref.shape, f"{what}: shape {got.shape} vs {ref.shape}"
    diff = bits(got) != bits(ref)
    if diff.any():
        idx = np.argwhere(diff)[:5]
        raise AssertionError(
            f"{what}: {int(diff.sum())} of {diff.size} elements differ; first at {idx.tolist()}: "
            f"got {got[tuple(idx[0])]!r} ref {ref[tuple(idx[0])]!r}")


def rel_fro(a: np.ndarray, b: np.ndarray) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / (np.linalg.norm(b) + 1e-30))
