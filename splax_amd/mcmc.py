"""Fixed-budget MCMC relocation on the gfx950 library, mirroring splax/mcmc.py.

``relocate`` teleports dead gaussians (opacity at or below ``min_opacity``) onto alive ones drawn
in proportion to opacity, and corrects opacity and scale so that gaussians sharing a location keep
the source's contribution (the relocation of gsplat's MCMC strategy, splax/mcmc.py:44-131).
``inject_noise`` perturbs the means with noise shaped by each gaussian's covariance and gated by
its opacity (splax/mcmc.py:134-169).

Differences of substance from the reference, all in ``include/splat_hip.h``:
- ``key`` is an integer seed of the library's Philox4x32-10 draw instead of a JAX PRNG key; the
  draw's distribution is the reference's (categorical over log-opacities of the alive gaussians,
  i.e. probability proportional to opacity; standard normals for the noise) and exact, but its
  random stream is the library's.
- ``compute_relocation`` is evaluated in double with exact binomial coefficients, so it agrees
  with gsplat's double loop to float32 rounding; the table argument fixes only its size.
"""

from __future__ import annotations

import math

import torch

from splax_amd import _lib


def make_binoms(n: int, device: torch.device | str | None = None) -> torch.Tensor:
    """Binomial table b[i, k] = C(i, k), zero for k > i (splax/mcmc.py:29-41)."""
    b = [[math.comb(i, k) if k <= i else 0 for k in range(n)] for i in range(n)]
    return torch.tensor(b, dtype=torch.float32, device=device)


def _n_max(binoms: torch.Tensor) -> int:
    if binoms.ndim != 2 or binoms.shape[0] != binoms.shape[1]:
        raise ValueError(f"binoms must be a square make_binoms table, got {tuple(binoms.shape)}")
    return int(binoms.shape[0])


def _f32c(t: torch.Tensor, name: str) -> torch.Tensor:
    if t.dtype != torch.float32:
        raise ValueError(f"{name} must be float32, got {t.dtype}")
    return t.contiguous()


def compute_relocation(opacities: torch.Tensor, scales: torch.Tensor, ratios: torch.Tensor,
                       binoms: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """New (opacities (N,), scales (N, 3)) for relocated multiplicities (splax/mcmc.py:44-71)."""
    opac = _f32c(opacities, "opacities").reshape(-1)
    sc = _f32c(scales, "scales").reshape(-1, 3)
    rat = _f32c(ratios, "ratios").reshape(-1)
    n = opac.numel()
    if sc.shape[0] != n or rat.numel() != n:
        raise ValueError("opacities, scales and ratios must have one row per gaussian")
    dev = _lib.require_gpu(opac, sc, rat)
    new_o = torch.empty_like(opac)
    new_s = torch.empty_like(sc)
    with torch.cuda.device(dev):
        st = _lib.lib().splat_mcmc_compute_relocation(
            _lib.stream_handle(dev), _lib.ptr(opac), _lib.ptr(sc), _lib.ptr(rat), n,
            _n_max(binoms), _lib.ptr(new_o), _lib.ptr(new_s))
    _lib.check(st, "compute_relocation")
    return new_o, new_s


def relocate_(key: int, means3d: torch.Tensor, log_scales: torch.Tensor, quats: torch.Tensor,
              logit_colors: torch.Tensor, logit_opacities: torch.Tensor, binoms: torch.Tensor,
              min_opacity: float = 0.005,
              return_source: bool = False):
    """In-place ``relocate`` on contiguous float32 GPU tensors; returns the reset mask (bool, N)
    and, with ``return_source``, the reference's ``source`` index per row (int32, N)."""
    n = means3d.shape[0]
    arrays = (means3d, log_scales, quats, logit_colors, logit_opacities)
    widths = (3, 3, 4, 3, 1)
    for name, t, w in zip(("means3d", "log_scales", "quats", "logit_colors", "logit_opacities"),
                          arrays, widths):
        if t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous float32 tensor")
        if t.numel() != n * w:
            raise ValueError(f"{name} must have {w} values per gaussian, got shape "
                             f"{tuple(t.shape)} for {n} gaussians")
    dev = _lib.require_gpu(*arrays)
    reset = torch.empty((n,), device=dev, dtype=torch.bool)
    source = torch.empty((n,), device=dev, dtype=torch.int32) if return_source else None
    with torch.cuda.device(dev):
        st = _lib.lib().splat_mcmc_relocate(
            _lib.stream_handle(dev), *(_lib.ptr(t) for t in arrays), n, _n_max(binoms),
            float(min_opacity), int(key) & 0xFFFFFFFFFFFFFFFF, _lib.ptr(source), _lib.ptr(reset))
    _lib.check(st, "relocate")
    return (reset, source) if return_source else reset


def relocate(key: int, means3d: torch.Tensor, log_scales: torch.Tensor, quats: torch.Tensor,
             logit_colors: torch.Tensor, logit_opacities: torch.Tensor, binoms: torch.Tensor,
             min_opacity: float = 0.005):
    """Relocate dead gaussians onto alive ones at a fixed count (splax/mcmc.py:74-131).

    Returns the new (means3d, log_scales, quats, logit_colors, logit_opacities), each of the
    input's shape, and the bool mask of rows whose optimizer moments should be zeroed.
    """
    new = tuple(_f32c(t, "parameter").clone() for t in (means3d, log_scales, quats,
                                                         logit_colors, logit_opacities))
    reset = relocate_(key, *new, binoms, min_opacity)
    return new, reset


def inject_noise(key: int, means3d: torch.Tensor, log_scales: torch.Tensor, quats: torch.Tensor,
                 logit_opacities: torch.Tensor, scaler: float, min_opacity: float = 0.005,
                 noise: torch.Tensor | None = None, *,
                 out: torch.Tensor | None = None) -> torch.Tensor:
    """Means perturbed by covariance- and opacity-weighted noise (splax/mcmc.py:134-169).

    Returns ``means3d + Sigma (z * sigmoid(100 (min_opacity - o)) * scaler)`` of shape (N, 3),
    with ``Sigma = R diag(exp(log_scales))^2 R^T`` (R from the normalized wxyz ``quats``),
    ``o = sigmoid(logit_opacities)`` and ``z`` standard normals: ``noise`` (N, 3) when given,
    else drawn on the device from Philox4x32-10 under ``key`` (the reference draws with
    ``jax.random.normal``; same distribution, another stream). ``out`` (a contiguous float32
    (N, 3) tensor on the means' device, ``means3d`` itself for an in-place update) receives the
    result when given.
    """
    m = _f32c(means3d, "means3d").reshape(-1, 3)
    n = m.shape[0]
    ls = _f32c(log_scales, "log_scales").reshape(-1)
    q = _f32c(quats, "quats").reshape(-1)
    lo = _f32c(logit_opacities, "logit_opacities").reshape(-1)
    if ls.numel() != 3 * n or q.numel() != 4 * n or lo.numel() != n:
        raise ValueError("log_scales, quats and logit_opacities must have 3, 4 and 1 values per "
                         f"gaussian for {n} gaussians")
    if out is not None and (out.dtype != torch.float32 or not out.is_contiguous()
                            or out.numel() != 3 * n or out.device != m.device):
        raise ValueError("out must be a contiguous float32 (N, 3) tensor on the means' device")
    z = None
    if noise is not None:
        z = _f32c(noise, "noise").reshape(-1)
        if z.numel() != 3 * n:
            raise ValueError(f"noise must have shape ({n}, 3), got {tuple(noise.shape)}")
    dev = _lib.require_gpu(m, ls, q, lo, *(() if z is None else (z,)))
    if out is None:
        out = torch.empty_like(m)
    with torch.cuda.device(dev):
        st = _lib.lib().splat_mcmc_inject_noise(
            _lib.stream_handle(dev), _lib.ptr(m), _lib.ptr(ls), _lib.ptr(q), _lib.ptr(lo), n,
            float(scaler), float(min_opacity), int(key) & 0xFFFFFFFFFFFFFFFF,
            _lib.ptr(z), _lib.ptr(out))
    _lib.check(st, "inject_noise")
    return out.reshape(means3d.shape)
