"""Pins the oracle's fixed-sequence exp / log and the packed-key layout (CPU only).

exp and log must be accurate to a couple of ulp (they replace the reference's fast-math
wp.exp / wp.log, splax/_rasterize/_kernels.py:188 and splax/_project/_kernels.py:227); the
float64 numpy functions are the truth. The key layout is checked against the closed form of
splax/_rasterize/_sort/_sort.py:56-60 and the per-config table derived independently by hand.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as O


def _ulp_err(got: np.ndarray, truth64: np.ndarray) -> np.ndarray:
    got = got.astype(np.float64)
    ulp = np.spacing(np.abs(truth64).astype(np.float32)).astype(np.float64)
    return np.abs(got - truth64) / ulp


def test_logf_accuracy_sweep():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        np.float32(1.0) + np.arange(-2000, 2000, dtype=np.float32) * np.float32(2.0 ** -23),
        rng.uniform(1.0, 255.0, 200_000).astype(np.float32),  # opac / (1/255) in projection
        np.exp(rng.uniform(-80, 80, 200_000)).astype(np.float32),
        np.array([1e-40, 1e-45, 3e-39, 1.17549435e-38, 2.0, 0.5, 255.0], np.float32),
    ])
    x = x[x > 0]
    got = O.logf(x)
    truth = np.log(x.astype(np.float64))
    err = _ulp_err(got, truth)
    nonzero = truth != 0
    assert err[nonzero].max() <= 2.0, f"max ulp error {err[nonzero].max()}"
    assert O.logf(np.float32(1.0))[0] == 0.0


def test_expf_accuracy_sweep():
    rng = np.random.default_rng(1)
    x = np.concatenate([
        rng.uniform(-87.0, 88.0, 400_000),
        rng.uniform(-6.0, 0.0, 400_000),  # the blend's range after the alpha cull
        np.arange(-2000, 2000) * 2.0 ** -20,
    ]).astype(np.float32)
    got = O.expf(x)
    truth = np.exp(x.astype(np.float64))
    err = _ulp_err(got, truth)
    assert err.max() <= 2.0, f"max ulp error {err.max()} at {x[np.argmax(err)]}"
    assert O.expf(np.float32(0.0))[0] == 1.0
    assert O.expf(np.float32(-0.0))[0] == 1.0


def test_expf_special_values():
    got = O.expf(np.array([np.nan, -1e9, -105.0, 100.0], np.float32))
    assert got[0] == 0.0 and got[1] == 0.0 and got[2] == 0.0
    assert np.isinf(got[3])
    sub = O.expf(np.array([-100.0], np.float32))[0]
    assert 0.0 < sub < 1e-40  # subnormal range is reached, never used for a blend decision


def test_expf_monotone_on_blend_range():
    x = np.sort(np.random.default_rng(2).uniform(-8.0, 0.0, 200_000).astype(np.float32))
    y = O.expf(x)
    assert np.all(np.diff(y.astype(np.float64)) >= 0.0)


def test_blend_expf_accuracy_sweep():
    """The blends' exp(-sigma) sequence against float64 exp: random points over its whole normal
    domain plus every 64th float of [-8, 0] (where the blends' x lives)."""
    rng = np.random.default_rng(5)
    dense = (np.arange(np.float32(-8.0).view(np.uint32), np.uint32(0x80000000) - 1, -64,
                       dtype=np.int64).astype(np.uint32).view(np.float32))
    # one float ln2 in the reduction: the error k (ln2 - fl(ln2)) grows with |k|, so the bound
    # widens with the range (opacity <= 1 keeps the blends inside [-5.6, 0])
    for lo, hi, bound, extra in ((-8.0, 0.0, 1.0, dense), (-30.0, -8.0, 2.0, None),
                                 (-87.0, -30.0, 5.0, None)):
        x = rng.uniform(lo, hi, 400_000).astype(np.float32)
        if extra is not None:
            x = np.concatenate([x, extra])
        err = _ulp_err(O.blend_expf(x), np.exp(x.astype(np.float64)))
        assert err.max() <= bound, f"[{lo}, {hi}]: max ulp error {err.max()} at {x[np.argmax(err)]}"
    assert O.blend_expf(np.float32(0.0))[0] == 1.0
    assert O.blend_expf(np.float32(-0.0))[0] == 1.0
    # where x = -m fl(ln2) is exact in float32 (fl(ln2) has 20 significant bits), the reduction
    # leaves r = 0 and the result is exactly 2^-m
    m = np.arange(0, 40)
    x64 = -m * np.float64(np.float32(np.log(2.0)))
    exact = x64.astype(np.float32).astype(np.float64) == x64
    assert exact.sum() >= 20
    y = O.blend_expf(x64[exact].astype(np.float32)).astype(np.float64)
    assert np.all(y == 2.0 ** -m[exact])


def test_blend_expf_monotone_and_below_range():
    x = np.sort(np.random.default_rng(6).uniform(-8.0, 0.0, 400_000).astype(np.float32))
    assert np.all(np.diff(O.blend_expf(x).astype(np.float64)) >= 0.0)
    # under 2^-126 the value is no exponential any more but tiny, negative or NaN, never a large
    # positive one, so the blends' alpha test (alpha >= 1/255, false for NaN) rejects it as it
    # would the exact value
    low = np.linspace(-95.0, -87.4, 20_000).astype(np.float32)
    assert not np.any(O.blend_expf(low) >= 2.0 ** -125)


@pytest.mark.parametrize(
    "B,H,W,tile_bits,image_bits,depth_bits,packed",
    [
        (1, 256, 256, 8, 0, 23, True),  # config 0: 16x16 tiles
        (1, 800, 800, 12, 0, 19, True),  # config 1: 50x50
        (1, 1080, 1920, 13, 0, 18, True),  # config 2: 120x68
        (16, 512, 512, 10, 4, 17, True),  # config 3: 32x32, 16 cameras
        (4, 1060, 1600, 13, 2, 16, True),  # config 4: 100x67, boundary case
        (8, 1080, 1920, 13, 3, 15, False),  # B=8 at 1080p needs the 64-bit key
        (1, 16, 16, 0, 0, 31, True),  # one tile
    ],
)
def test_key_layout_table(B, H, W, tile_bits, image_bits, depth_bits, packed):
    lay, ok = O.key_layout(B, H, W)
    assert lay["tile_n_bits"] == tile_bits
    assert lay["image_n_bits"] == image_bits
    assert lay["depth_bits"] == depth_bits
    assert ok == packed
    nt = lay["num_tiles"]
    assert nt == ((W + 15) // 16) * ((H + 15) // 16)
    assert (nt - 1) < (1 << tile_bits) and (B - 1) < (1 << image_bits)


def test_compensation_rho_closed_form_and_vjp():
    """rho^2 = det(S) / det(S + 0.3 I) for the conic of S + 0.3 I (the projection's dilation,
    splax/_project/_kernels.py:204-212); the cotangent rule equals float64 autograd of the
    reference expression away from the clip boundaries, and follows the reference's conventions
    on them (1/2 at a tie, NaN where rho = 0 and the cotangent is 0)."""
    import torch

    rng = np.random.default_rng(8)
    n = 500
    L = rng.normal(size=(n, 2, 2)) * rng.uniform(0.1, 3.0, (n, 1, 1))
    S = L @ np.transpose(L, (0, 2, 1))
    Sd = S + 0.3 * np.eye(2)
    det = Sd[:, 0, 0] * Sd[:, 1, 1] - Sd[:, 0, 1] ** 2
    conics = np.stack([Sd[:, 1, 1] / det, -Sd[:, 0, 1] / det, Sd[:, 0, 0] / det], 1)
    conics = conics.astype(np.float32)
    rho, rho2 = O.compensation_rho(conics)
    want = (S[:, 0, 0] * S[:, 1, 1] - S[:, 0, 1] ** 2) / det
    np.testing.assert_allclose(rho2, want, atol=2e-6)
    np.testing.assert_allclose(rho, np.sqrt(np.clip(want, 0, 1)), atol=2e-3)
    # cotangents against float64 autograd of the same expression (interior points)
    vbo = rng.normal(size=n).astype(np.float32)
    opac = rng.uniform(0.05, 1.0, n).astype(np.float32)
    v_o, v_c = O.compensation_vjp(vbo, opac, conics)
    c64 = torch.tensor(conics, dtype=torch.float64, requires_grad=True)
    o64 = torch.tensor(opac, dtype=torch.float64, requires_grad=True)
    a, b, c = c64[:, 0], c64[:, 1], c64[:, 2]
    r2 = 1.0 - 0.3 * (a + c) + 0.09 * (a * c - b * b)
    bo = o64 * torch.sqrt(torch.clamp(r2, 0.0, 1.0))
    bo.backward(torch.tensor(vbo, dtype=torch.float64))
    # float32 rho2 cancels: its absolute error is ~1e-7 of the terms, so compare where rho2 is
    # well inside (0, 1)
    inside = (rho2 > 0.05) & (rho2 < 1 - 1e-6)
    assert inside.sum() > 300
    np.testing.assert_allclose(v_o[inside], o64.grad.numpy()[inside], rtol=1e-4, atol=1e-7)
    np.testing.assert_allclose(v_c[inside], c64.grad.numpy()[inside], rtol=1e-3, atol=1e-6)
    # boundaries: zero conic (culled item) -> rho 1, a tie of the upper clip -> half gradient
    v_o0, v_c0 = O.compensation_vjp([2.0], [0.5], [[0.0, 0.0, 0.0]])
    assert v_o0[0] == 2.0
    np.testing.assert_array_equal(v_c0[0], np.float32([-0.3, 0.0, -0.3]) * np.float32(0.25))
    # rho = 0 with a zero cotangent: NaN, as the reference's sqrt rule gives
    v_o1, v_c1 = O.compensation_vjp([0.0], [0.5], [[4.0, 0.0, 1.0]])
    assert O.compensation_rho([[4.0, 0.0, 1.0]])[0][0] == 0.0  # rho2 = (1 - 1.2)(1 - 0.3) < 0
    assert np.isnan(v_c1).all() and v_o1[0] == 0.0
