"""Pins the float64 truth of the backward (oracle.rasterize_bwd_f64, oracle/truth64.py) on the
CPU.

The truth evaluates the reference's backward formulas (splax/_rasterize/_kernels.py:530-665,
1212-1254; splax/_project/_kernels.py:356-606) in double at the float32 forward's accept
decisions. It is pinned by:
- float64 torch autograd (tests/torch_ref.py, matrix form, written from the mathematics) of the
  brute-force blend fed the float32 forward's positions and conics, and of the projection with
  the unclamped J (the reference's backward is that derivative where no item reaches the
  1.3 tan(fov) clamp): agreement to float64 rounding (projection, given autograd's own conics) or
  to the float32 final transmittance's rounding (blend, which recovers T from final_Ts);
- the float32 oracle within float32 rounding on well-conditioned scenes, with and without the
  clamp, and batched with a per-image viewmat;
- planted mistakes (a dropped depth cotangent, a transposed conic cotangent) that the autograd
  check rejects.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import random_scene, rel_fro
from oracle import oracle as O
from oracle import truth64
from torch_ref import blend_ref, project_ref, tile_members


def _scene(seed, n=150):
    # means near the optical axis so no item reaches the 1.3 tan(fov) clamp
    return random_scene(n, 48, 56, seed=seed, scale_range=(0.03, 0.12), mean_scale=0.4,
                        opac_range=(0.2, 0.9))


def _forward(sc, n):
    H, W = sc["img_shape"]
    q = np.roll(sc["quats"], -1, axis=-1)
    proj = O.project_fwd(sc["means"], sc["scales"], q, sc["vm"], sc["opac"], n=n, total=n,
                         img_shape=(H, W), f=sc["f"], c=sc["c"])
    xys, depths, radii, conics, nth, cum = proj
    img, Ts, fidx, _, _ = O.rasterize_fwd(sc["colors"], sc["opac"], sc["opac"], sc["bg"], xys,
                                          depths, radii, conics, cum, n=n, B=1, img_shape=(H, W))
    return proj, img, Ts, fidx


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_blend_truth_matches_autograd(seed):
    """rasterize_bwd_f64 equals float64 autograd of the brute-force blend over the same tile
    assignment and order, fed the float32 forward's positions and conics (leaf tensors)."""
    n = 150
    sc = _scene(seed, n)
    H, W = sc["img_shape"]
    proj, img, Ts, fidx = _forward(sc, n)
    xys, depths, radii, conics, nth, cum = proj
    w = np.random.default_rng(100 + seed).uniform(-1, 1, (H, W, 3))
    truth = O.rasterize_bwd_f64(sc["colors"], sc["opac"], sc["opac"], sc["bg"], xys, depths,
                                radii, conics, cum, Ts, fidx, w.astype(np.float32), n=n, B_out=1,
                                B_geom=1, img_shape=(H, W))
    sk, sid, _ = O.sort_and_bin(xys, depths, radii, conics, sc["opac"], cum, n=n, B=1,
                                img_shape=(H, W))
    lay, _ = O.key_layout(1, H, W)
    dq = sk & ((1 << lay["depth_bits"]) - 1)
    first = {}
    for d, g in zip(dq, sid):
        first.setdefault(int(g), int(d))
    order = np.array(sorted(first, key=lambda g: (first[g], g)), np.int64)
    mem = torch.from_numpy(tile_members(sk, sid, order, img_shape=(H, W),
                                        depth_bits=lay["depth_bits"],
                                        tile_bits=lay["tile_n_bits"]))
    t = lambda a: torch.from_numpy(np.asarray(a, np.float64)).requires_grad_(True)  # noqa: E731
    x, cn, o, col = t(xys), t(conics), t(sc["opac"][:, 0]), t(sc["colors"])
    timg, _, _ = blend_ref(x, cn, o, col, torch.from_numpy(sc["bg"].astype(np.float64)), order,
                           mem, img_shape=(H, W))
    assert np.abs(timg.detach().numpy() - img.reshape(H, W, 3)).max() < 1e-5
    (torch.from_numpy(w) * timg).sum().backward()
    vis = radii > 0
    assert vis.sum() > 50
    for k, got, ref in (("colors", truth[0], col.grad), ("opac", truth[1], o.grad),
                        ("xy", truth[2][vis], x.grad[vis]), ("conic", truth[3][vis], cn.grad[vis])):
        r = rel_fro(got, ref.numpy())
        # the truth recovers T from the float32 final transmittance (6e-8 relative)
        assert r < 2e-6, f"{k}: relative Frobenius error {r:.2e} against autograd"
    # the float32 oracle is within float32 rounding of the truth
    f32 = O.rasterize_bwd(sc["colors"], sc["opac"], sc["opac"], sc["bg"], xys, depths, radii,
                          conics, cum, Ts, fidx, w.astype(np.float32), n=n, B_out=1, B_geom=1,
                          img_shape=(H, W))
    for k, a, b in zip(("colors", "opac", "xy", "conic"), f32[:4], truth[:4]):
        r = rel_fro(a.reshape(b.shape), b)
        assert r < 1e-5, f"{k}: float32 oracle vs truth {r:.2e}"


def _projection_autograd(sc, n, v_xy, v_depth, v_conic):
    """float64 autograd of the unclamped projection (tests/torch_ref.py) for the given output
    cotangents; returns its conics too."""
    H, W = sc["img_shape"]
    t = lambda a: torch.from_numpy(np.asarray(a, np.float64)).requires_grad_(True)  # noqa: E731
    means, scales, quats, vm = t(sc["means"]), t(sc["scales"]), t(sc["quats"]), t(sc["vm"])
    xys, depths, conics, _ = project_ref(means, scales, quats, vm, f=sc["f"], c=sc["c"],
                                         img_shape=(H, W), clamp=False)
    loss = ((xys * torch.from_numpy(v_xy)).sum() + (depths * torch.from_numpy(v_depth)).sum()
            + (conics * torch.from_numpy(v_conic)).sum())
    loss.backward()
    return (means.grad.numpy(), scales.grad.numpy(), np.roll(quats.grad.numpy(), -1, axis=-1),
            vm.grad.numpy(), conics.detach().numpy())


@pytest.mark.parametrize("seed", [0, 3])
def test_projection_truth_matches_autograd(seed):
    """project_bwd_f64 equals float64 autograd of the unclamped projection to float64 rounding
    when given autograd's own conics; a dropped depth cotangent or a transposed conic cotangent
    is rejected."""
    n = 400
    sc = dict(_scene(seed, n))
    # exactly unit quaternions (float64): warp's rotation form and the textbook one then agree
    q64 = sc["quats"].astype(np.float64)
    sc["quats"] = q64 / np.linalg.norm(q64, axis=-1, keepdims=True)
    rng = np.random.default_rng(seed)
    v_xy, v_depth, v_conic = rng.normal(size=(n, 2)), rng.normal(size=n), rng.normal(size=(n, 3))
    gm, gs, gq, gv, conics64 = _projection_autograd(sc, n, v_xy, v_depth, v_conic)
    q = np.roll(sc["quats"], -1, axis=-1)
    radii = np.ones(n, np.int32)
    tm, ts, tq, tv = truth64.project_bwd_f64(sc["means"], sc["scales"], q, sc["vm"], radii,
                                             conics64, v_xy, v_depth, v_conic, n=n, B=1,
                                             f=sc["f"])
    for k, a, b in (("means", tm, gm), ("scales", ts, gs), ("quats", tq, gq),
                    ("viewmat", tv[0], gv)):
        r = rel_fro(a, b)
        assert r < 1e-11, f"{k}: relative Frobenius error {r:.2e} against autograd"
    # planted mistakes
    bad = truth64.project_bwd_f64(sc["means"], sc["scales"], q, sc["vm"], radii, conics64, v_xy,
                                  np.zeros(n), v_conic, n=n, B=1, f=sc["f"])
    assert rel_fro(bad[0], gm) > 1e-3
    bad = truth64.project_bwd_f64(sc["means"], sc["scales"], q, sc["vm"], radii, conics64, v_xy,
                                  v_depth, v_conic[:, ::-1].copy(), n=n, B=1, f=sc["f"])
    assert rel_fro(bad[1], gs) > 1e-3


@pytest.mark.parametrize("B", [1, 3])
def test_projection_truth_matches_float32_oracle(B):
    """On a scene whose outer items reach the frustum clamp, batched over B viewmats: the truth
    within float32 rounding of the float32 oracle (per item and per image), zero rows for
    culled items."""
    n = 2000
    sc = random_scene(n, 64, 80, seed=21 + B, mean_scale=2.5)  # items past the clamp
    H, W = sc["img_shape"]
    vms = np.stack([sc["vm"]] * B)
    for b in range(1, B):
        vms[b, 0, 3] += 0.2 * b
    q = np.roll(sc["quats"], -1, axis=-1)
    xys, depths, radii, conics, nth, cum = O.project_fwd(
        sc["means"], sc["scales"], q, vms.reshape(-1, 4), sc["opac"], n=n, total=B * n,
        img_shape=(H, W), f=sc["f"], c=sc["c"])
    p = (np.einsum("ij,nj->ni", sc["vm"][:3, :3].astype(np.float64), sc["means"])
         + sc["vm"][:3, 3])
    lim = 1.3 * 0.5 * W / sc["f"][0]
    assert (np.abs(p[:, 0] / p[:, 2]) > lim).sum() > 20  # some items reach the clamp
    rng = np.random.default_rng(B)
    v_xy = rng.normal(size=(B * n, 2)).astype(np.float32)
    v_depth = rng.normal(size=B * n).astype(np.float32)
    v_conic = rng.normal(size=(B * n, 3)).astype(np.float32)
    f32 = O.project_bwd(sc["means"], sc["scales"], q, vms.reshape(-1, 4), radii, conics, v_xy,
                        v_depth, v_conic, n=n, B=B, f=sc["f"])
    tr = truth64.project_bwd_f64(sc["means"], sc["scales"], q, vms, radii, conics, v_xy,
                                 v_depth, v_conic, n=n, B=B, f=sc["f"])
    ca, cb, cc = (conics[:, k].astype(np.float64) for k in range(3))
    cond = (ca + cc) ** 2 / np.maximum(ca * cc - cb * cb, 1e-300)
    well = (radii.ravel() > 0) & (cond < 1e2)
    assert well.sum() > 500
    for k, a, b in (("means", f32[0], tr[0]), ("scales", f32[1], tr[1]),
                    ("quats", f32[2], tr[2])):
        r = rel_fro(a[well], b[well])
        assert r < 1e-5, f"{k}: float32 oracle vs truth {r:.2e}"
        assert (b[radii.ravel() <= 0] == 0).all()
    r = rel_fro(f32[3].reshape(B, 4, 4), tr[3])
    assert r < 1e-5, f"viewmat: {r:.2e}"


def test_compensation_truth_matches_float32():
    """compensation_vjp_f64 within float32 rounding of the oracle's float32 compensation_vjp
    inside (0, 1), with the same boundary conventions (NaN where rho = 0)."""
    rng = np.random.default_rng(4)
    conics = np.abs(rng.normal(size=(3000, 3))).astype(np.float32)
    conics[:, 1] *= 0.1
    opac = rng.uniform(0.1, 1.0, 3000).astype(np.float32)
    vbo = rng.normal(size=3000).astype(np.float32)
    o32, c32 = O.compensation_vjp(vbo, opac, conics)
    o64, c64 = truth64.compensation_vjp_f64(vbo, opac, conics)
    fin = np.isfinite(c32).all(1)
    np.testing.assert_array_equal(np.isfinite(c64).all(1), fin)
    assert fin.sum() > 1000
    assert rel_fro(o32, o64) < 1e-6
    assert rel_fro(c32[fin], c64[fin]) < 1e-5
