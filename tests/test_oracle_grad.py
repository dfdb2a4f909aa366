"""Pins the oracle's VJPs against float64 torch autograd and finite differences (CPU only).

The oracle's blend VJP (splax/_rasterize/_kernels.py:530-665,1212-1254) and projection VJP
(splax/_project/_kernels.py:356-606) are chained exactly as the reference's custom_vjp rules
(splax/_rasterize/_rasterize.py:191-231, splax/_project/_project.py:236-275) and compared with
autograd through tests/torch_ref.py on scenes without frustum clamping (there the reference's
unclamped-J backward is the exact derivative). Tolerance: relative Frobenius < 2e-4 per array
(float32 oracle vs float64 truth); a dropped term or a wrong sign is O(1).
FD: directional derivative along the gradient, rel < 8e-2 (tests/test_warp_grad.py:147-184).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import random_scene, rel_fro
from oracle import oracle as O
from torch_ref import blend_ref, project_ref, tile_members


def _oracle_forward(sc, n, vm=None):
    H, W = sc["img_shape"]
    q = np.roll(sc["quats"], -1, axis=-1)
    vm = sc["vm"] if vm is None else vm
    proj = O.project_fwd(sc["means"], sc["scales"], q, vm, sc["opac"], n=n, total=n,
                         img_shape=(H, W), f=sc["f"], c=sc["c"])
    xys, depths, radii, conics, nth, cum = proj
    out = O.rasterize_fwd(sc["colors"], sc["opac"], sc["opac"], sc["bg"], xys, depths, radii,
                          conics, cum, n=n, B=1, img_shape=(H, W))
    return proj, out


def _oracle_grads(sc, n, w):
    H, W = sc["img_shape"]
    q = np.roll(sc["quats"], -1, axis=-1)
    proj, (img, Ts, fidx, stats, M) = _oracle_forward(sc, n)
    xys, depths, radii, conics, nth, cum = proj
    v_colors, v_opac, v_xy, v_conic, _ = O.rasterize_bwd(
        sc["colors"], sc["opac"], sc["opac"], sc["bg"], xys, depths, radii, conics, cum, Ts, fidx,
        w.astype(np.float32), n=n, B_out=1, B_geom=1, img_shape=(H, W))
    v_mean, v_scale, v_quat, v_view, _ = O.project_bwd(
        sc["means"], sc["scales"], q, sc["vm"], radii, conics, v_xy, np.zeros(n, np.float32),
        v_conic, n=n, B=1, f=sc["f"])
    v_quat_wxyz = np.roll(v_quat, 1, axis=-1)
    return dict(colors=v_colors, opac=v_opac, xy=v_xy, conic=v_conic, means=v_mean,
                scales=v_scale, quats=v_quat_wxyz, viewmat=v_view), proj, img


def _torch_grads(sc, n, w, proj):
    """Autograd of the float64 restatement over the oracle's tile assignment and order."""
    H, W = sc["img_shape"]
    xys_o, depths_o, radii_o, conics_o, nth_o, cum_o = proj
    sk, sid, bins = O.sort_and_bin(xys_o, depths_o, radii_o, conics_o, sc["opac"], cum_o, n=n,
                                   B=1, img_shape=(H, W))
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
    means, scales, quats = t(sc["means"]), t(sc["scales"]), t(sc["quats"])
    colors, opac, vm = t(sc["colors"]), t(sc["opac"][:, 0]), t(sc["vm"])
    xys, depths, conics, _ = project_ref(means, scales, quats, vm, f=sc["f"], c=sc["c"],
                                         img_shape=(H, W), clamp=False)
    xys.retain_grad()
    conics.retain_grad()
    img, _, _ = blend_ref(xys, conics, opac, colors, torch.from_numpy(sc["bg"].astype(np.float64)),
                          order, mem, img_shape=(H, W))
    loss = (torch.from_numpy(w.astype(np.float64)) * img).sum()
    loss.backward()
    g = dict(colors=colors.grad, opac=opac.grad, xy=xys.grad, conic=conics.grad,
             means=means.grad, scales=scales.grad, quats=quats.grad, viewmat=vm.grad)
    return {k: v.numpy() for k, v in g.items()}, img.detach().numpy()


def _scene(seed):
    # means near the optical axis so no item reaches the 1.3 tan(fov) clamp
    return random_scene(150, 48, 56, seed=seed, scale_range=(0.03, 0.12), mean_scale=0.4,
                        opac_range=(0.2, 0.9))


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_vjps_match_autograd(seed):
    sc = _scene(seed)
    H, W = sc["img_shape"]
    n = 150
    w = np.random.default_rng(100 + seed).uniform(-1, 1, (H, W, 3))
    go, proj, img = _oracle_grads(sc, n, w)
    gt, timg = _torch_grads(sc, n, w, proj)
    assert np.abs(img.reshape(H, W, 3) - timg).max() < 1e-5
    vis = proj[2] > 0
    assert vis.sum() > 50
    for k in ("colors", "opac", "xy", "conic", "means", "scales", "quats"):
        a = go[k].reshape(gt[k].shape)
        b = gt[k]
        if k in ("xy", "conic", "means", "scales", "quats"):
            a, b = a[vis], b[vis]
        r = rel_fro(a, b)
        assert r < 2e-4, f"{k}: relative Frobenius error {r:.2e}"
    r = rel_fro(go["viewmat"][:3], gt["viewmat"][:3])
    assert r < 2e-4, f"viewmat: relative Frobenius error {r:.2e}"
    assert (go["viewmat"][3] == 0).all()  # bottom row carries no gradient


def _loss_oracle(sc, n, w, means=None, scales=None, quats=None, colors=None, opac=None):
    s = dict(sc)
    for k, v in (("means", means), ("scales", scales), ("quats", quats), ("colors", colors),
                 ("opac", opac)):
        if v is not None:
            s[k] = np.ascontiguousarray(v, np.float32)
    _, (img, *_rest) = _oracle_forward(s, n)
    return float((w * img.reshape(w.shape).astype(np.float64)).mean())


def test_finite_difference_along_gradient():
    sc = random_scene(400, 80, 80, seed=7, scale_range=(0.02, 0.08), mean_scale=0.5)
    n = 400
    H, W = sc["img_shape"]
    w = np.random.default_rng(5).uniform(0, 1, (H, W, 3))
    go, proj, _ = _oracle_grads(sc, n, (w / w.size).astype(np.float32))
    names = ("means", "scales", "quats", "colors", "opac")
    base = {"means": sc["means"], "scales": sc["scales"], "quats": sc["quats"],
            "colors": sc["colors"], "opac": sc["opac"]}
    grads = {k: go[k].reshape(base[k].shape).astype(np.float64) for k in names}
    dirs = {k: g / (np.linalg.norm(g) + 1e-12) for k, g in grads.items()}
    analytic = sum(float((grads[k] * dirs[k]).sum()) for k in names)
    eps = 2e-3
    plus = {k: base[k] + eps * dirs[k] for k in names}
    minus = {k: base[k] - eps * dirs[k] for k in names}
    numeric = (_loss_oracle(sc, n, w, **plus) - _loss_oracle(sc, n, w, **minus)) / (2 * eps)
    rel = abs(analytic - numeric) / (abs(numeric) + 1e-12)
    assert rel < 8e-2, f"FD mismatch: analytic {analytic:.6e} numeric {numeric:.6e} ({rel:.2e})"


def test_viewmat_finite_difference():
    """Directional FD of the pose gradient on its 12 entries (tests/test_warp_grad.py:240-263)."""
    sc = random_scene(4000, 120, 120, seed=11, scale_range=(0.02, 0.08), mean_scale=0.5,
                      opac_range=(0.1, 0.6))
    n = 4000
    H, W = sc["img_shape"]
    w = np.random.default_rng(4).uniform(0, 1, (H, W, 3))
    go, proj, _ = _oracle_grads(sc, n, (w / w.size).astype(np.float32))
    g = go["viewmat"].astype(np.float64)
    assert np.isfinite(g).all() and (g[3] == 0).all()
    d = np.zeros((4, 4))
    d[:3] = g[:3] / (np.linalg.norm(g[:3]) + 1e-12)
    analytic = float((g * d).sum())
    eps = 1e-3

    def loss(vm):
        return float((w * _oracle_forward(sc, n, vm=vm.astype(np.float32))[1][0]
                      .reshape(H, W, 3)).mean())

    numeric = (loss(sc["vm"] + eps * d) - loss(sc["vm"] - eps * d)) / (2 * eps)
    rel = abs(analytic - numeric) / (abs(numeric) + 1e-12)
    assert rel < 8e-2, f"viewmat FD: analytic {analytic:.6e} numeric {numeric:.6e} ({rel:.2e})"


# ---------------------------------------------------------------- depth channel
# The depth-channel backward (splax/_rasterize/_kernels.py:797-1080,1257-1302) chained as
# splax/_rasterize/_rasterize.py:316-357: v_depths flows into the projection's depth cotangent.


def _oracle_depth_grads(sc, n, w, wd):
    H, W = sc["img_shape"]
    q = np.roll(sc["quats"], -1, axis=-1)
    proj = O.project_fwd(sc["means"], sc["scales"], q, sc["vm"], sc["opac"], n=n, total=n,
                         img_shape=(H, W), f=sc["f"], c=sc["c"])
    xys, depths, radii, conics, nth, cum = proj
    img, Ts, fidx, _, _, dimg = O.rasterize_fwd(sc["colors"], sc["opac"], sc["opac"], sc["bg"],
                                                xys, depths, radii, conics, cum, n=n, B=1,
                                                img_shape=(H, W), render_depth=True)
    v_colors, v_opac, v_xy, v_conic, _, v_dep = O.rasterize_bwd(
        sc["colors"], sc["opac"], sc["opac"], sc["bg"], xys, depths, radii, conics, cum, Ts, fidx,
        w.astype(np.float32), n=n, B_out=1, B_geom=1, img_shape=(H, W),
        v_out_depth=wd.astype(np.float32))
    v_mean, v_scale, v_quat, v_view, _ = O.project_bwd(
        sc["means"], sc["scales"], q, sc["vm"], radii, conics, v_xy, v_dep, v_conic, n=n, B=1,
        f=sc["f"])
    return dict(colors=v_colors, opac=v_opac, xy=v_xy, conic=v_conic, depths=v_dep,
                means=v_mean, scales=v_scale, quats=np.roll(v_quat, 1, axis=-1),
                viewmat=v_view), proj, img, dimg


@pytest.mark.parametrize("seed", [0, 3])
def test_depth_vjps_match_autograd(seed):
    sc = _scene(seed)
    H, W = sc["img_shape"]
    n = 150
    rng = np.random.default_rng(200 + seed)
    w = rng.uniform(-1, 1, (H, W, 3))
    wd = rng.uniform(-1, 1, (H, W))
    go, proj, img, dimg = _oracle_depth_grads(sc, n, w, wd)
    xys_o, depths_o, radii_o, conics_o, nth_o, cum_o = proj
    sk, sid, bins = O.sort_and_bin(xys_o, depths_o, radii_o, conics_o, sc["opac"], cum_o, n=n,
                                   B=1, img_shape=(H, W))
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
    means, scales, quats = t(sc["means"]), t(sc["scales"]), t(sc["quats"])
    colors, opac, vm = t(sc["colors"]), t(sc["opac"][:, 0]), t(sc["vm"])
    xys, tz, conics, _ = project_ref(means, scales, quats, vm, f=sc["f"], c=sc["c"],
                                     img_shape=(H, W), clamp=False)
    # the projection's depths output, as its own node: tz also feeds xys and J, whose
    # contributions are not part of the depth output's cotangent
    depths = tz + 0.0
    for x in (xys, depths, conics):
        x.retain_grad()
    timg, _, _, tdep = blend_ref(xys, conics, opac, colors,
                                 torch.from_numpy(sc["bg"].astype(np.float64)), order, mem,
                                 img_shape=(H, W), depths=depths)
    assert np.abs(dimg.reshape(H, W) - tdep.detach().numpy()).max() < 1e-5
    loss = ((torch.from_numpy(w) * timg).sum() + (torch.from_numpy(wd) * tdep).sum())
    loss.backward()
    gt = dict(colors=colors.grad, opac=opac.grad, xy=xys.grad, conic=conics.grad,
              depths=depths.grad.reshape(-1), means=means.grad, scales=scales.grad,
              quats=quats.grad, viewmat=vm.grad)
    vis = proj[2] > 0
    for k in ("colors", "opac", "xy", "conic", "depths", "means", "scales", "quats"):
        a = go[k].reshape(gt[k].shape)
        b = gt[k].numpy()
        if k in ("xy", "conic", "depths", "means", "scales", "quats"):
            a, b = a[vis], b[vis]
        r = rel_fro(a, b)
        assert r < 2e-4, f"{k}: relative Frobenius error {r:.2e}"
    assert rel_fro(go["viewmat"][:3], gt["viewmat"][:3].numpy()) < 2e-4


def _depth_loss_oracle(sc, n, w, wd, mode, **params):
    s = dict(sc)
    for k, v in params.items():
        s[k] = np.ascontiguousarray(v, np.float32)
    H, W = sc["img_shape"]
    q = np.roll(s["quats"], -1, axis=-1)
    xys, depths, radii, conics, nth, cum = O.project_fwd(
        s["means"], s["scales"], q, s["vm"], s["opac"], n=n, total=n, img_shape=(H, W), f=s["f"],
        c=s["c"])
    img, _, _, _, _, dimg = O.rasterize_fwd(s["colors"], s["opac"], s["opac"], s["bg"], xys,
                                            depths, radii, conics, cum, n=n, B=1,
                                            img_shape=(H, W), render_depth=True)
    dl = float((wd * dimg.reshape(H, W).astype(np.float64)).mean())
    if mode == "depth_only":
        return dl
    return float((w * img.reshape(H, W, 3).astype(np.float64)).mean()) + dl


@pytest.mark.parametrize("mode", ["depth_only", "mixed"])
def test_depth_finite_difference(mode):
    """Directional FD of a depth (and mixed colour + depth) loss, as the reference's
    tests/test_depth_reg.py:126-163; a depth-only loss has exactly zero colour gradient."""
    sc = random_scene(400, 80, 80, seed=7, scale_range=(0.02, 0.08), mean_scale=0.5)
    n = 400
    H, W = sc["img_shape"]
    rng = np.random.default_rng(9)
    wd = rng.uniform(0, 1, (H, W))
    w = rng.uniform(0, 1, (H, W, 3)) if mode == "mixed" else np.zeros((H, W, 3))
    go, _, _, _ = _oracle_depth_grads(sc, n, (w / w.size).astype(np.float32),
                                      (wd / wd.size).astype(np.float32))
    if mode == "depth_only":
        assert float(np.abs(go["colors"]).max()) == 0.0
    assert float(np.linalg.norm(go["means"])) > 0.0
    names = ("means", "scales", "quats", "colors", "opac")
    base = {k: sc[k] for k in names}
    grads = {k: go[k].reshape(base[k].shape).astype(np.float64) for k in names}
    dirs = {k: g / (np.linalg.norm(g) + 1e-12) for k, g in grads.items()}
    analytic = sum(float((grads[k] * dirs[k]).sum()) for k in names)
    eps = 2e-3
    plus = {k: base[k] + eps * dirs[k] for k in names}
    minus = {k: base[k] - eps * dirs[k] for k in names}
    numeric = (_depth_loss_oracle(sc, n, w, wd, mode, **plus) -
               _depth_loss_oracle(sc, n, w, wd, mode, **minus)) / (2 * eps)
    rel = abs(analytic - numeric) / (abs(numeric) + 1e-12)
    assert rel < 8e-2, f"FD mismatch: analytic {analytic:.6e} numeric {numeric:.6e} ({rel:.2e})"
