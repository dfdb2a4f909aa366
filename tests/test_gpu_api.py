"""GPU tests of the torch-facing API (splax_amd.render / project / rasterize with autograd).

Mirrors the reference's API tests: render == oracle pipeline, gradients == the oracle's chained
VJPs (tests/test_warp_grad.py), batched cameras == stacked single renders and summed shared
gradients (tests/test_warp_batch.py, tests/test_warp_grad_batched.py), antialiased compensation
(tests/test_antialiased.py), render_log, rigid transforms (tests/test_transforms.py), the
broadcast-geometry backward (B_geom = 1 < B_out) and the empty / single-intersection edge cases.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import splax_amd
from conftest import assert_bit_exact, random_scene, rel_fro
from oracle import oracle as O
from splax_amd import _lib, _ops

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _device_healthy():
    yield
    assert _lib.check_device() == 0


def _case(msg):
    print(f"[case] {msg}", flush=True)


def _t(a, grad=False):
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return t.requires_grad_(True) if grad else t


def _np(t):
    return t.detach().cpu().numpy()


def _oracle_render_and_grads(sc, n, w, opac_blend=None, vm=None):
    """The oracle's forward and chained backward of sum(img * w); with B stacked viewmats (vm of
    shape (B, 4, 4), w of shape (B, H, W, 3)) the per-camera item gradients are summed."""
    H, W = sc["img_shape"]
    vm = sc["vm"] if vm is None else vm
    B = vm.size // 16
    q = np.roll(sc["quats"], -1, axis=-1)
    xys, depths, radii, conics, nth, cum = O.project_fwd(
        sc["means"], sc["scales"], q, vm.reshape(-1, 4), sc["opac"], n=n, total=B * n,
        img_shape=(H, W), f=sc["f"], c=sc["c"])
    ob = sc["opac"] if opac_blend is None else opac_blend
    img, Ts, fidx, _, _ = O.rasterize_fwd(sc["colors"], ob, sc["opac"], sc["bg"], xys, depths,
                                          radii, conics, cum, n=n, B=B, img_shape=(H, W))
    vc, vo, vxy, vcon, _ = O.rasterize_bwd(sc["colors"], ob, sc["opac"], sc["bg"], xys, depths,
                                           radii, conics, cum, Ts, fidx,
                                           w.reshape(-1, 3).astype(np.float32), n=n, B_out=B,
                                           B_geom=B, img_shape=(H, W))
    vm_, vs_, vq_, vv_, _ = O.project_bwd(sc["means"], sc["scales"], q, vm.reshape(-1, 4), radii,
                                          conics, vxy, np.zeros(B * n, np.float32), vcon, n=n,
                                          B=B, f=sc["f"])
    fold = (lambda a: a.reshape(B, n, -1).astype(np.float64).sum(0).astype(np.float32)) \
        if B > 1 else (lambda a: a)
    shape = (B, H, W, 3) if B > 1 else (H, W, 3)
    return img.reshape(shape), dict(means=fold(vm_), scales=fold(vs_),
                                    quats=np.roll(fold(vq_), 1, axis=-1), colors=fold(vc),
                                    opac=fold(vo.reshape(-1, 1)),
                                    viewmat=vv_.reshape(B, 4, 4) if B > 1 else vv_)


def test_render_and_grads_match_oracle():
    _case("render + grads vs oracle")
    n, H, W = 6000, 128, 160
    sc = random_scene(n, H, W, seed=3)
    w = np.random.default_rng(1).uniform(-1, 1, (H, W, 3)).astype(np.float32)
    ref_img, ref_g = _oracle_render_and_grads(sc, n, w)
    p = {k: _t(sc[k], grad=True) for k in ("means", "scales", "quats", "colors", "opac")}
    vm = _t(sc["vm"], grad=True)
    img, depth = splax_amd.render(p["means"], p["scales"], p["quats"], p["colors"], p["opac"],
                                  viewmat=vm, background=_t(sc["bg"]), img_shape=(H, W),
                                  f=sc["f"], c=sc["c"])
    assert depth is None and img.shape == (H, W, 3)
    assert_bit_exact(_np(img), ref_img, "render/img")
    (img * _t(w)).sum().backward()
    for k in ("means", "scales", "quats", "colors", "opac"):
        r = rel_fro(_np(p[k].grad), ref_g[k])
        assert r < 1e-5, f"{k}: relative Frobenius error {r:.2e}"
    assert rel_fro(_np(vm.grad), ref_g["viewmat"]) < 1e-5
    assert (_np(vm.grad)[3] == 0).all()


def test_size_one_background_renders_one_image():
    """A background of shape (1, 3) is one shared colour (the reference reshapes it to (1, 3)
    inside rasterize, splax/_rasterize/_rasterize.py:131): the image stays (H, W, 3) and equals
    the render with a (3,) background bit for bit, loss and gradients included."""
    _case("background (1, 3)")
    n, H, W = 3000, 64, 80
    sc = random_scene(n, H, W, seed=12)
    outs = []
    for bg in (sc["bg"], sc["bg"].reshape(1, 3), sc["bg"].reshape(1, 1, 3)):
        p = [_t(sc[k], grad=True) for k in ("means", "scales", "quats", "colors", "opac")]
        img, _ = splax_amd.render(*p, viewmat=_t(sc["vm"]), background=_t(bg),
                                  img_shape=(H, W), f=sc["f"], c=sc["c"])
        assert img.shape == (H, W, 3), bg.shape
        img.sum().backward()
        loss, img2 = splax_amd.render_loss(*[_t(sc[k]) for k in ("means", "scales", "quats",
                                                                  "colors", "opac")],
                                           target=torch.zeros((H, W, 3), device="cuda"),
                                           viewmat=_t(sc["vm"]), background=_t(bg),
                                           img_shape=(H, W), f=sc["f"], c=sc["c"])
        assert img2.shape == (H, W, 3)
        outs.append([_np(img), _np(loss)] + [_np(t.grad) for t in p])
    for other in outs[1:]:
        for k, (a, b) in enumerate(zip(other, outs[0])):
            assert_bit_exact(a, b, f"output {k}")


def _stress_scene():
    """test_gpu_parity's extremes scene (huge, needle-thin and near-plane gaussians, opacities at
    the clamp and the threshold), in random_scene's dictionary form."""
    import importlib.util
    from pathlib import Path

    spec = importlib.util.spec_from_file_location(
        "gpu_parity", Path(__file__).with_name("test_gpu_parity.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod._stress_scene()


@pytest.mark.parametrize("scene", ["random", "stress"])
def test_batched_cameras_equal_stacked(scene):
    _case(f"batched viewmats {scene}")
    if scene == "random":
        sc = random_scene(4000, 96, 96, seed=8)
    else:
        sc = _stress_scene()
    H, W = sc["img_shape"]
    vms = np.stack([sc["vm"]] * 3)
    vms[1, 0, 3] += 0.25
    vms[2, 1, 3] -= 0.2
    w = np.random.default_rng(2).uniform(-1, 1, (3, H, W, 3)).astype(np.float32)

    def run(vm_np, w_np):
        p = {k: _t(sc[k], grad=True) for k in ("means", "scales", "quats", "colors", "opac")}
        img, _ = splax_amd.render(p["means"], p["scales"], p["quats"], p["colors"], p["opac"],
                                  viewmat=_t(vm_np), background=_t(sc["bg"]), img_shape=(H, W),
                                  f=sc["f"], c=sc["c"])
        (img * _t(w_np)).sum().backward()
        return _np(img), {k: _np(v.grad) for k, v in p.items()}

    bimg, bg = run(vms, w)
    assert bimg.shape == (3, H, W, 3)
    singles = [run(vms[b], w[b]) for b in range(3)]
    if scene == "random":
        for b in range(3):
            assert_bit_exact(bimg[b], singles[b][0], f"batched/img[{b}]")
        for k in bg:
            summed = sum(s[1][k].astype(np.float64) for s in singles)
            r = rel_fro(bg[k], summed)
            assert r < 1e-5, f"batched/{k}: {r:.2e}"
        return
    # three images leave 20 depth bits against a single render's 22 (the key's image field), so
    # items whose quantized depths tie only in the batch blend in another order there, as in the
    # reference, whose batched key has this layout: the batch is held to the oracle's batched
    # forward bit for bit, the single renders to within float rounding
    import timed_path as TP

    rimg, rg, cond = TP.weighted_chain(sc, w, vm=vms)
    _, tg, _ = TP.weighted_chain(sc, w, vm=vms, truth=True)
    assert_bit_exact(bimg, rimg.reshape(bimg.shape), "batched/img vs the batched oracle")
    for b in range(3):
        np.testing.assert_allclose(bimg[b], singles[b][0], rtol=1e-5, atol=1e-6)
    # the mean / scale / quaternion gradients of a needle-thin item are ill-conditioned in
    # float32: v_cov2d = -conic v_conic conic scales rounding in v_conic (and the conic-weighted
    # v_xy) by up to cond(conic)^2, so the float32 oracle and the kernel, which sum pixels in
    # different orders, both stray from the float64 truth there. Every gradient is held per
    # condition band to the truth (at most timed_path.FACTOR times the float32 oracle's error, or
    # 1e-5), items below condition 1e2 in every camera to the oracle at the usual bar, and each
    # single render to its own truth the same way.
    well = cond < 1e2
    assert well.sum() > 4000 and (~well).sum() > 2000
    for k in bg:
        ref = np.asarray(rg[k], np.float64).reshape(bg[k].shape)
        truth = np.asarray(tg[k], np.float64).reshape(bg[k].shape)
        r = rel_fro(bg[k][well], ref[well])
        assert r < 1e-5, f"batched/{k} (cond < 1e2) vs the batched oracle: {r:.2e}"
        TP.assert_bands(bg[k], ref, truth, cond, f"batched/{k}")
    for b in range(3):
        _, r1, c1 = TP.weighted_chain(sc, w[b], vm=vms[b])
        _, t1, _ = TP.weighted_chain(sc, w[b], vm=vms[b], truth=True)
        for k in bg:
            TP.assert_bands(singles[b][1][k], np.asarray(r1[k]).reshape(bg[k].shape),
                            np.asarray(t1[k]).reshape(bg[k].shape), c1, f"single {b}/{k}")


def test_batched_viewmat_grads_per_pose():
    _case("batched viewmat grads")
    n, H, W = 3000, 64, 80
    sc = random_scene(n, H, W, seed=9)
    vms = np.stack([sc["vm"]] * 2)
    vms[1, 0, 3] += 0.3
    vm = _t(vms, grad=True)
    args = [_t(sc[k]) for k in ("means", "scales", "quats", "colors", "opac")]
    img, _ = splax_amd.render(*args, viewmat=vm, background=_t(sc["bg"]), img_shape=(H, W),
                              f=sc["f"], c=sc["c"])
    img.sum().backward()
    g = _np(vm.grad)
    for b in range(2):
        v1 = _t(vms[b], grad=True)
        i1, _ = splax_amd.render(*args, viewmat=v1, background=_t(sc["bg"]), img_shape=(H, W),
                                 f=sc["f"], c=sc["c"])
        i1.sum().backward()
        assert rel_fro(g[b], _np(v1.grad)) < 1e-5


def test_antialiased_matches_compensated_oracle():
    _case("antialiased")
    n, H, W = 3000, 96, 96
    sc = random_scene(n, H, W, seed=4)
    img_aa, _ = splax_amd.render(*[_t(sc[k]) for k in ("means", "scales", "quats", "colors",
                                                        "opac")], viewmat=_t(sc["vm"]),
                                 background=_t(sc["bg"]), img_shape=(H, W), f=sc["f"],
                                 c=sc["c"], antialiased=True)
    q = np.roll(sc["quats"], -1, axis=-1)
    xys, depths, radii, conics, nth, cum = O.project_fwd(
        sc["means"], sc["scales"], q, sc["vm"], sc["opac"], n=n, total=n, img_shape=(H, W),
        f=sc["f"], c=sc["c"])
    rho = _np(splax_amd.opacity_compensation(_t(conics), _t(radii)))
    ob = (sc["opac"] * rho[:, None]).astype(np.float32)
    ref, _, _, _, _ = O.rasterize_fwd(sc["colors"], ob, sc["opac"], sc["bg"], xys, depths, radii,
                                      conics, cum, n=n, B=1, img_shape=(H, W))
    assert_bit_exact(_np(img_aa), ref.reshape(H, W, 3), "antialiased/img")
    plain, _ = splax_amd.render(*[_t(sc[k]) for k in ("means", "scales", "quats", "colors",
                                                       "opac")], viewmat=_t(sc["vm"]),
                                background=_t(sc["bg"]), img_shape=(H, W), f=sc["f"], c=sc["c"])
    assert np.abs(_np(plain) - _np(img_aa)).max() > 1e-3


def test_antialiased_grads_match_unfused_path():
    """render(antialiased=True) fuses the compensation into the blend; its gradients equal the
    composition of opacity_compensation (torch autograd) and rasterize."""
    _case("antialiased grads")
    n, H, W = 3000, 96, 96
    sc = random_scene(n, H, W, seed=4)
    keys = ("means", "scales", "quats", "colors", "opac")
    target = torch.rand((H, W, 3), device="cuda", generator=torch.Generator("cuda").manual_seed(3))

    def leaves():
        return [_t(sc[k]).requires_grad_(True) for k in keys]

    a = leaves()
    img, _ = splax_amd.render(*a, viewmat=_t(sc["vm"]), background=_t(sc["bg"]),
                              img_shape=(H, W), f=sc["f"], c=sc["c"], antialiased=True)
    (img - target).abs().mean().backward()
    b = leaves()
    xys, depths, radii, conics, _, cum = splax_amd.project(
        b[0], b[1], b[2], _t(sc["vm"]), opacities=b[4], img_shape=(H, W), f=sc["f"], c=sc["c"])
    rho = splax_amd.opacity_compensation(conics, radii).unsqueeze(-1)
    img2 = splax_amd.rasterize(b[3], b[4] * rho, _t(sc["bg"]), xys, depths, radii, conics, cum,
                               img_shape=(H, W), map_opacities=b[4])
    assert_bit_exact(_np(img), _np(img2), "antialiased fused vs unfused image")
    (img2 - target).abs().mean().backward()
    for k, x, y in zip(keys, a, b):
        g, r = _np(x.grad), _np(y.grad)
        assert rel_fro(g, r) < 1e-5, (k, rel_fro(g, r))


def test_render_log_equals_render():
    _case("render_log")
    n, H, W = 2000, 64, 64
    sc = random_scene(n, H, W, seed=12)
    rng = np.random.default_rng(3)
    log_s = np.log(sc["scales"])
    logit_c = rng.normal(size=(n, 3)).astype(np.float32)
    logit_o = rng.normal(size=(n, 1)).astype(np.float32)
    quats = (sc["quats"] * 1.7).astype(np.float32)
    cam = dict(viewmat=_t(sc["vm"]), background=_t(sc["bg"]), img_shape=(H, W), f=sc["f"],
               c=sc["c"])
    a, _ = splax_amd.render_log(_t(sc["means"]), _t(log_s), _t(quats), _t(logit_c), _t(logit_o),
                                **cam)
    from oracle import train_oracle as TO

    act = TO.log_params_fwd(log_s, quats, logit_c, logit_o)  # the library's parameter map
    b, _ = splax_amd.render(_t(sc["means"]), _t(act[0]), _t(act[1]), _t(act[2]),
                            _t(act[3].reshape(n, 1)), **cam)
    assert_bit_exact(_np(a), _np(b), "render_log")
    # within float32 rounding of torch's own exp / norm / sigmoid
    tq = _t(quats)
    c, _ = splax_amd.render(_t(sc["means"]), torch.exp(_t(log_s)),
                            tq / (torch.linalg.norm(tq, dim=-1, keepdim=True) + 1e-8),
                            torch.sigmoid(_t(logit_c)), torch.sigmoid(_t(logit_o)), **cam)
    assert np.abs(_np(a) - _np(c)).max() < 1e-4


def test_rigid_transforms_forward_and_grads():
    _case("transforms")
    n, H, W = 2000, 80, 80
    sc = random_scene(n, H, W, seed=21)
    ang = 0.2
    tf = np.eye(4, dtype=np.float32)
    tf[:3, :3] = [[np.cos(ang), -np.sin(ang), 0], [np.sin(ang), np.cos(ang), 0], [0, 0, 1]]
    tf[:3, 3] = [0.05, 0.1, -0.1]
    tft = _t(tf[None], grad=True)
    cam = dict(viewmat=_t(sc["vm"]), background=_t(sc["bg"]), img_shape=(H, W), f=sc["f"],
               c=sc["c"])
    args = [_t(sc[k]) for k in ("means", "scales", "quats", "colors", "opac")]
    img, _ = splax_amd.render(*args, gaussian_transforms=tft, gaussian_slices=[(500, 1500)],
                              **cam)
    # identity transform == plain render, bit for bit
    eye = _t(np.eye(4, dtype=np.float32)[None])
    img_id, _ = splax_amd.render(*args, gaussian_transforms=eye, gaussian_slices=[(500, 1500)],
                                 **cam)
    plain, _ = splax_amd.render(*args, **cam)
    assert_bit_exact(_np(img_id), _np(plain), "identity transform")
    assert np.abs(_np(img) - _np(plain)).max() > 1e-3
    img.sum().backward()
    g = _np(tft.grad)
    assert np.isfinite(g).all() and np.abs(g[0, :3]).max() > 0 and (g[0, 3] == 0).all()


def test_broadcast_geometry_backward():
    """B_geom = 1 < B_out (one render differentiated against B targets) through the C ABI."""
    _case("broadcast geometry backward")
    n, H, W = 3000, 64, 64
    sc = random_scene(n, H, W, seed=30)
    q = np.roll(sc["quats"], -1, axis=-1)
    xys, depths, radii, conics, nth, cum = O.project_fwd(
        sc["means"], sc["scales"], q, sc["vm"], sc["opac"], n=n, total=n, img_shape=(H, W),
        f=sc["f"], c=sc["c"])
    img, Ts, fidx, _, _ = O.rasterize_fwd(sc["colors"], sc["opac"], sc["opac"], sc["bg"], xys,
                                          depths, radii, conics, cum, n=n, B=1, img_shape=(H, W))
    B_out = 3
    vout = np.random.default_rng(0).uniform(-1, 1, (B_out, H, W, 3)).astype(np.float32)
    ref = O.rasterize_bwd(sc["colors"], sc["opac"], sc["opac"], sc["bg"], xys, depths, radii,
                          conics, cum, Ts, fidx, vout, n=n, B_out=B_out, B_geom=1,
                          img_shape=(H, W))
    got = _ops.rasterize_bwd(_t(sc["colors"]), _t(sc["opac"]).reshape(-1),
                             _t(sc["opac"]).reshape(-1), _t(sc["bg"]), _t(xys), _t(depths),
                             _t(radii), _t(conics), _t(cum), _t(Ts), _t(fidx),
                             _t(vout).reshape(-1, 3), n=n, B_out=B_out, B_geom=1,
                             img_shape=(H, W))
    for label, g, r in zip(("v_colors", "v_opacity", "v_xy", "v_conic"), got, ref[:4]):
        assert rel_fro(_np(g).reshape(r.shape), r) < 1e-5, label


def test_empty_and_single_intersection():
    _case("M == 0 and M == 1")
    H = W = 48
    bg = np.array([0.2, 0.4, 0.6], np.float32)
    means = np.array([[0.0, 0.0, -3.0]], np.float32)  # behind the camera: M == 0
    ones = dict(scales=np.full((1, 3), 0.02, np.float32),
                quats=np.array([[1.0, 0, 0, 0]], np.float32),
                colors=np.array([[1.0, 0, 0]], np.float32), opac=np.array([[0.9]], np.float32))
    p = {k: _t(v, grad=True) for k, v in ones.items()}
    mt = _t(means, grad=True)
    img, _ = splax_amd.render(mt, p["scales"], p["quats"], p["colors"], p["opac"],
                              viewmat=_t(np.eye(4, dtype=np.float32)), background=_t(bg),
                              img_shape=(H, W), f=(40.0, 40.0))
    np.testing.assert_array_equal(_np(img), np.broadcast_to(bg, (H, W, 3)))
    img.sum().backward()
    assert (_np(mt.grad) == 0).all() and (_np(p["colors"].grad) == 0).all()
    # one small gaussian in one tile: the lone bin stays [0, 0), nothing is drawn and no
    # gradient flows (the blend never visits the intersection, whose partial sums are zeroed
    # rather than read from whatever the scratch held); a large render first leaves the
    # gradient scratch non-zero
    big = random_scene(3000, 64, 64, seed=12)
    bp = [_t(big[k], grad=True) for k in ("means", "scales", "quats", "colors", "opac")]
    splax_amd.render(*bp, viewmat=_t(big["vm"]), background=_t(big["bg"]), img_shape=(64, 64),
                     f=big["f"], c=big["c"])[0].sum().backward()
    for k in p:
        p[k].grad = None
    m1 = _t(np.array([[0.0, 0.0, 4.0]], np.float32), grad=True)
    img1, _ = splax_amd.render(m1, p["scales"], p["quats"], p["colors"], p["opac"],
                               viewmat=_t(np.eye(4, dtype=np.float32)), background=_t(bg),
                               img_shape=(H, W), f=(40.0, 40.0), c=(40.0, 40.0))
    np.testing.assert_array_equal(_np(img1), np.broadcast_to(bg, (H, W, 3)))
    img1.sum().backward()
    for g in (m1.grad, *(v.grad for v in p.values())):
        assert g is not None and (_np(g) == 0).all()


def test_render_depth_and_grads_match_oracle():
    """render(render_depth=True) (splax/_render.py:112-114): image bit-exact with the plain
    render, expected depth bit-exact with the oracle, and the gradients of a mixed colour + depth
    loss through project -> rasterize_depth (v_depths feeding the projection's depth cotangent)."""
    _case("render_depth + grads vs oracle")
    n, H, W = 6000, 128, 160
    sc = random_scene(n, H, W, seed=5)
    rng = np.random.default_rng(6)
    w = rng.uniform(-1, 1, (H, W, 3)).astype(np.float32)
    wd = rng.uniform(-1, 1, (H, W)).astype(np.float32)
    q = np.roll(sc["quats"], -1, axis=-1)
    xys, depths, radii, conics, nth, cum = O.project_fwd(
        sc["means"], sc["scales"], q, sc["vm"], sc["opac"], n=n, total=n, img_shape=(H, W),
        f=sc["f"], c=sc["c"])
    img, Ts, fidx, _, _, dimg = O.rasterize_fwd(sc["colors"], sc["opac"], sc["opac"], sc["bg"],
                                                xys, depths, radii, conics, cum, n=n, B=1,
                                                img_shape=(H, W), render_depth=True)
    vc, vo, vxy, vcon, _, vdep = O.rasterize_bwd(
        sc["colors"], sc["opac"], sc["opac"], sc["bg"], xys, depths, radii, conics, cum, Ts, fidx,
        w, n=n, B_out=1, B_geom=1, img_shape=(H, W), v_out_depth=wd)
    vm_, vs_, vq_, vv_, _ = O.project_bwd(sc["means"], sc["scales"], q, sc["vm"], radii, conics,
                                          vxy, vdep, vcon, n=n, B=1, f=sc["f"])
    ref = dict(means=vm_, scales=vs_, quats=np.roll(vq_, 1, axis=-1), colors=vc,
               opac=vo.reshape(-1, 1))
    p = {k: _t(sc[k], grad=True) for k in ("means", "scales", "quats", "colors", "opac")}
    vm = _t(sc["vm"], grad=True)
    common = dict(viewmat=vm, background=_t(sc["bg"]), img_shape=(H, W), f=sc["f"], c=sc["c"])
    gimg, gdep = splax_amd.render(p["means"], p["scales"], p["quats"], p["colors"], p["opac"],
                                  render_depth=True, **common)
    assert gdep.shape == (H, W)
    plain, _ = splax_amd.render(*[v.detach() for v in p.values()], **common)
    assert_bit_exact(_np(gimg), _np(plain), "render_depth/img vs plain render")
    assert_bit_exact(_np(gimg), img.reshape(H, W, 3), "render_depth/img")
    assert_bit_exact(_np(gdep), dimg.reshape(H, W), "render_depth/depth")
    ((gimg * _t(w)).sum() + (gdep * _t(wd)).sum()).backward()
    for k in ("means", "scales", "quats", "colors", "opac"):
        r = rel_fro(_np(p[k].grad), ref[k])
        assert r < 1e-5, f"{k}: relative Frobenius error {r:.2e}"
    assert rel_fro(_np(vm.grad), vv_) < 1e-5


def test_render_depth_batched_equals_sequential():
    """Batched cameras on the depth path equal the per-camera renders (image and depth bit for
    bit, gradients summed), as the reference's tests/test_depth_reg.py:194-229."""
    _case("render_depth batched")
    n, H, W = 2000, 64, 64
    sc = random_scene(n, H, W, seed=12)
    vms = np.stack([sc["vm"]] * 3)
    vms[1, 0, 3] += 0.2
    vms[2, 2, 3] += 0.3
    wd = np.random.default_rng(3).uniform(0, 1, (3, H, W)).astype(np.float32)

    def run(vm_np, wd_np):
        p = {k: _t(sc[k], grad=True) for k in ("means", "scales", "quats", "colors", "opac")}
        img, dep = splax_amd.render(p["means"], p["scales"], p["quats"], p["colors"], p["opac"],
                                    viewmat=_t(vm_np), background=_t(sc["bg"]), img_shape=(H, W),
                                    f=sc["f"], c=sc["c"], render_depth=True)
        (dep * _t(wd_np)).sum().backward()
        return _np(img), _np(dep), {k: _np(v.grad) for k, v in p.items()}

    bimg, bdep, bg = run(vms, wd)
    assert bdep.shape == (3, H, W)
    singles = [run(vms[b], wd[b]) for b in range(3)]
    for b in range(3):
        assert_bit_exact(bimg[b], singles[b][0], f"batched depth/img[{b}]")
        assert_bit_exact(bdep[b], singles[b][1], f"batched depth/depth[{b}]")
    assert float(np.abs(bg["colors"]).max()) == 0.0  # a depth-only loss: no colour gradient
    for k in ("means", "scales", "quats", "opac"):
        summed = sum(s[2][k].astype(np.float64) for s in singles)
        r = rel_fro(bg[k], summed)
        assert r < 1e-5, f"batched depth/{k}: {r:.2e}"


def test_wide_keys_batch_equals_stack_bit_exact():
    """With the 64-bit key each image's (tile, depth) order does not depend on B, so a batched
    render equals the per-camera renders bit for bit (the reference's tests/test_warp_batch.py
    forces the 64-bit key for exactly this, :45-56)."""
    _case("wide keys batch == stack")
    from splax_amd import _lib

    n, H, W = 3000, 96, 96
    sc = random_scene(n, H, W, seed=14)
    vms = np.stack([sc["vm"]] * 3)
    vms[1, 0, 3] += 0.2
    vms[2, 1, 3] -= 0.2
    args = [_t(sc[k]) for k in ("means", "scales", "quats", "colors", "opac")]
    common = dict(background=_t(sc["bg"]), img_shape=(H, W), f=sc["f"], c=sc["c"])
    _lib.set_wide_keys(True)
    try:
        bimg, _ = splax_amd.render(*args, viewmat=_t(vms), **common)
        singles = [splax_amd.render(*args, viewmat=_t(vms[b]), **common)[0] for b in range(3)]
    finally:
        _lib.set_wide_keys(False)
    for b in range(3):
        assert_bit_exact(_np(bimg[b]), _np(singles[b]), f"wide batch/img[{b}]")


def test_principal_point_defaults_to_center():
    """Omitting c equals passing the image centre (W / 2, H / 2) bit for bit, through render and
    render_loss (the reference's tests/test_warp_rasterize.py:198-205)."""
    _case("principal point default")
    sc = random_scene(10_000, 256, 192, seed=42)
    H, W = sc["img_shape"]
    args = [_t(sc[k]) for k in ("means", "scales", "quats", "colors", "opac")]
    kw = dict(viewmat=_t(sc["vm"]), background=_t(sc["bg"]), img_shape=(H, W), f=sc["f"])
    explicit = _np(splax_amd.render(*args, c=(W / 2, H / 2), **kw)[0])
    defaulted = _np(splax_amd.render(*args, **kw)[0])
    assert_bit_exact(defaulted, explicit, "render image")
    tgt = _t(np.zeros((H, W, 3), np.float32))
    le, ie = splax_amd.render_loss(*args, target=tgt, c=(W / 2, H / 2), **kw)
    ld, idf = splax_amd.render_loss(*args, target=tgt, **kw)
    assert_bit_exact(_np(idf), _np(ie), "render_loss image")
    assert float(ld.item()) == float(le.item())
