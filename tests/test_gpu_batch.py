"""Nested batching on the GPU: leading batch axes fold into one launch, outer axis major, as the
reference's nested_vmap flattens nested jax.vmap axes (splax/_batching.py:32-115). Mirrors the
reference's tests/test_warp_batch.py:157-244: an A splats x B viewmats grid equals the double loop
bit for bit, a shared splat with viewmats on both axes and transforms on the outer axis only
equals the double loop bit for bit, and nested gradients equal the double loop of gradients
within the gradient bar (the blend backward's per-record sums over a tile's waves may add in
another order).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import splax_amd
from conftest import assert_bit_exact, random_scene, rel_fro
from splax_amd import _lib

pytestmark = pytest.mark.gpu

N = 2000
H, W = 64, 80
KW = dict(img_shape=(H, W), f=(70.0, 70.0), c=(40.0, 32.0))


@pytest.fixture(autouse=True)
def _device_healthy():
    yield
    assert _lib.check_device() == 0


def _case(msg):
    print(f"[case] {msg}", flush=True)


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _np(t):
    return t.detach().cpu().numpy()


def _splat(seed):
    sc = random_scene(N, H, W, seed=seed, scale_range=(0.01, 0.06), mean_scale=0.8)
    return [_t(sc[k]) for k in ("means", "scales", "quats", "colors", "opac")]


def _viewmat(shift):
    vm = np.eye(4, dtype=np.float32)
    vm[:3, 3] = [0.2 + shift, -0.1 + 0.5 * shift, 5.0]
    return vm


VIEWS = np.stack([_viewmat(0.1 * i) for i in range(3)])
BG = np.array([1.0, 1.0, 1.0], np.float32)


def _render(m, s, q, c, o, vm, **kw):
    return splax_amd.render(m, s, q, c, o, viewmat=vm, background=_t(BG), **KW, **kw)[0]


def test_nested_grid_equals_double_loop():
    """A splats (outer axis) x B viewmats (inner axis) in one launch == the A x B double loop."""
    _case("nested grid 3 x 3")
    scenes = [_splat(s) for s in (3, 4, 5)]
    A, B = len(scenes), VIEWS.shape[0]
    stacked = [torch.stack([sc[i] for sc in scenes])[:, None] for i in range(5)]  # (A, 1, N, .)
    out = _render(*stacked, _t(VIEWS))
    assert out.shape == (A, B, H, W, 3)
    for a in range(A):
        for b in range(B):
            ref = _render(*scenes[a], _t(VIEWS[b]))
            assert_bit_exact(_np(out[a, b]), _np(ref), f"grid ({a}, {b})")


def test_nested_shared_splat_outer_transforms():
    """Shared splat, viewmats on both axes, transforms on the outer axis only
    (tests/test_warp_batch.py:174-203 of the reference)."""
    _case("nested shared splat + outer transforms")
    m, s, q, c, o = _splat(6)
    slices = [(0, N // 2), (N // 2, N)]
    n_worlds, n_cams = 2, 3
    vms = np.stack([np.stack([_viewmat(0.1 * w + 0.03 * cam) for cam in range(n_cams)])
                    for w in range(n_worlds)])
    tfs = np.zeros((n_worlds, 2, 4, 4), np.float32)
    for w in range(n_worlds):
        tfs[w] = np.eye(4, dtype=np.float32)
        tfs[w, :, 0, 3] = 0.02 * w
    out = _render(m, s, q, c, o, _t(vms), gaussian_transforms=_t(tfs)[:, None],
                  gaussian_slices=slices)
    assert out.shape == (n_worlds, n_cams, H, W, 3)
    for w in range(n_worlds):
        for cam in range(n_cams):
            ref = _render(m, s, q, c, o, _t(vms[w, cam]), gaussian_transforms=_t(tfs[w]),
                          gaussian_slices=slices)
            assert_bit_exact(_np(out[w, cam]), _np(ref), f"world {w} cam {cam}")


def test_nested_grad_equals_double_loop_of_grads():
    """Gradients of per-(a, b) means under the nested batch == each single render's gradient."""
    _case("nested grad 2 x 3")
    m, s, q, c, o = _splat(12)
    means = torch.stack([m, m * 1.01])  # (A, N, 3)
    A, B = 2, VIEWS.shape[0]
    leaf = means[:, None].expand(A, B, N, 3).clone().requires_grad_(True)
    _render(leaf, s, q, c, o, _t(VIEWS)).sum().backward()
    for a in range(A):
        for b in range(B):
            mm = means[a].clone().requires_grad_(True)
            _render(mm, s, q, c, o, _t(VIEWS[b])).sum().backward()
            got, ref = _np(leaf.grad[a, b]), _np(mm.grad)
            r = rel_fro(got, ref)
            assert r < 1e-5, f"({a}, {b}): relative Frobenius error {r:.2e}"
            np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-5 * np.abs(ref).max())


def test_partly_batched_geometry_is_tiled():
    """Geometry projected for B cameras (inner axis) rasterized with colours batched over an
    outer axis: the geometry is tiled over the outer axis and its global tile-count prefix formed
    again, as the reference tiles a partly batched operand (splax/_batching.py:96-97). Compared
    bit for bit with the oracle's render of the tiled batch. (Against single renders the images
    may differ: six images leave 23 depth bits where one leaves 26, so two depths 5e-7 apart can
    share a quantized depth and blend in id order, which the reference's key does as well.)"""
    from oracle import oracle as O

    _case("partly batched geometry")
    sc = random_scene(N, H, W, seed=8, scale_range=(0.01, 0.06), mean_scale=0.8)
    m, s, q, c, o = [_t(sc[k]) for k in ("means", "scales", "quats", "colors", "opac")]
    B = VIEWS.shape[0]
    xys, depths, radii, conics, nth, cum = splax_amd.project(m, s, q, _t(VIEWS), opacities=o,
                                                             **KW)
    colors = torch.stack([c, 1.0 - c])[:, None]  # (2, 1, N, 3)
    out = splax_amd.rasterize(colors, o, _t(BG), xys, depths, radii, conics, cum,
                              img_shape=KW["img_shape"])
    assert out.shape == (2, B, H, W, 3)
    rep = lambda t, w: np.concatenate([_np(t).reshape(B * N, w)] * 2)  # noqa: E731
    nth_t = np.concatenate([_np(nth).reshape(-1)] * 2)
    cols = np.concatenate([np.repeat(_np(colors)[a], B, axis=0).reshape(B * N, 3)
                           for a in range(2)])
    ref = O.rasterize_fwd(cols, sc["opac"], sc["opac"], BG, rep(xys, 2), rep(depths, 1),
                          rep(radii, 1), rep(conics, 3), np.cumsum(nth_t).astype(np.int32),
                          n=N, B=2 * B, img_shape=KW["img_shape"])[0]
    assert_bit_exact(_np(out).reshape(ref.shape), ref, "tiled geometry vs oracle")


def test_nested_render_loss_equals_render_then_loss():
    """render_loss over a nested batch (A splats on the outer axis x B viewmats on the inner one,
    folded into one launch) against render over the same batch followed by the library's MSE:
    the target's (A, B) images line up with the folded images, so the image, the loss and the
    gradients agree (image bit for bit, loss within one ulp, gradients within the bar)."""
    from splax_amd.train import mse_loss

    _case("nested render_loss 3 x 3")
    scenes = [_splat(s) for s in (7, 8, 9)]
    A, B = len(scenes), VIEWS.shape[0]
    tgt = _t(np.random.default_rng(11).uniform(size=(A, B, H, W, 3)).astype(np.float32))
    outs = []
    for fused in (True, False):
        stacked = [torch.stack([sc[i] for sc in scenes])[:, None].clone().requires_grad_(True)
                   for i in range(5)]  # (A, 1, N, .)
        kw = dict(viewmat=_t(VIEWS), background=_t(BG), **KW)
        if fused:
            loss, img = splax_amd.render_loss(*stacked, target=tgt, loss="mse", **kw)
        else:
            img = splax_amd.render(*stacked, **kw)[0]
            loss = mse_loss(img, tgt)
        loss.backward()
        torch.cuda.synchronize()
        outs.append((_np(img), float(loss.item()), [_np(t.grad) for t in stacked]))
    (fi, fl, fg), (ui, ul, ug) = outs
    assert fi.shape == (A, B, H, W, 3)
    assert_bit_exact(fi, ui, "nested image")
    assert abs(fl - ul) <= float(np.spacing(np.float32(ul))), (fl, ul)
    for k, (a, b) in enumerate(zip(fg, ug)):
        r = rel_fro(a.astype(np.float64), b.astype(np.float64))
        assert r < 1e-5, f"gradient {k}: {r:.2e}"
