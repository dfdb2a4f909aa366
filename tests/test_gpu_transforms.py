"""GPU parity of the per-object rigid transforms (splax/_project/_kernels.py:176-180,461-484,
536-557,627-644), through the C ABI, against the CPU oracle (whose transform forward and VJP
tests/test_oracle_transforms.py pins against float64 autograd and finite differences).

Bars: projection outputs and the per-item gradients (v_mean3d, v_scale, v_quat) bit-exact, the
folded per-gaussian gradients bit-exact against the oracle's rows summed in image order;
v_viewmat and v_transforms, which the GPU sums with float atomics per workgroup, within relative
Frobenius 1e-5 plus allclose(rtol=1e-4, atol=1e-5 * max|ref|). The slices put workgroups of 256
items in all three of the reference's cases: one shared transform (block reduction), a slice
boundary inside the workgroup (per-thread atomics) and static items, plus workgroups whose ids
are at or past num_transforms (static, nothing added).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import assert_bit_exact, rel_fro
from oracle import oracle as O
from splax_amd import _ops

pytestmark = pytest.mark.gpu

F = (300.0, 300.0)
HW = (200, 232)
C = (116.0, 100.0)


@pytest.fixture(autouse=True)
def _device_healthy():
    yield
    from splax_amd import _lib

    assert _lib.check_device() == 0, "a device-side invariant failed"


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _np(t):
    return t.detach().cpu().numpy()


def _case(msg):
    print(f"[case] {msg}", flush=True)


def _grad_compare(got, ref, label, rel_tol=1e-5):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    r = rel_fro(got, ref)
    assert r < rel_tol, f"{label}: relative Frobenius error {r:.3e}"
    scale = float(np.abs(ref).max()) + 1e-30
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-5 * scale, err_msg=label)


def _rot(rng, max_angle):
    axis = rng.normal(size=3)
    axis /= np.linalg.norm(axis)
    ang = rng.uniform(-max_angle, max_angle)
    K = np.array([[0, -axis[2], axis[1]], [axis[2], 0, -axis[0]], [-axis[1], axis[0], 0]])
    return np.eye(3) + np.sin(ang) * K + (1 - np.cos(ang)) * K @ K


def _transforms(rng, count):
    tf = np.zeros((count, 4, 4), np.float32)
    for k in range(count):
        tf[k, :3, :3] = _rot(rng, 0.5)
        tf[k, :3, 3] = rng.uniform(-0.2, 0.2, 3)
        tf[k, 3, 3] = 1.0
    return tf


def _scene(n, seed):
    rng = np.random.default_rng(seed)
    means = (rng.normal(size=(n, 3)) * 0.6).astype(np.float32)
    scales = rng.uniform(0.01, 0.06, (n, 3)).astype(np.float32)
    q = rng.normal(size=(n, 4))
    quats = (q / np.linalg.norm(q, axis=-1, keepdims=True)).astype(np.float32)  # wxyz
    opac = rng.uniform(0.05, 0.95, n).astype(np.float32)
    return rng, means, scales, quats, opac


def _viewmats(B):
    vms = np.tile(np.eye(4, dtype=np.float32), (B, 1, 1))
    for b in range(B):
        vms[b, :3, 3] = [0.15 * b, -0.1, 4.0 + 0.3 * b]
    return vms


N = 3000
K = 3


def _ids(kind):
    ids = np.full(N, -1, np.int32)
    if kind == "slices":
        # block [0,256) uniform 0; [256,512) boundary at 300; [512,1024) uniform 1;
        # [1024,1280) boundary at 1100 between 1 and 2; [1280,1700) 2 then static to the end
        ids[0:300] = 0
        ids[300:1100] = 1
        ids[1100:1700] = 2
    else:  # "out_of_range": uniform and mixed blocks of ids >= num_transforms
        ids[0:256] = 0
        ids[256:512] = K  # a whole workgroup one past the last transform
        ids[512:600] = K + 7
        ids[600:800] = 1
        ids[1024:1280] = -1
        ids[1280:2000] = 2
    return ids


@pytest.mark.parametrize("B,batched_tf,kind", [(1, False, "slices"), (3, False, "slices"),
                                               (3, True, "slices"), (2, False, "out_of_range"),
                                               (2, True, "out_of_range")])
def test_transform_project_fwd_bwd_match_oracle(B, batched_tf, kind):
    _case(f"transforms B={B} batched_tf={batched_tf} ids={kind}")
    rng, means, scales, quats, opac = _scene(N, 40 + B + 3 * batched_tf)
    ids = _ids(kind)
    tf = _transforms(rng, B * K if batched_tf else K)
    vms = _viewmats(B)
    q = np.roll(quats, -1, axis=-1)  # xyzw, the kernel's layout
    total = B * N
    ref = O.project_fwd(means, scales, q, vms.reshape(-1, 4), opac, n=N, total=total,
                        img_shape=HW, f=F, c=C, transforms=tf, transform_ids=ids,
                        num_transforms=K)
    got = _ops.project_fwd(_t(means), _t(scales), _t(q), _t(vms).reshape(-1, 4), _t(opac),
                           _t(tf), _t(ids), n=N, total=total, num_transforms=K,
                           has_transforms=True, img_shape=HW, f=F, c=C, glob_scale=1.0,
                           clip_thresh=0.01)
    torch.cuda.synchronize()
    for label, a, r in zip(("xys", "depths", "radii", "conics", "nth", "cum"), got, ref):
        assert_bit_exact(_np(a).reshape(np.shape(r)), r, f"fwd {label}")
    xys, depths, radii, conics, nth, cum = ref
    assert (radii > 0).mean() > 0.5
    v_xy = rng.normal(size=(total, 2)).astype(np.float32)
    v_depth = rng.normal(size=total).astype(np.float32)
    v_conic = rng.normal(size=(total, 3)).astype(np.float32)
    rb = O.project_bwd(means, scales, q, vms.reshape(-1, 4), radii, conics, v_xy, v_depth,
                       v_conic, n=N, B=B, f=F, transforms=tf, transform_ids=ids,
                       num_transforms=K)
    args = (_t(means), _t(scales), _t(q), _t(vms).reshape(-1, 4), _t(radii), _t(conics),
            _t(v_xy), _t(v_depth), _t(v_conic), _t(tf), _t(ids))
    gb = _ops.project_bwd(*args, n=N, B=B, num_transforms=K, has_transforms=True, f=F,
                          glob_scale=1.0)
    torch.cuda.synchronize()
    for label, a, r in zip(("v_mean3d", "v_scale", "v_quat"), gb[:3], rb[:3]):
        assert_bit_exact(_np(a).reshape(r.shape), r, f"bwd {label}")
    _grad_compare(_np(gb[3]), rb[3], "v_viewmat")
    _grad_compare(_np(gb[4]).reshape(rb[4].shape), rb[4], "v_transforms")
    assert (_np(gb[4]).reshape(-1, 4, 4)[:, 3] == 0).all()
    if kind == "out_of_range":
        # only transforms 0..2 that some in-range id names receive gradient; nothing else moved
        assert np.abs(rb[4]).reshape(B, K, 16).max(-1).min() > 0
    if B > 1:
        # shared means / scales / quats: the folded backward equals the rows summed in image
        # order, bit for bit
        fb = _ops.project_bwd(*args, n=N, B=B, num_transforms=K, has_transforms=True, f=F,
                              glob_scale=1.0, fold=True)
        torch.cuda.synchronize()
        for label, a, r in zip(("v_mean3d", "v_scale", "v_quat"), fb[:3], rb[:3]):
            r = r.reshape(B, N, -1)
            acc = np.zeros_like(r[0])
            for b in range(B):
                acc = acc + r[b]
            assert_bit_exact(_np(a).reshape(acc.shape), acc, f"fold {label}")
        _grad_compare(_np(fb[4]).reshape(rb[4].shape), rb[4], "fold v_transforms")


def test_render_with_transforms_matches_oracle():
    """splax_amd.render with gaussian_transforms / gaussian_slices: image bit-exact and the
    transform gradient (through the blend backward and the projection VJP) within the bar of
    the oracle's chained custom-VJP rules."""
    import splax_amd

    _case("render with transforms")
    n = 2500
    rng, means, scales, quats, opac = _scene(n, 77)
    colors = rng.uniform(size=(n, 3)).astype(np.float32)
    bg = rng.uniform(size=3).astype(np.float32)
    vm = _viewmats(1)[0]
    slices = [(100, 700), (900, 2000)]
    tf = _transforms(rng, len(slices))
    ids = np.full(n, -1, np.int32)
    for k, (a, b) in enumerate(slices):
        ids[a:b] = k
    tft = _t(tf).requires_grad_(True)
    img, _ = splax_amd.render(_t(means), _t(scales), _t(quats), _t(colors), _t(opac[:, None]),
                              viewmat=_t(vm), background=_t(bg), img_shape=HW, f=F, c=C,
                              gaussian_transforms=tft, gaussian_slices=slices)
    w = rng.uniform(-1, 1, img.shape).astype(np.float32)
    (img * _t(w)).sum().backward()
    torch.cuda.synchronize()
    q = np.roll(quats, -1, axis=-1)
    xys, depths, radii, conics, nth, cum = O.project_fwd(
        means, scales, q, vm, opac, n=n, total=n, img_shape=HW, f=F, c=C, transforms=tf,
        transform_ids=ids, num_transforms=len(slices))
    rimg, Ts, fidx, _, _ = O.rasterize_fwd(colors, opac, opac, bg, xys, depths, radii, conics,
                                           cum, n=n, B=1, img_shape=HW)
    assert_bit_exact(_np(img).reshape(rimg.shape), rimg, "render image")
    v_colors, v_opac, v_xy, v_conic, _ = O.rasterize_bwd(
        colors, opac, opac, bg, xys, depths, radii, conics, cum, Ts, fidx, w.reshape(-1, 3),
        n=n, B_out=1, B_geom=1, img_shape=HW)
    rb = O.project_bwd(means, scales, q, vm, radii, conics, v_xy, np.zeros(n, np.float32),
                       v_conic, n=n, B=1, f=F, transforms=tf, transform_ids=ids,
                       num_transforms=len(slices))
    # the blend gradients are float sums on both sides; their chain into v_transforms too
    r = rel_fro(_np(tft.grad)[:, :3], rb[4][:, :3])
    assert r < 1e-4, f"v_transforms through render: relative Frobenius error {r:.3e}"
