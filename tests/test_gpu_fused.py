"""The fused render path (splat_render_fwd / splat_render_bwd, behind splax_amd.render) against
the two-call path (project then rasterize, each with its own backward) on the GPU.

The fused forward's projection also packs the blend records and forms the per-image depth range
(the sort's depth-range pass and the record pack do not run); the fused backward keeps the
per-item 2D cotangents in library scratch. Bars: projection outputs, kept lists, records
and the image bit-exact. The backward is deterministic (no sum depends on the GPU's scheduling),
so one camera's gradients are bit-exact as well, and two runs of one render agree bit for bit;
batched renders, whose two-call path sums the shared gaussians' per-camera gradients in torch
rather than in the library, are held to relative Frobenius 1e-5 plus allclose(rtol=1e-4,
atol=1e-5 * max|ref|).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import splax_amd
from conftest import assert_bit_exact, random_scene, rel_fro
from splax_amd import _lib, _ops
from splax_amd._rasterize import _rasterize_checked
from splax_amd.scenes import make_scene

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


def _grad_compare(got, ref, label, rel_tol=1e-5, elementwise=True):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    # non-finite entries (the reference's compensation rule gives NaN for a visible item whose
    # rho2 <= 0, and a NaN item cotangent makes the viewmat sum NaN) must agree in place and value
    bad = ~np.isfinite(ref)
    np.testing.assert_array_equal(~np.isfinite(got), bad, err_msg=f"{label}: non-finite entries")
    np.testing.assert_array_equal(got[bad], ref[bad], err_msg=f"{label}: non-finite values")
    got, ref = got[~bad], ref[~bad]
    if ref.size == 0:
        return
    r = rel_fro(got, ref)
    assert r < rel_tol, f"{label}: relative Frobenius error {r:.3e}"
    if not elementwise:
        return
    scale = float(np.abs(ref).max()) + 1e-30
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-5 * scale, err_msg=label)


def _two_call(p, vm, bg, cam, antialiased, render_depth, tf=None, slices=None):
    """splax.render composed from the public project and rasterize calls (the unfused path)."""
    tf_ids = None
    if tf is not None:
        tf_ids = splax_amd.transform_ids(p["means"].shape[-2], slices, device="cuda")
    xys, depths, radii, conics, _, cum = splax_amd.project(
        p["means"], p["scales"], p["quats"], vm, opacities=p["opac"], gaussian_transforms=tf,
        transform_ids=tf_ids, **cam)
    return _rasterize_checked(p["colors"], p["opac"], bg, xys, depths, radii, conics, cum,
                              cam["img_shape"], None, render_depth, compensate=antialiased)


def _stress_as_scene():
    """test_gpu_parity's extremes scene (huge, needle-thin and near-plane gaussians, opacities
    at the clamp and the threshold) as a Scene."""
    import importlib.util
    from pathlib import Path

    from splax_amd.scenes import Scene

    spec = importlib.util.spec_from_file_location(
        "gpu_parity", Path(__file__).with_name("test_gpu_parity.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    d = mod._stress_scene()
    return Scene(name="stress", means=d["means"], scales=d["scales"], quats=d["quats"],
                 colors=d["colors"], opacities=d["opac"], viewmats=d["vm"][None],
                 background=d["bg"], img_shape=d["img_shape"], f=d["f"],
                 targets=d["target"][None])


CASES = {
    "cfg0": dict(scene=lambda: make_scene(0), B=1),
    "cfg2_60k": dict(scene=lambda: make_scene(2, n=60_000), B=1),
    "cfg3_20k_B4": dict(scene=lambda: make_scene(3, n=20_000), B=4),
    "aa_depth": dict(scene=lambda: make_scene(1, n=30_000), B=1, antialiased=True, depth=True),
    "small_n": dict(scene=lambda: make_scene(0, n=700), B=2),  # depth range via the sort's pass
    "stress_aa_depth": dict(scene=_stress_as_scene, B=1, antialiased=True, depth=True),
}


@pytest.mark.parametrize("name", list(CASES))
def test_fused_render_equals_two_call_path(name):
    _case(f"fused render {name}")
    cfg = CASES[name]
    s = cfg["scene"]()
    B = cfg["B"]
    aa, rd = cfg.get("antialiased", False), cfg.get("depth", False)
    cam = dict(img_shape=s.img_shape, f=s.f, c=s.c)
    vms = s.viewmats[:B] if s.B >= B else np.stack([s.viewmats[0]] * B)
    vm_np = vms if B > 1 else vms[0]
    outs = []
    for fused in (True, False):
        p = {k: _t(v, grad=True) for k, v in (("means", s.means), ("scales", s.scales),
                                               ("quats", s.quats), ("colors", s.colors),
                                               ("opac", s.opacities))}
        vm = _t(vm_np, grad=True)
        bg = _t(s.background)
        if fused:
            img, depth = splax_amd.render(p["means"], p["scales"], p["quats"], p["colors"],
                                          p["opac"], viewmat=vm, background=bg, antialiased=aa,
                                          render_depth=rd, **cam)
        else:
            img, depth = _two_call(p, vm, bg, cam, aa, rd)
        w = torch.from_numpy(np.random.default_rng(7).uniform(-1, 1, img.shape)
                             .astype(np.float32)).cuda()
        loss = (img * w).sum()
        if rd:
            wd = torch.from_numpy(np.random.default_rng(8).uniform(-1, 1, depth.shape)
                                  .astype(np.float32)).cuda()
            loss = loss + (depth * wd).sum()
        loss.backward()
        torch.cuda.synchronize()
        grads = {k: _np(v.grad) for k, v in p.items()}
        grads["viewmat"] = _np(vm.grad)
        outs.append((_np(img), None if depth is None else _np(depth), grads))
    (fi, fd, fg), (ui, ud, ug) = outs
    assert_bit_exact(fi, ui, f"{name}/img")
    if rd:
        assert_bit_exact(fd, ud, f"{name}/depth")
    if B == 1:
        # one camera: the same records, lists, order and kernels on both paths, and no sum
        # whose order the GPU's scheduling decides
        for k in ug:
            assert_bit_exact(fg[k], ug[k], f"{name}/{k}")
        return
    # batched: the two-call path sums the shared gaussians' per-camera gradients in torch
    for k in ug:
        _grad_compare(fg[k], ug[k], f"{name}/{k}")


@pytest.mark.parametrize("name", ["cfg2_60k", "cfg3_20k_B4", "stress_aa_depth"])
def test_backward_is_deterministic(name):
    """Two runs of one render and its backward give every gradient bit for bit: the blend
    backward's per-record sums over a tile's four waves use two accumulator copies with at most
    two adds each (float addition commutes), the gather adds each item's intersections in
    emission order and the viewmat gradient is reduced in a fixed order."""
    _case(f"deterministic backward {name}")
    cfg = CASES[name]
    s = cfg["scene"]()
    B = cfg["B"]
    aa, rd = cfg.get("antialiased", False), cfg.get("depth", False)
    cam = dict(img_shape=s.img_shape, f=s.f, c=s.c)
    vms = s.viewmats[:B] if s.B >= B else np.stack([s.viewmats[0]] * B)
    runs = []
    for _ in range(2):
        p = {k: _t(v, grad=True) for k, v in (("means", s.means), ("scales", s.scales),
                                               ("quats", s.quats), ("colors", s.colors),
                                               ("opac", s.opacities))}
        vm = _t(vms if B > 1 else vms[0], grad=True)
        img, depth = splax_amd.render(p["means"], p["scales"], p["quats"], p["colors"],
                                      p["opac"], viewmat=vm, background=_t(s.background),
                                      antialiased=aa, render_depth=rd, **cam)
        w = torch.from_numpy(np.random.default_rng(7).uniform(-1, 1, img.shape)
                             .astype(np.float32)).cuda()
        loss = (img * w).sum()
        if rd:
            loss = loss + depth.sum()
        loss.backward()
        torch.cuda.synchronize()
        g = {k: _np(v.grad) for k, v in p.items()}
        g["viewmat"] = _np(vm.grad)
        runs.append(g)
    for k in runs[0]:
        assert_bit_exact(runs[1][k], runs[0][k], f"{name}/{k} run 2 vs run 1")


def test_fused_render_with_transforms_and_nested_batch():
    """Rigid transforms with per-world transforms on the outer axis, viewmats on both axes."""
    _case("fused render transforms + nested batch")
    n, H, W = 3000, 72, 96
    sc = random_scene(n, H, W, seed=51)
    slices = [(0, 1400), (1400, 2600)]
    tfs = np.tile(np.eye(4, dtype=np.float32), (2, 2, 1, 1))
    tfs[1, :, 0, 3] = 0.05
    tfs[0, 1, 1, 3] = -0.04
    vms = np.stack([np.stack([sc["vm"]] * 3)] * 2)
    vms[:, 1, 0, 3] += 0.1
    vms[:, 2, 1, 3] -= 0.1
    cam = dict(img_shape=(H, W), f=sc["f"], c=sc["c"])
    outs = []
    for fused in (True, False):
        p = {k: _t(sc[k], grad=True) for k in ("means", "scales", "quats", "colors", "opac")}
        tf = _t(tfs[:, None], grad=True)  # (2, 1, K, 4, 4): outer axis only
        vm = _t(vms)
        bg = _t(sc["bg"])
        if fused:
            img, _ = splax_amd.render(p["means"], p["scales"], p["quats"], p["colors"],
                                      p["opac"], viewmat=vm, background=bg,
                                      gaussian_transforms=tf, gaussian_slices=slices, **cam)
        else:
            # the two-call path takes one flat batch: fold the axes by hand
            tff = tf.expand(2, 3, 2, 4, 4).reshape(6, 2, 4, 4)
            img, _ = _two_call(p, vm.reshape(6, 4, 4), bg, cam, False, False, tf=tff,
                               slices=slices)
            img = img.reshape(2, 3, H, W, 3)
        assert img.shape == (2, 3, H, W, 3)
        w = torch.from_numpy(np.random.default_rng(3).uniform(-1, 1, img.shape)
                             .astype(np.float32)).cuda()
        (img * w).sum().backward()
        torch.cuda.synchronize()
        g = {k: _np(v.grad) for k, v in p.items()}
        g["transforms"] = _np(tf.grad)
        outs.append((_np(img), g))
    assert_bit_exact(outs[0][0], outs[1][0], "img")
    for k in outs[1][1]:
        _grad_compare(outs[0][1][k], outs[1][1][k], k)


def test_fused_forward_buffers_equal_two_call_buffers():
    """Through the tensor wrappers: projection outputs, sorted lists, bins, records and image of
    splat_render_fwd equal splat_project_fwd + splat_rasterize_fwd_keep bit for bit."""
    _case("fused forward buffers")
    s = make_scene(2, n=40_000)
    n = s.n
    q = _t(s.quats)
    args = (_t(s.means), _t(s.scales), q, _t(s.colors), _t(s.opacities).reshape(-1),
            _t(s.viewmats[0]), _t(s.background))
    tf = torch.zeros((1, 4, 4), device="cuda")
    ids = torch.full((1,), -1, device="cuda", dtype=torch.int32)
    for aa in (False, True):
        img, Ts, fidx, kept, _ = _ops.render_fwd(
            *args, tf, ids, n=n, B=1, num_transforms=1, has_transforms=False,
            img_shape=s.img_shape, f=s.f, c=s.c, glob_scale=1.0, clip_thresh=0.01,
            compensate=aa)
        proj = _ops.project_fwd(args[0], args[1], q, args[5], args[4], tf, ids, n=n, total=n,
                                num_transforms=1, has_transforms=False, img_shape=s.img_shape,
                                f=s.f, c=s.c, glob_scale=1.0, clip_thresh=0.01,
                                quats_wxyz=True)
        xys, depths, radii, conics, nth, cum = proj
        img2, Ts2, fidx2, k2, _ = _ops.rasterize_fwd_keep(
            args[3], args[4], args[4], args[6], xys, depths, radii, conics, cum, n=n, B=1,
            img_shape=s.img_shape, compensate=aa)
        torch.cuda.synchronize()
        for label, a, b in (("xys", kept.xys, xys), ("depths", kept.depths, depths),
                            ("radii", kept.radii, radii), ("conics", kept.conics, conics),
                            ("cum", kept.cum, cum), ("img", img, img2), ("Ts", Ts, Ts2),
                            ("fidx", fidx, fidx2), ("bins", kept.sort.bins, k2.bins),
                            ("records", kept.sort.records, k2.records)):
            assert_bit_exact(_np(a), _np(b), f"aa={aa} {label}")
        M = kept.sort.M
        assert M == k2.M and M > 0
        assert_bit_exact(_np(kept.sort.ids)[:M], _np(k2.ids)[:M], f"aa={aa} ids")
        assert_bit_exact(_np(kept.sort.pos)[:M], _np(k2.pos)[:M], f"aa={aa} pos")


def test_deferred_count_at_every_capacity():
    """The kept forwards (splat_render_fwd, splat_rasterize_fwd_keep) launch the sort and the
    blend before the intersection count reaches the host: the launches are sized by the list
    capacity and bounded on the device by the count, which the host settles after its last
    launch. Capacities below the count (0, half, one short) must report ERR_TOO_MANY with the
    count, after a truncated run that stays inside the buffers (the wrapper then retries with a
    larger capacity); capacities at or above it must give the same lists and image bit for bit."""
    _case("deferred count")
    s = make_scene(2, n=40_000)
    n = s.n
    q = _t(s.quats)
    args = (_t(s.means), _t(s.scales), q, _t(s.colors), _t(s.opacities).reshape(-1),
            _t(s.viewmats[0]), _t(s.background))
    tf = torch.zeros((1, 4, 4), device="cuda")
    tids = torch.full((1,), -1, device="cuda", dtype=torch.int32)
    key = str(args[0].device)

    def fused():
        img, Ts, fidx, kept, _ = _ops.render_fwd(
            *args, tf, tids, n=n, B=1, num_transforms=1, has_transforms=False,
            img_shape=s.img_shape, f=s.f, c=s.c, glob_scale=1.0, clip_thresh=0.01)
        return img, Ts, fidx, kept.sort, kept.cum

    def keep():
        xys, depths, radii, conics, _, cum = _ops.project_fwd(
            args[0], args[1], q, args[5], args[4], tf, tids, n=n, total=n, num_transforms=1,
            has_transforms=False, img_shape=s.img_shape, f=s.f, c=s.c, glob_scale=1.0,
            clip_thresh=0.01, quats_wxyz=True)
        img, Ts, fidx, ks, _ = _ops.rasterize_fwd_keep(
            args[3], args[4], args[4], args[6], xys, depths, radii, conics, cum, n=n, B=1,
            img_shape=s.img_shape)
        return img, Ts, fidx, ks, cum

    for label, call in (("render_fwd", fused), ("rasterize_fwd_keep", keep)):
        _ops._KEEP_CAPACITY[key] = 0
        ref = call()
        torch.cuda.synchronize()
        M = ref[3].M
        assert M > 1000 and M == int(ref[4][-1].item())
        assert _ops._KEEP_CAPACITY[key] == int(M * 1.25) + 1  # the first attempt fell short
        for cap in (0, M // 2, M - 1, M, M + 1, 3 * M):
            _case(f"deferred count {label} capacity {cap} (M = {M})")
            _ops._KEEP_CAPACITY[key] = cap
            got = call()
            torch.cuda.synchronize()
            # below the count the first attempt reports it and the wrapper retries larger
            assert _ops._KEEP_CAPACITY[key] == (cap if cap >= M else int(M * 1.25) + 1), cap
            assert got[3].M == M
            for name, a, b in (("img", got[0], ref[0]), ("Ts", got[1], ref[1]),
                               ("fidx", got[2], ref[2]), ("bins", got[3].bins, ref[3].bins)):
                assert_bit_exact(_np(a), _np(b), f"{label} cap={cap} {name}")
            assert_bit_exact(_np(got[3].ids)[:M], _np(ref[3].ids)[:M], f"{label} cap={cap} ids")
            assert_bit_exact(_np(got[3].pos)[:M], _np(ref[3].pos)[:M], f"{label} cap={cap} pos")
    _ops._KEEP_CAPACITY.pop(key, None)


@pytest.mark.parametrize("name", ["cfg2_60k", "cfg3_20k_B4", "aa_depth", "stress_aa_depth"])
def test_forward_only_render_equals_autograd_forward(name):
    """Under no_grad (or with no operand requiring grad) splax_amd.render runs splat_render_fwd
    with no position buffer, so the sort moves no emission positions: image, depth, sorted ids
    and bins must equal those of the forward that keeps everything for a backward, bit for
    bit."""
    _case(f"forward-only render {name}")
    cfg = CASES[name]
    s = cfg["scene"]()
    B = cfg["B"]
    aa, rd = cfg.get("antialiased", False), cfg.get("depth", False)
    cam = dict(img_shape=s.img_shape, f=s.f, c=s.c)
    vms = s.viewmats[:B] if s.B >= B else np.stack([s.viewmats[0]] * B)
    vm_np = vms if B > 1 else vms[0]
    outs = []
    for grad in (True, False):
        p = [_t(v, grad=grad) for v in (s.means, s.scales, s.quats, s.colors, s.opacities)]
        with torch.set_grad_enabled(grad):
            img, depth = splax_amd.render(*p, viewmat=_t(vm_np), background=_t(s.background),
                                          antialiased=aa, render_depth=rd, **cam)
        assert img.requires_grad == grad
        torch.cuda.synchronize()
        outs.append((_np(img), None if depth is None else _np(depth)))
    assert_bit_exact(outs[1][0], outs[0][0], f"{name}/img")
    if rd:
        assert_bit_exact(outs[1][1], outs[0][1], f"{name}/depth")
    # the library lists themselves, with and without positions
    q = _t(s.quats)
    args = (_t(s.means), _t(s.scales), q, _t(s.colors), _t(s.opacities).reshape(-1),
            _t(vm_np).reshape(-1, 4), _t(s.background))
    tf = torch.zeros((1, 4, 4), device="cuda")
    tids = torch.full((1,), -1, device="cuda", dtype=torch.int32)
    kept = []
    for backward in (True, False):
        r = _ops.render_fwd(*args, tf, tids, n=s.n, B=B, num_transforms=1, has_transforms=False,
                            img_shape=s.img_shape, f=s.f, c=s.c, glob_scale=1.0,
                            clip_thresh=0.01, compensate=aa, render_depth=rd, backward=backward)
        torch.cuda.synchronize()
        kept.append(r[3].sort)
    assert kept[1].pos is None and kept[0].M == kept[1].M > 0
    M = kept[0].M
    assert_bit_exact(_np(kept[1].ids)[:M], _np(kept[0].ids)[:M], f"{name}/ids")
    assert_bit_exact(_np(kept[1].bins), _np(kept[0].bins), f"{name}/bins")


@pytest.fixture
def _forced_wide_keys():
    from oracle import oracle as O

    _lib.set_wide_keys(True)
    O.set_wide_keys(True)
    yield O
    _lib.set_wide_keys(False)
    O.set_wide_keys(False)


@pytest.mark.parametrize("backward", [True, False])
def test_fused_forward_with_wide_keys_matches_oracle(_forced_wide_keys, backward):
    """The fused forward (deferred count, capacity-sized grids) on the 64-bit key path, forced as
    the reference's tests force it, with and without the positions a backward needs: sorted ids,
    bins and the image bit-exact against the oracle (its sort_and_bin and rasterize_fwd on the
    projection's outputs)."""
    O = _forced_wide_keys
    _case(f"fused forward wide keys backward={backward}")
    s = make_scene(2, n=40_000)
    q = _t(s.quats)
    args = (_t(s.means), _t(s.scales), q, _t(s.colors), _t(s.opacities).reshape(-1),
            _t(s.viewmats[0]), _t(s.background))
    tf = torch.zeros((1, 4, 4), device="cuda")
    tids = torch.full((1,), -1, device="cuda", dtype=torch.int32)
    img, Ts, fidx, kept, _ = _ops.render_fwd(
        *args, tf, tids, n=s.n, B=1, num_transforms=1, has_transforms=False,
        img_shape=s.img_shape, f=s.f, c=s.c, glob_scale=1.0, clip_thresh=0.01,
        backward=backward)
    torch.cuda.synchronize()
    xys, depths, radii, conics, cum = (_np(t) for t in (kept.xys, kept.depths, kept.radii,
                                                         kept.conics, kept.cum))
    rk, rid, rbins = O.sort_and_bin(xys, depths, radii, conics, s.opacities, cum, n=s.n, B=1,
                                    img_shape=s.img_shape)
    assert rk.dtype == np.int64  # the 64-bit key
    M = kept.sort.M
    assert M == len(rid) > 0
    assert_bit_exact(_np(kept.sort.ids)[:M], rid, "wide fused ids")
    assert_bit_exact(_np(kept.sort.bins), rbins, "wide fused bins")
    rimg, rT, ridx, _, rM = O.rasterize_fwd(s.colors, s.opacities, s.opacities, s.background,
                                            xys, depths, radii, conics, cum, n=s.n, B=1,
                                            img_shape=s.img_shape)
    assert rM == M
    assert_bit_exact(_np(img).reshape(rimg.shape), rimg, "wide fused img")
    if backward:
        assert_bit_exact(_np(fidx).reshape(ridx.shape), ridx, "wide fused final_idx")
        assert kept.sort.pos is not None
    else:
        assert Ts is None and fidx is None and kept.sort.pos is None


def test_render_fwd_cum_is_whole_at_every_capacity():
    """splat_render_fwd leaves cum_tiles_hit chunk-local in the projection and finalizes it in the
    emission (or, with no emission at capacity 0, in a separate pass): at capacity 0 (status 6),
    below the count (status 6) and above it, xys, radii and cum_tiles_hit equal the two-call
    projection's bit for bit, and num_intersects is the count."""
    import ctypes

    _case("render_fwd cum at every capacity")
    s = make_scene(2, n=40_000)
    n = s.n
    H, W = s.img_shape
    tiles = ((W + 15) // 16) * ((H + 15) // 16)
    dev = torch.device("cuda", 0)
    q, means, scales = _t(s.quats), _t(s.means), _t(s.scales)
    colors, opac = _t(s.colors), _t(s.opacities).reshape(-1)
    vm, bg = _t(s.viewmats[0]), _t(s.background)
    tf = torch.zeros((1, 4, 4), device="cuda")
    tids = torch.full((1,), -1, device="cuda", dtype=torch.int32)
    ref = _ops.project_fwd(means, scales, q, vm, opac, tf, tids, n=n, total=n, num_transforms=1,
                           has_transforms=False, img_shape=s.img_shape, f=s.f, c=s.c,
                           glob_scale=1.0, clip_thresh=0.01, quats_wxyz=True)
    torch.cuda.synchronize()
    M = int(ref[5][-1].item())
    assert n > 2 * 1024 and M > 0  # several projection chunks
    e = lambda *shape, dt=torch.float32: torch.empty(shape, device=dev, dtype=dt)  # noqa: E731
    p = _lib.ptr
    for cap in (0, M // 3, M, 2 * M):
        _case(f"render_fwd cum capacity {cap} (M = {M})")
        xys, depths, conics = e(n, 2), e(n), e(n, 3)
        radii, nth = e(n, dt=torch.int32), e(n, dt=torch.int32)
        cum = torch.full((n,), -7, device=dev, dtype=torch.int32)
        ids, pos = e(max(cap, 1), dt=torch.int32), e(max(cap, 1), dt=torch.int32)
        bins, recs = e(tiles, 2, dt=torch.int32), e(n, 16)
        order, Ts, fidx = e(tiles, dt=torch.int32), e(H, W), e(H, W, dt=torch.int32)
        img = e(H, W, 3)
        m = ctypes.c_int64(-1)
        st = _lib.lib().splat_render_fwd(
            _lib.stream_handle(dev), p(means), n, p(scales), n, p(q), n, p(vm), 4, p(opac), n,
            p(colors), n, p(bg), 1, p(tf), 1, p(tids), n, 1, 0, 1, H, W, s.f[0], s.f[1],
            s.c[0], s.c[1], 1.0, 0.01, 1, 0, p(xys), p(depths), p(radii), p(conics), p(nth),
            p(cum), cap, p(ids), p(pos), p(bins), p(recs), p(order), p(Ts), p(fidx), p(img),
            None, ctypes.byref(m), None, 0, None)
        torch.cuda.synchronize()
        assert st == (0 if cap >= M else _lib.ERR_TOO_MANY), (cap, st)
        assert m.value == M
        for label, got, want in (("xys", xys, ref[0]), ("radii", radii, ref[2]),
                                 ("num_tiles_hit", nth, ref[4]), ("cum", cum, ref[5])):
            assert_bit_exact(_np(got), _np(want), f"capacity {cap} {label}")


LOSS_CASES = {
    "cfg2_60k_mse": dict(scene=lambda: make_scene(2, n=60_000), B=1, loss="mse"),
    "cfg3_20k_B4_mse_pose": dict(scene=lambda: make_scene(3, n=20_000), B=4, loss="mse",
                                 pose=True),
    "cfg1_30k_aa_l1": dict(scene=lambda: make_scene(1, n=30_000), B=1, loss="l1",
                           antialiased=True),
    "cfg4_20k_B2_aa_l1": dict(scene=lambda: make_scene(4, n=20_000), B=2, loss="l1",
                              antialiased=True),
}


@pytest.mark.parametrize("name", list(LOSS_CASES))
def test_render_loss_equals_render_then_loss(name):
    """render_loss (the pixel loss fused into the blends) against render followed by the
    library's own loss (splat_mse_loss_* / splat_l1_loss_*): the image bit for bit, the loss
    value within one float ulp (both are double sums of exact terms, added in another order),
    and the gradients, scaled by a non-unit loss cotangent, within the bar."""
    from splax_amd.train import l1_loss, mse_loss

    _case(f"render_loss {name}")
    cfg = LOSS_CASES[name]
    s = cfg["scene"]()
    B, kind = cfg["B"], cfg["loss"]
    aa, pose = cfg.get("antialiased", False), cfg.get("pose", False)
    cam = dict(img_shape=s.img_shape, f=s.f, c=s.c, antialiased=aa)
    vm_np = s.viewmats[:B] if B > 1 else s.viewmats[0]
    tgt = _t(s.targets[:B] if B > 1 else s.targets[0])
    g = 2.5  # the loss cotangent
    outs = []
    for fused in (True, False):
        p = {k: _t(v, grad=True) for k, v in (("means", s.means), ("scales", s.scales),
                                               ("quats", s.quats), ("colors", s.colors),
                                               ("opac", s.opacities))}
        vm = _t(vm_np, grad=pose)
        bg = _t(s.background)
        if fused:
            loss, img = splax_amd.render_loss(*p.values(), target=tgt, loss=kind, viewmat=vm,
                                              background=bg, **cam)
            assert not img.requires_grad and loss.shape == ()
        else:
            img, _ = splax_amd.render(*p.values(), viewmat=vm, background=bg, **cam)
            loss = (l1_loss if kind == "l1" else mse_loss)(img, tgt)
        (loss * g).backward()
        torch.cuda.synchronize()
        grads = {k: _np(v.grad) for k, v in p.items()}
        if pose:
            grads["viewmat"] = _np(vm.grad)
        outs.append((_np(img), float(loss.item()), grads))
    (fi, fl, fg), (ui, ul, ug) = outs
    assert fi.shape == ((B,) if B > 1 else ()) + (*s.img_shape, 3)
    assert_bit_exact(fi, ui, f"{name}/img")
    d = fi.astype(np.float32) - _np(tgt)
    ref = np.float32((np.abs(d) if kind == "l1" else d.astype(np.float64) ** 2)
                     .astype(np.float64).sum() / d.size)
    ulp = float(np.spacing(ref))
    assert abs(fl - ul) <= ulp and abs(fl - float(ref)) <= ulp, (fl, ul, float(ref))
    for k in ug:
        _grad_compare(fg[k], ug[k], f"{name}/{k}")
    # without autograd the fused forward gives the same value
    with torch.no_grad():
        p = [_t(v) for v in (s.means, s.scales, s.quats, s.colors, s.opacities)]
        loss2, img2 = splax_amd.render_loss(*p, target=tgt, loss=kind, viewmat=_t(vm_np),
                                            background=_t(s.background), **cam)
    assert float(loss2.item()) == fl
    assert_bit_exact(_np(img2), fi, f"{name}/img (no grad)")


def test_render_loss_validates_its_target():
    s = make_scene(0, n=500)
    p = [_t(v) for v in (s.means, s.scales, s.quats, s.colors, s.opacities)]
    cam = dict(viewmat=_t(s.viewmats[0]), background=_t(s.background), img_shape=s.img_shape,
               f=s.f)
    with pytest.raises(ValueError, match="target must be float32 of the image's shape"):
        splax_amd.render_loss(*p, target=_t(s.targets), **cam)  # (1, H, W, 3) for one image
    with pytest.raises(ValueError, match="loss must be one of"):
        splax_amd.render_loss(*p, target=_t(s.targets[0]), loss="huber", **cam)


def test_render_loss_with_no_intersections():
    """M == 0 (the only gaussian behind the camera; and, second, one small gaussian whose lone
    tile bin stays empty): every pixel is the background, so the fused loss is the mean of
    |bg - target| or (bg - target)^2 over the image, and every gradient is exactly zero."""
    _case("render_loss M == 0")
    H = W = 48
    bg = np.array([0.2, 0.4, 0.6], np.float32)
    tgt = np.random.default_rng(4).uniform(size=(H, W, 3)).astype(np.float32)
    ones = dict(scales=np.full((1, 3), 0.02, np.float32),
                quats=np.array([[1.0, 0, 0, 0]], np.float32),
                colors=np.array([[1.0, 0, 0]], np.float32), opac=np.array([[0.9]], np.float32))
    for means, c in ((np.array([[0.0, 0.0, -3.0]], np.float32), None),
                     (np.array([[0.0, 0.0, 4.0]], np.float32), (40.0, 40.0))):
        for kind in ("mse", "l1"):
            p = {k: _t(v, grad=True) for k, v in ones.items()}
            mt = _t(means, grad=True)
            loss, img = splax_amd.render_loss(
                mt, p["scales"], p["quats"], p["colors"], p["opac"], target=_t(tgt), loss=kind,
                viewmat=_t(np.eye(4, dtype=np.float32)), background=_t(bg), img_shape=(H, W),
                f=(40.0, 40.0), c=c)
            np.testing.assert_array_equal(_np(img), np.broadcast_to(bg, (H, W, 3)))
            d = (np.broadcast_to(bg, (H, W, 3)) - tgt).astype(np.float64)
            ref = np.float32((d * d if kind == "mse" else np.abs(d)).sum() / d.size)
            assert abs(float(loss.item()) - float(ref)) <= float(np.spacing(ref))
            loss.backward()
            for g in (mt.grad, *(v.grad for v in p.values())):
                assert g is not None and (_np(g) == 0).all()


def test_render_log_loss_equals_render_log_then_l1():
    """render_log_loss (the training step's call: parameter map, antialiased render and L1 fused
    into the blends) against render_log followed by the library's L1 loss, over a batch of two
    cameras: image bit for bit, loss within one float ulp, gradients of the log / logit
    parameters within the bar."""
    from splax_amd.train import l1_loss, params_from_scene

    _case("render_log_loss")
    s = make_scene(4, n=20_000)
    B = 2
    tgt = _t(s.targets[:B])
    kw = dict(viewmat=_t(s.viewmats[:B]), background=_t(s.background), img_shape=s.img_shape,
              f=s.f, c=s.c, antialiased=True)
    outs = []
    for fused in (True, False):
        params = {k: v.clone().requires_grad_(True) for k, v in params_from_scene(s).items()}
        if fused:
            loss, img = splax_amd.render_log_loss(*params.values(), target=tgt, loss="l1", **kw)
        else:
            img, _ = splax_amd.render_log(*params.values(), **kw)
            loss = l1_loss(img, tgt)
        loss.backward()
        torch.cuda.synchronize()
        outs.append((_np(img), float(loss.item()), {k: _np(v.grad) for k, v in params.items()}))
    (fi, fl, fg), (ui, ul, ug) = outs
    assert_bit_exact(fi, ui, "img")
    assert abs(fl - ul) <= float(np.spacing(np.float32(ul))), (fl, ul)
    for k in ug:
        _grad_compare(fg[k], ug[k], f"log/{k}")
