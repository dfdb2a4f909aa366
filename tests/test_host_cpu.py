"""Host-side logic and the C-ABI library, without a GPU.

- libsplat_hip.so loads and exports every entry point include/splat_hip.h declares, and the
  Python binding covers all of them.
- Argument validation mirrors the reference's ValueErrors (splax/_render.py:81-89,
  splax/_project/_project.py:126-132, splax/_rasterize/_sort/_sort.py:61-66).
- opacity_compensation closed form (splax/_project/_project.py:95-117), transform_ids, the
  synthetic scene generators and look_at.
- The product path refuses to run without a GPU (no CPU fallback).
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch

import splax_amd
from splax_amd import _lib
from splax_amd._rasterize import check_key_fits, key_layout
from splax_amd.scenes import make_scene
from splax_amd.utils import look_at

ROOT = Path(__file__).resolve().parents[1]


def _declared_symbols():
    text = (ROOT / "include" / "splat_hip.h").read_text()
    return sorted(set(re.findall(r"\b(splat_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    names = _declared_symbols()
    assert len(names) >= 10
    handle = ctypes.CDLL(str(_lib.LIB_PATH))
    for name in names:
        assert hasattr(handle, name), f"{name} declared in include/splat_hip.h but not exported"
    assert set(names) == set(_lib._SIGS), "Python binding and header disagree"
    lib = _lib.lib()
    assert lib.splat_abi_version() == _lib.ABI_VERSION
    assert isinstance(lib.splat_last_error(), bytes)


def test_binding_refuses_a_library_of_another_abi(monkeypatch):
    """lib() compares splat_abi_version() with the version the binding was written for, so a
    stale library exporting the same symbols raises instead of running under a changed
    contract."""
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "ABI_VERSION", _lib.ABI_VERSION + 1)
    with pytest.raises(ImportError, match="ABI version"):
        _lib.lib()


def test_no_cpu_fallback():
    if torch.cuda.is_available():
        pytest.skip("GPU present")
    x = torch.zeros((4, 3))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        splax_amd.project(x, x + 0.1, torch.tensor([[1.0, 0, 0, 0]]).repeat(4, 1), torch.eye(4),
                          opacities=torch.ones(4, 1), img_shape=(32, 32), f=(30.0, 30.0))


def test_transform_ids_and_validation():
    ids = splax_amd.transform_ids(10, [(2, 5), (7, 9)])
    assert ids.tolist() == [-1, -1, 0, 0, 0, -1, -1, 1, 1, -1]
    with pytest.raises(ValueError, match="outside"):
        splax_amd.transform_ids(10, [(5, 12)])
    with pytest.raises(ValueError, match="overlap"):
        splax_amd.transform_ids(10, [(0, 5), (4, 6)])
    x = torch.zeros((4, 3))
    with pytest.raises(ValueError, match="passed together"):
        splax_amd.render(x, x, torch.zeros(4, 4), x, torch.ones(4, 1), viewmat=torch.eye(4),
                         background=torch.zeros(3), img_shape=(16, 16), f=(10.0, 10.0),
                         gaussian_transforms=torch.zeros(1, 4, 4))
    with pytest.raises(ValueError, match="does not match"):
        splax_amd.render(x, x, torch.zeros(4, 4), x, torch.ones(4, 1), viewmat=torch.eye(4),
                         background=torch.zeros(3), img_shape=(16, 16), f=(10.0, 10.0),
                         gaussian_transforms=torch.zeros(2, 4, 4), gaussian_slices=[(0, 2)])


def test_opacity_compensation_closed_form():
    rng = np.random.default_rng(0)
    a = rng.uniform(0.1, 2.0, 50)
    c = rng.uniform(0.1, 2.0, 50)
    b = rng.uniform(-0.5, 0.5, 50) * np.sqrt(a * c)
    conics = torch.tensor(np.stack([a, b, c], -1))
    radii = torch.tensor((np.arange(50) % 7 != 0).astype(np.int32))[:, None]
    rho = splax_amd.opacity_compensation(conics, radii).numpy()
    eps = 0.3
    ref = np.sqrt(np.clip(1 - eps * (a + c) + eps ** 2 * (a * c - b * b), 0, 1))
    ref[np.arange(50) % 7 == 0] = 1.0
    np.testing.assert_allclose(rho, ref, rtol=1e-12)
    # an isotropic screen gaussian of variance s2: conic = 1/(s2 + 0.3) -> rho = s2 / (s2 + 0.3)
    s2 = 2.0
    iso = torch.tensor([[1 / (s2 + 0.3), 0.0, 1 / (s2 + 0.3)]], dtype=torch.float64)
    got = splax_amd.opacity_compensation(iso, torch.ones(1, 1)).item()
    assert abs(got - s2 / (s2 + 0.3)) < 1e-12


def test_key_layout_and_overflow_error():
    assert key_layout(1, 1080, 1920)["depth_bits"] == 18
    assert key_layout(16, 512, 512)["depth_bits"] == 17
    assert key_layout(4, 1060, 1600)["packed"]
    check_key_fits(4, 1060, 1600)
    lay = key_layout(8, 1080, 1920)  # 15 depth bits: the 64-bit key, which fits
    assert not lay["packed"] and not lay["overflow"]
    check_key_fits(8, 1080, 1920)
    with pytest.raises(ValueError, match="key overflow"):
        check_key_fits(1 << 20, 1080, 1920)  # 20 image + 13 tile bits


def test_scenes_deterministic_and_shaped():
    a = make_scene(0)
    b = make_scene(0)
    np.testing.assert_array_equal(a.means, b.means)
    np.testing.assert_array_equal(a.targets, b.targets)
    assert a.n == 10_000 and a.img_shape == (256, 256) and a.B == 1
    assert np.allclose(np.linalg.norm(a.quats, axis=-1), 1.0, atol=1e-6)
    assert (a.opacities > 0).all() and (a.opacities < 1).all()
    s3 = make_scene(3, n=1000)
    assert s3.B == 16 and s3.img_shape == (512, 512)
    s2 = make_scene(2, n=2000)
    assert s2.img_shape == (1080, 1920) and np.abs(s2.means).max() < 6


def test_look_at_properties():
    eyes = np.array([[0.5, 0.2, 4.0], [3.0, -2.0, 1.0]])
    vm = look_at(eyes, np.zeros(3), up=(0, 0, 1))
    for k in range(2):
        R = vm[k, :3, :3].astype(np.float64)
        np.testing.assert_allclose(R @ R.T, np.eye(3), atol=1e-6)
        np.testing.assert_allclose(np.linalg.det(R), 1.0, atol=1e-6)
        e = vm[k] @ np.r_[eyes[k], 1.0]
        np.testing.assert_allclose(e[:3], 0.0, atol=1e-5)  # the eye is the camera origin
        o = vm[k] @ np.array([0, 0, 0, 1.0])
        np.testing.assert_allclose(o[:2], 0.0, atol=1e-5)  # the target lies on the +z axis
        assert o[2] > 0


def test_abi_rejects_rows_that_are_neither_shared_nor_batched():
    """Operands must have n (shared) or B*n (batched) rows; the C ABI rejects anything else
    with status 1 before touching the device (so this runs without a GPU)."""
    import ctypes

    lib = _lib.lib()
    lib.splat_last_error.restype = ctypes.c_char_p
    f = ctypes.c_float
    n, total = 10, 30  # B = 3
    null = None

    def fwd(rows_means, rows_view):
        return lib.splat_project_fwd(null, null, rows_means, null, n, null, n, null, rows_view,
                                     null, n, null, 1, null, n, 1, 0, total, 16, 16, f(10.0),
                                     f(10.0), f(8.0), f(8.0), f(1.0), f(0.01), null, null, null,
                                     null, null, null, 1)

    assert fwd(20, 4) == 1  # between n and B*n
    assert b"rows" in lib.splat_last_error()
    assert fwd(5, 4) == 1   # fewer than n
    assert fwd(n, 8) == 1   # viewmat neither 4 nor 4B
    rc = lib.splat_rasterize_fwd(null, null, n, null, n, null, n, null, 2, null, null, null,
                                 null, null, n, 3, 16, 16, null, null, null, null)
    assert rc == 1 and b"background" in lib.splat_last_error()


def test_training_entry_points_validate_before_touching_the_device():
    """Adam / relocation arguments are checked on the host (no device call is made)."""
    lib = _lib.lib()
    groups = (_lib.AdamGroup * 9)()
    addr = ctypes.addressof(groups)
    assert lib.splat_adam_step(None, addr, 9, 0.9, 0.999, 1e-8, 0.0, 1) == _lib.ERR_ARGS
    assert lib.splat_adam_step(None, addr, 1, 0.9, 0.999, 1e-8, 0.0, 0) == _lib.ERR_ARGS
    assert lib.splat_adam_reset_rows(None, addr, 9, None, 4) == _lib.ERR_ARGS
    # the mapped update: an unknown map, and a quaternion group that is not rows of 4 floats or
    # not 16-byte aligned (fake device addresses: the checks precede any device call)
    one = (_lib.AdamGroup * 1)()
    one[0] = _lib.AdamGroup(1 << 20, 2 << 20, 3 << 20, 4 << 20, 8, 1e-3)
    bad_map = (ctypes.c_int32 * 1)(4)
    assert lib.splat_adam_step_mapped(None, ctypes.addressof(one), 1, ctypes.addressof(bad_map),
                                      0.9, 0.999, 1e-8, 0.0, 1) == _lib.ERR_ARGS
    assert b"unknown parameter map" in lib.splat_last_error()
    quat_map = (ctypes.c_int32 * 1)(3)
    one[0] = _lib.AdamGroup(1 << 20, 2 << 20, 3 << 20, 4 << 20, 6, 1e-3)
    assert lib.splat_adam_step_mapped(None, ctypes.addressof(one), 1, ctypes.addressof(quat_map),
                                      0.9, 0.999, 1e-8, 0.0, 1) == _lib.ERR_ARGS
    one[0] = _lib.AdamGroup((1 << 20) + 4, 2 << 20, 3 << 20, 4 << 20, 8, 1e-3)
    assert lib.splat_adam_step_mapped(None, ctypes.addressof(one), 1, ctypes.addressof(quat_map),
                                      0.9, 0.999, 1e-8, 0.0, 1) == _lib.ERR_ARGS
    assert b"16-byte aligned" in lib.splat_last_error()
    assert lib.splat_mcmc_relocate(None, None, None, None, None, None, 10, 63, 0.005, 1, None,
                                   None) == _lib.ERR_ARGS
    assert lib.splat_mcmc_relocate(None, None, None, None, None, None, 10, 51, 0.005, 1, None,
                                   None) == _lib.ERR_ARGS
    assert lib.splat_mcmc_compute_relocation(None, None, None, None, -1, 51, None,
                                             None) == _lib.ERR_ARGS
    assert lib.splat_mcmc_compute_relocation(None, None, None, None, 4, 0, None,
                                             None) == _lib.ERR_ARGS
    assert b"binomial" in lib.splat_last_error()


def _reference_fold_two_axes(x, outer: bool, inner: bool, A: int, Bn: int):
    """The reference's nested_vmap rule (splax/_batching.py:91-100) applied for an inner vmap of
    size Bn then an outer one of size A: per operand, the flat rows it hands the kernel."""
    # inner vmap: batched operands keep their rows, others stay shared
    if inner and outer:  # folded before and newly batched: reshape(sz * cur)
        return x.reshape(A * Bn, *x.shape[2:])
    if inner:  # folded before, not newly batched: tile over the outer axis
        return x.repeat(A, *(1,) * (x.ndim - 1))
    if outer:  # newly batched, not folded before: repeat each row over the inner axis
        return x.repeat_interleave(Bn, dim=0)
    return x  # shared


@pytest.mark.parametrize("outer,inner", [(True, True), (True, False), (False, True),
                                         (False, False)])
def test_nested_batch_fold_matches_reference_rule(outer, inner):
    """splax_amd._batching folds leading axes exactly as the reference's nested vmap flattens
    them: outer axis major, tile for inner-only, repeat for outer-only, shared otherwise."""
    from splax_amd._batching import batch_shape, fold

    A, Bn, n = 3, 4, 5
    base = torch.arange(n * 3, dtype=torch.float32).reshape(n, 3)
    full = base + 100 * torch.arange(A * Bn, dtype=torch.float32).reshape(A, Bn, 1, 1)
    if outer and inner:
        x, ref_in = full, full
    elif outer:
        x = full[:, :1]  # (A, 1, n, 3)
        ref_in = x[:, 0]
    elif inner:
        x = full[0]  # (Bn, n, 3): aligned from the right, the inner axis
        ref_in = x
    else:
        x, ref_in = base, base
    other = torch.zeros((A, Bn, 4, 4))  # a fully batched operand fixes the batch shape
    S = batch_shape({"x": (x, 2), "viewmat": (other, 2)})
    assert S == (A, Bn)
    got = fold(x, 2, S)
    want = _reference_fold_two_axes(ref_in, outer, inner, A, Bn)
    assert torch.equal(got, want)


def test_nested_batch_shapes_and_errors():
    from splax_amd._batching import batch_shape, fold

    x = torch.zeros((2, 1, 7, 3))
    v = torch.zeros((3, 4, 4))
    assert batch_shape({"x": (x, 2), "v": (v, 2)}) == (2, 3)
    assert fold(torch.zeros((1, 1, 7, 3)), 2, (2, 3)).shape == (7, 3)  # size-1 axes: shared
    assert fold(x, 2, ()).shape == x.shape
    with pytest.raises(ValueError, match="inconsistent batch shapes"):
        batch_shape({"x": (torch.zeros((2, 7, 3)), 2), "v": (torch.zeros((3, 4, 4)), 2)})


def test_size_one_background_is_shared():
    """A background of shape (1, 3) (or any size-1 leading dims) is one shared colour, not a
    batch axis: the reference reshapes it to (1, 3) inside rasterize
    (splax/_rasterize/_rasterize.py:131), so an unbatched render stays (H, W, 3)."""
    from splax_amd._batching import batch_shape, shared_background

    means, vm = torch.zeros((7, 3)), torch.eye(4)
    for bg in (torch.ones(3), torch.ones((1, 3)), torch.ones((1, 1, 3))):
        b = shared_background(bg)
        assert b.shape == (3,)
        assert batch_shape({"means": (means, 2), "viewmat": (vm, 2), "bg": (b, 1)}) == ()
    # a per-image background stays a batch axis
    assert shared_background(torch.ones((2, 3))).shape == (2, 3)
    assert batch_shape({"viewmat": (torch.zeros((2, 4, 4)), 2),
                        "bg": (shared_background(torch.ones((1, 3))), 1)}) == (2,)


_BUF = 256  # a stand-in device address (16-byte aligned; only the host checks run)


def test_missing_required_buffers_are_rejected():
    """A NULL required input or output of project_fwd / project_bwd / render_fwd /
    render_bwd is status 1 before any device work (the placeholder addresses are never
    dereferenced)."""
    lib = _lib.lib()
    lib.splat_last_error.restype = ctypes.c_char_p
    n, buf, f = 10, _BUF, ctypes.c_float
    m = ctypes.c_int64(0)

    def project_fwd(**null):
        a = dict(means=buf, scales=buf, quats=buf, viewmat=buf, opac=buf, xys=buf, depths=buf,
                 radii=buf, conics=buf, nth=buf, cum=buf)
        a.update(null)
        return lib.splat_project_fwd(None, a["means"], n, a["scales"], n, a["quats"], n,
                                     a["viewmat"], 4, a["opac"], n, None, 1, None, n, 1, 0, n,
                                     16, 16, f(10.0), f(10.0), f(8.0), f(8.0), f(1.0), f(0.01),
                                     a["xys"], a["depths"], a["radii"], a["conics"], a["nth"],
                                     a["cum"], 1)

    for k in ("means", "scales", "quats", "viewmat", "opac", "xys", "depths", "radii", "conics",
              "nth", "cum"):
        assert project_fwd(**{k: None}) == _lib.ERR_ARGS, k
        assert b"missing input or output buffer" in lib.splat_last_error(), k

    def project_bwd(**null):
        a = dict(means=buf, scales=buf, quats=buf, viewmat=buf, radii=buf, conics=buf, v_xy=buf,
                 v_conic=buf, v_mean=buf, v_scale=buf, v_quat=buf)
        a.update(null)
        return lib.splat_project_bwd(None, a["means"], n, a["scales"], n, a["quats"], n,
                                     a["viewmat"], 4, a["radii"], n, a["conics"], n, a["v_xy"],
                                     n, None, n, a["v_conic"], n, None, 1, None, n, 1, 0, 1,
                                     f(10.0), f(10.0), f(1.0), a["v_mean"], a["v_scale"],
                                     a["v_quat"], None, None, 1, 0)

    for k in ("means", "scales", "quats", "viewmat", "radii", "conics", "v_xy", "v_conic",
              "v_mean", "v_scale", "v_quat"):
        assert project_bwd(**{k: None}) == _lib.ERR_ARGS, k
        assert b"missing input or output buffer" in lib.splat_last_error(), k

    def render_fwd(colors=buf, background=buf, xys=buf, radii=buf):
        return lib.splat_render_fwd(None, buf, n, buf, n, buf, n, buf, 4, buf, n, colors, n,
                                    background, 1, None, 1, None, n, 1, 0, 1, 16, 16, 100.0,
                                    100.0, 8.0, 8.0, 1.0, 0.01, 1, 0, xys, buf, radii, buf, buf,
                                    buf, 0, buf, buf, buf, buf, buf, buf, buf, buf, None,
                                    ctypes.byref(m), None, 0, None)

    for k in ("xys", "radii"):
        assert render_fwd(**{k: None}) == _lib.ERR_ARGS, k
        assert b"missing input or output buffer" in lib.splat_last_error(), k
    for k in ("colors", "background"):
        assert render_fwd(**{k: None}) == _lib.ERR_ARGS, k
        assert b"missing input buffer" in lib.splat_last_error(), k

    def render_bwd(**null):
        a = dict(means=buf, radii=buf, v_means=buf, v_scales=buf, v_quats=buf, v_colors=buf,
                 v_opac=buf)
        a.update(null)
        return lib.splat_render_bwd(None, a["means"], n, buf, n, buf, n, buf, 4, buf, n, buf, n,
                                    buf, 1, None, 1, None, n, 1, 0, 1, 16, 16, 100.0, 100.0, 1.0,
                                    1, 0, buf, buf, a["radii"], buf, buf, buf, buf, buf, buf, buf,
                                    0, buf, buf, buf, 16, None, 0, a["v_means"], a["v_scales"],
                                    a["v_quats"], a["v_colors"], a["v_opac"], None, None, 0,
                                    None, 0, None, None)

    for k in ("means", "radii", "v_means", "v_scales", "v_quats", "v_colors", "v_opac"):
        assert render_bwd(**{k: None}) == _lib.ERR_ARGS, k
        assert b"missing" in lib.splat_last_error(), k

    def noise(**null):
        a = dict(means=buf, ls=buf, quats=buf, logit=buf, out=buf)
        a.update(null)
        return lib.splat_mcmc_inject_noise(None, a["means"], a["ls"], a["quats"], a["logit"], n,
                                           1.0, 0.005, 0, None, a["out"])

    for k in ("means", "ls", "quats", "logit", "out"):
        assert noise(**{k: None}) == _lib.ERR_ARGS, k
        assert b"inject_noise: missing arrays" in lib.splat_last_error(), k
    assert lib.splat_mcmc_inject_noise(None, buf, buf, buf, buf, -1, 1.0, 0.005, 0, None,
                                       buf) == _lib.ERR_ARGS
    assert b"negative count" in lib.splat_last_error()


def test_inject_noise_validates_shapes_before_the_device():
    from splax_amd import mcmc

    m, ls, q, lo = torch.zeros(4, 3), torch.zeros(4, 3), torch.zeros(4, 4), torch.zeros(4, 1)
    with pytest.raises(ValueError, match="values per"):
        mcmc.inject_noise(0, m, ls, q[:3], lo, 1.0)
    with pytest.raises(ValueError, match="noise must have shape"):
        mcmc.inject_noise(0, m, ls, q, lo, 1.0, noise=torch.zeros(4, 2))
    with pytest.raises(ValueError, match="out must be"):
        mcmc.inject_noise(0, m, ls, q, lo, 1.0, out=torch.zeros(4, 3, dtype=torch.float64))
    with pytest.raises(ValueError, match="float32"):
        mcmc.inject_noise(0, m.double(), ls, q, lo, 1.0)


def test_backward_requires_the_final_buffers():
    """A forward-only render may leave final_Ts / final_idx out; the backward entry points
    reject missing final buffers or a missing image cotangent with status 1 before touching the
    device (the placeholder addresses are never dereferenced)."""
    import ctypes

    lib = _lib.lib()
    lib.splat_last_error.restype = ctypes.c_char_p
    n = 10
    buf = 256  # a stand-in device address (8-byte aligned; only the host checks run)

    def bwd(final_Ts, final_idx, v_out):
        return lib.splat_rasterize_bwd(None, buf, n, buf, n, buf, n, buf, 1, buf, buf, buf, buf,
                                       buf, final_Ts, final_idx, v_out, 16, n, 1, 1, 16, 16, buf,
                                       buf, buf, buf)

    for args in ((None, buf, buf), (buf, None, buf), (buf, buf, None)):
        assert bwd(*args) == _lib.ERR_ARGS, args
        assert b"final_Ts, final_idx and the image cotangent" in lib.splat_last_error()


def test_forward_requires_the_image_output():
    """The blends write the image unconditionally, so a missing image output is status 1 before
    any launch (placeholder addresses are never dereferenced)."""
    import ctypes

    lib = _lib.lib()
    lib.splat_last_error.restype = ctypes.c_char_p
    n, buf = 10, 256
    m = ctypes.c_int64(0)
    rc = lib.splat_rasterize_fwd(None, buf, n, buf, n, buf, n, buf, 1, buf, buf, buf, buf, buf, n,
                                 1, 16, 16, buf, buf, None, ctypes.byref(m))
    assert rc == _lib.ERR_ARGS and b"missing image output" in lib.splat_last_error()


def test_fused_loss_arguments_are_checked():
    """splat_render_fwd / splat_render_bwd reject an unknown loss kind, and a fused loss without
    its target, value, image or cotangent, with status 1 before touching the device."""
    import ctypes

    lib = _lib.lib()
    lib.splat_last_error.restype = ctypes.c_char_p
    n, buf = 10, 256
    m = ctypes.c_int64(0)

    def fwd(kind, target, loss):
        return lib.splat_render_fwd(None, *([buf, n] * 8), buf, n, 1, 0, 1, 16, 16, 100.0, 100.0,
                                    8.0, 8.0, 1.0, 0.01, 1, 0, *([buf] * 6), 0, *([buf] * 9),
                                    ctypes.byref(m), target, kind, loss)

    def bwd(kind, target, img, v_loss):
        return lib.splat_render_bwd(None, buf, n, buf, n, buf, n, buf, 4, buf, n, buf, n, buf, 1,
                                    buf, 1, buf, n, 1, 0, 1, 16, 16, 100.0, 100.0, 1.0, 1, 0,
                                    *([buf] * 10), 0, buf, buf, None, 16, None, 0, *([buf] * 7),
                                    0, target, kind, img, v_loss)

    for rc in (fwd(3, buf, buf), bwd(3, buf, buf, buf), fwd(-1, buf, buf)):
        assert rc == _lib.ERR_ARGS and b"loss_kind must be" in lib.splat_last_error()
    for args in ((None, buf), (buf, None)):
        assert fwd(2, *args) == _lib.ERR_ARGS, args
        assert b"fused loss needs" in lib.splat_last_error()
    for args in ((None, buf, buf), (buf, None, buf), (buf, buf, None)):
        assert bwd(1, *args) == _lib.ERR_ARGS, args
        assert b"fused loss needs" in lib.splat_last_error()
    # without a fused loss the image cotangent is required as before
    assert bwd(0, None, None, None) == _lib.ERR_ARGS
    assert b"image cotangent are required" in lib.splat_last_error()


def test_opacity_compensation_backward_follows_the_reference_rules():
    """opacity_compensation's backward follows the reference's jax rules, like the oracle's
    compensation_vjp (which the fused antialiased blend follows): the same float32 cotangents
    inside the clip and NaN conic cotangents where rho2 <= 0 (sqrt' = 0.5 / rho times the
    cotangent, then the clip's 0 multiplier), where torch's own clamp rule would give 0."""
    from oracle import oracle as O

    rng = np.random.default_rng(3)
    n = 400
    a = rng.uniform(0.05, 3.0, n)
    c = rng.uniform(0.05, 3.0, n)
    b = rng.uniform(-0.9, 0.9, n) * np.sqrt(a * c)
    conics = np.stack([a, b, c], -1).astype(np.float32)
    conics[:5] = 0.0  # rho2 = 1: the upper clip's tie
    opac = rng.uniform(0.05, 1.0, n).astype(np.float32)
    vbo = rng.normal(size=n).astype(np.float32)
    _, rho2 = O.compensation_rho(conics)
    assert (rho2 < 0).sum() > 20 and ((rho2 > 0) & (rho2 < 1)).sum() > 100
    c_t = torch.tensor(conics, requires_grad=True)
    o_t = torch.tensor(opac, requires_grad=True)
    bo = o_t * splax_amd.opacity_compensation(c_t, torch.ones(n, 1, dtype=torch.int32))
    bo.backward(torch.tensor(vbo))
    v_o, v_c = O.compensation_vjp(vbo, opac, conics)
    g_c = c_t.grad.numpy()
    # NaN exactly where the oracle has it (every rho2 < 0 row); the rest within float32 rounding
    # of the two evaluations (torch's CPU kernels and numpy may differ by an ulp in rho)
    np.testing.assert_array_equal(np.isnan(g_c), np.isnan(v_c))
    assert np.isnan(g_c[rho2 < 0]).all() and not np.isnan(g_c[rho2 >= 0]).any()
    np.testing.assert_allclose(o_t.grad.numpy(), v_o, rtol=1e-6, atol=0)
    fin = ~np.isnan(v_c)
    np.testing.assert_allclose(g_c[fin], v_c[fin], rtol=1e-5, atol=1e-7)


def test_fused_loss_operands_are_validated_on_the_host():
    """The fused render loss's operands are checked before any library call: the loss kind, the
    target's size, dtype and device, and the loss value / cotangent scalar."""
    from splax_amd import _ops

    cpu = torch.device("cpu")
    ok = dict(target=torch.zeros(48), scalar=torch.zeros(()))
    _ops._check_loss_operands(_ops.LOSS_MSE, ok["target"], 1, 4, 4, cpu, ok["scalar"])
    bad = [
        (3, ok["target"], ok["scalar"], "loss_kind must be"),
        (_ops.LOSS_L1, None, ok["scalar"], "loss target must hold"),
        (_ops.LOSS_L1, torch.zeros(47), ok["scalar"], "loss target must hold"),
        (_ops.LOSS_L1, torch.zeros(48, dtype=torch.float64), ok["scalar"], "loss target"),
        (_ops.LOSS_MSE, ok["target"], None, "one float32"),
        (_ops.LOSS_MSE, ok["target"], torch.zeros(2), "one float32"),
    ]
    for kind, target, scalar, msg in bad:
        with pytest.raises(ValueError, match=msg):
            _ops._check_loss_operands(kind, target, 1, 4, 4, cpu, scalar)
    with pytest.raises(ValueError, match="loss must be one of"):
        x = torch.zeros((4, 3))
        splax_amd.render_loss(x, x, torch.zeros(4, 4), x, torch.ones(4, 1), target=x,
                              loss="l2", viewmat=torch.eye(4), background=torch.zeros(3),
                              img_shape=(16, 16), f=(10.0, 10.0))
