"""The library's device scratch on the GPU (the counterpart of splax/_cache.py): renders on warm
scratch, left by differently sized calls, equal renders on freshly cleared scratch; a call with
a new workload signature (B, n, tiles) releases the previous workload's buffers, as the
reference drops its scratch entry (splax/_cache.py:61-75); clear_cache() returns the rest and
forgets the kept-list capacity estimate. Mirrors the reference's scratch invariants
(tests/test_warp_rasterize.py:208-242) through the fused render with its loss and gradients."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import splax_amd
from conftest import assert_bit_exact, cached_scene, random_scene, rel_fro
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


def _render(sc, target):
    """render_loss (MSE) and its gradients: (image, loss, gradients)."""
    p = [_t(sc[k], grad=True) for k in ("means", "scales", "quats", "colors", "opac")]
    loss, img = splax_amd.render_loss(*p, target=_t(target), loss="mse", viewmat=_t(sc["vm"]),
                                      background=_t(sc["bg"]), img_shape=sc["img_shape"],
                                      f=sc["f"], c=sc["c"])
    loss.backward()
    torch.cuda.synchronize()
    return (img.cpu().numpy(), float(loss.item()),
            [t.grad.detach().cpu().numpy().astype(np.float64) for t in p])


def test_scratch_reuse_across_sizes():
    """Shrinking then growing workloads back to back, each rendered on the warm scratch and again
    after clear_cache(): images and loss bit for bit, gradients within the bar (the backward's
    per-record sums add in an order the GPU's scheduling decides)."""
    for n, H, W in ((200_000, 300, 400), (10_000, 256, 256), (100_000, 512, 512),
                    (10_000, 256, 256)):
        _case(f"scratch reuse n={n} {H}x{W}")
        sc = random_scene(n, H, W, seed=n)
        target = np.random.default_rng(n + 1).uniform(size=(H, W, 3)).astype(np.float32)
        warm = _render(sc, target)
        splax_amd.clear_cache()
        cold = _render(sc, target)
        assert_bit_exact(warm[0], cold[0], f"n={n} image")
        assert warm[1] == cold[1], (warm[1], cold[1])
        for k, (a, b) in enumerate(zip(warm[2], cold[2])):
            r = rel_fro(a, b)
            assert r < 1e-5, f"n={n} gradient {k}: {r:.2e}"


def test_clear_cache_returns_the_scratch():
    """A large render's scratch (sorted lists, records, per-intersection sums) is device memory
    the library holds until clear_cache(), which gives it back to the device."""
    _case("clear_cache releases")
    sc = random_scene(500_000, 1080, 1920, seed=1)
    target = np.zeros((1080, 1920, 3), np.float32)
    _render(sc, target)
    torch.cuda.synchronize()
    free_before, _ = torch.cuda.mem_get_info()
    splax_amd.clear_cache()
    free_after, _ = torch.cuda.mem_get_info()
    assert free_after - free_before > 32 << 20, (free_before, free_after)
    # and the library works again afterwards (scratch regrown on demand)
    img, loss, _ = _render(random_scene(5_000, 128, 128, seed=2),
                           np.zeros((128, 128, 3), np.float32))
    assert np.isfinite(loss) and img.shape == (128, 128, 3)


def _free_after_release() -> int:
    """Free device memory once torch's cached blocks are returned."""
    import gc

    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return torch.cuda.mem_get_info()[0]


def test_new_workload_signature_releases_the_scratch():
    """After a config-4-size training render (3M gaussians, four 1600x1060 cameras, 31M
    intersections) the library holds gigabytes of sort and gradient scratch; the next call with
    another workload signature (a config-0 render) drops it first, and its kept-list capacity
    estimate starts again from that call's count. clear_cache() then returns the small
    workload's scratch and forgets the estimate."""
    _case("scratch dropped on a new workload signature")
    s = cached_scene(4)
    p = [_t(a, grad=True) for a in (s.means, s.scales, s.quats, s.colors, s.opacities)]
    loss, _ = splax_amd.render_loss(*p, target=_t(s.targets), loss="l1",
                                    viewmat=_t(s.viewmats), background=_t(s.background),
                                    img_shape=s.img_shape, f=s.f, c=s.c, antialiased=True)
    loss.backward()
    key = str(p[0].device)
    big_cap = _ops._KEEP_CAPACITY[key]
    assert big_cap > 30_000_000
    del p, loss
    free_big = _free_after_release()
    small = random_scene(10_000, 256, 256, seed=4)
    img, _, _ = _render(small, np.zeros((256, 256, 3), np.float32))
    assert img.shape == (256, 256, 3)
    small_cap = _ops._KEEP_CAPACITY[key]
    assert 0 < small_cap < big_cap // 100, (small_cap, big_cap)
    free_small = _free_after_release()
    # the intersection-sized sort buffers and per-intersection sums alone are several GB
    assert free_small - free_big > 2 << 30, (free_big, free_small)
    splax_amd.clear_cache()
    assert key not in _ops._KEEP_CAPACITY
    assert _free_after_release() >= free_small
