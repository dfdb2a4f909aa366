"""splat_project_fwd_noalloc (the projection for callers that cannot allocate) through the C ABI.

Its outputs must equal splat_project_fwd's bit for bit (the same kernels; integer and float
outputs alike), on two calls in a row, the second with a smaller input, so that a stale chunk
total left in the shared fixed scratch by the first call would show. Sizes above the fixed
scratch are rejected before anything runs.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import assert_bit_exact
from splax_amd import _lib
from splax_amd.scenes import make_scene

pytestmark = pytest.mark.gpu

MAX_ITEMS = 65536 * 1024


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _call(name, s, vms, B, wxyz_quats):
    n = s.n
    total = B * n
    dev = torch.device("cuda", 0)
    means, scales, quats = _t(s.means), _t(s.scales), _t(wxyz_quats)
    vm, opac = _t(vms).reshape(-1, 4), _t(s.opacities).reshape(-1)
    tf = torch.zeros((1, 4, 4), device=dev)
    ids = torch.full((1,), -1, device=dev, dtype=torch.int32)
    outs = [torch.full((total, 2), -7.0, device=dev), torch.full((total,), -7.0, device=dev),
            torch.full((total,), -7, device=dev, dtype=torch.int32),
            torch.full((total, 3), -7.0, device=dev),
            torch.full((total,), -7, device=dev, dtype=torch.int32),
            torch.full((total,), -7, device=dev, dtype=torch.int32)]
    H, W = s.img_shape
    p = _lib.ptr
    with torch.cuda.device(dev):
        st = getattr(_lib.lib(), name)(
            _lib.stream_handle(dev), p(means), n, p(scales), n, p(quats), n, p(vm),
            vm.shape[0], p(opac), n, p(tf), 1, p(ids), n, 1, 0, total, H, W, s.f[0], s.f[1],
            s.c[0], s.c[1], 1.0, 0.01, *map(p, outs), 1)
    _lib.check(st, name)
    torch.cuda.synchronize()
    return [o.cpu().numpy() for o in outs]


@pytest.mark.parametrize("first,second", [((2, None, 1), (0, None, 1)),
                                          ((3, 200_000, 16), (1, None, 1))])
def test_noalloc_projection_equals_allocating_entry(first, second):
    """Two calls in a row (the second smaller); each equals splat_project_fwd bit for bit."""
    for cfg, n, B in (first, second):
        s = make_scene(cfg) if n is None else make_scene(cfg, n=n)
        vms = s.viewmats[:B] if s.B >= B else np.stack([s.viewmats[0]] * B)
        B = vms.shape[0]
        print(f"[case] noalloc config {cfg} n={s.n} B={B}", flush=True)
        got = _call("splat_project_fwd_noalloc", s, vms, B, s.quats)
        ref = _call("splat_project_fwd", s, vms, B, s.quats)
        for label, a, r in zip(("xys", "depths", "radii", "conics", "nth", "cum"), got, ref):
            assert_bit_exact(a, r, f"noalloc {label} (config {cfg}, B={B})")
        assert int(ref[5][-1]) > 0
    assert _lib.check_device() == 0


def test_noalloc_rejects_sizes_beyond_its_scratch():
    """More items than the fixed scratch covers: status 1 (invalid arguments), nothing runs."""
    lib = _lib.lib()
    n = 1 << 20
    total = MAX_ITEMS + n  # 65 images of 1Mi gaussians
    st = lib.splat_project_fwd_noalloc(None, 1, n, 1, n, 1, n, 1, 4, 1, n, 1, 1, 1, n, 1, 0,
                                       total, 64, 64, 50.0, 50.0, 32.0, 32.0, 1.0, 0.01, 16, 16,
                                       16, 16, 16, 16, 1)
    assert st == _lib.ERR_ARGS
    assert b"fixed scratch" in lib.splat_last_error()
