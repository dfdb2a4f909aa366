"""GPU parity of the training-step entry points against the CPU oracle (oracle/train_oracle.py).

- Adam (splat_adam_step) and the moment reset: bit-exact, both sides run the same float32
  sequence.
- compute_relocation: within one float32 ulp (both evaluate in double and round once; the
  double pow / log of the two math libraries may differ in the last double bit).
- relocate: sources, reset rows and every copied parameter bit-exact (the draw is integer
  arithmetic); relocated opacity logits and log scales within one float32 ulp. At the config-4
  size (3M gaussians) through size-independent properties: determinism, alive sources, rows
  sharing a source carry identical values, r copies of the new opacity compose to the old one,
  and the draw frequencies follow opacity.
- inject_noise: with the caller's normals, the displacement within 1e-5 relative Frobenius (and
  per element within 1e-5 of the largest) of the oracle's float64 transform (float32 exp,
  sigmoid and rotation on the device, double in the oracle); with the device's own Philox draw,
  the same bar against the oracle's float64 Box-Muller of the same Philox words (the stream
  itself is pinned); at 1M gaussians the normals' moments, correlations and Kolmogorov-Smirnov
  distance; determinism per key; in place equal to out of place; the reference's opacity check
  (tests/test_mcmc.py:102-114); and the trainer's noise equal to the call on its parameters.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from conftest import assert_bit_exact
from oracle import train_oracle as T
from splax_amd import _lib, mcmc, optim

pytestmark = pytest.mark.gpu


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _np(t):
    return t.detach().cpu().numpy()


def _case(msg):
    print(f"[case] {msg}", flush=True)


def _max_ulp(a, b):
    a = np.ascontiguousarray(a, np.float32).reshape(-1).view(np.int32).astype(np.int64)
    b = np.ascontiguousarray(b, np.float32).reshape(-1).view(np.int32).astype(np.int64)
    a = np.where(a < 0, -(a & 0x7FFFFFFF), a)  # monotone integer order of the floats
    b = np.where(b < 0, -(b & 0x7FFFFFFF), b)
    return int(np.abs(a - b).max()) if a.size else 0


GROUPS = {"means": 3, "log_scales": 3, "quats": 4, "colors_logit": 3, "opac_logit": 1}
LRS = {"means": optim.exponential_decay(1.6e-3, 30000, 0.01), "log_scales": 5e-3,
       "quats": 1e-3, "colors_logit": 1e-2, "opac_logit": 5e-2}


def _params(n, seed):
    rng = np.random.default_rng(seed)
    return {k: rng.normal(size=(n, w)).astype(np.float32) for k, w in GROUPS.items()}


def _misaligned(a: np.ndarray) -> torch.Tensor:
    """A device copy of ``a`` that starts one float into its allocation (4-byte aligned only)."""
    flat = torch.empty(a.size + 1, device="cuda", dtype=torch.float32)
    flat[1:] = _t(a.reshape(-1))
    return flat[1:].view(a.shape)


@pytest.mark.parametrize("n,misalign", [(1, False), (1000, False), (10007, False),
                                        (10007, True)])
def test_adam_step_bit_exact(n, misalign):
    """Four steps and a row reset bit-exact against the oracle, also for parameters that start
    off a 16-byte boundary (views one float into their allocation)."""
    _case(f"adam n={n} misalign={misalign}")
    rng = np.random.default_rng(n)
    ref = _params(n, n)
    mu = {k: np.zeros_like(v) for k, v in ref.items()}
    nu = {k: np.zeros_like(v) for k, v in ref.items()}
    dev = {k: (_misaligned(v) if misalign else _t(v)) for k, v in ref.items()}
    opt = optim.Adam(dev, LRS)
    for step in range(1, 5):
        grads = {k: (rng.normal(size=v.shape) * 10.0 ** rng.uniform(-6, 1)).astype(np.float32)
                 for k, v in ref.items()}
        grads["quats"][: n // 3] = 0.0
        for k in ref:
            lr = LRS[k](step - 1) if callable(LRS[k]) else LRS[k]
            ref[k], mu[k], nu[k] = T.adam_step(ref[k], grads[k], mu[k], nu[k], lr=lr,
                                               count=step)
        opt.step({k: _t(g) for k, g in grads.items()})
        torch.cuda.synchronize()
        for k in ref:
            assert_bit_exact(_np(dev[k]), ref[k], f"adam {k} step {step}")
            assert_bit_exact(_np(opt.mu[k]), mu[k], f"adam mu {k} step {step}")
            assert_bit_exact(_np(opt.nu[k]), nu[k], f"adam nu {k} step {step}")
    reset = rng.uniform(size=n) < 0.3
    opt.reset_rows(_t(reset))
    torch.cuda.synchronize()
    for k in ref:
        m2, n2 = T.reset_rows(mu[k], nu[k], reset)
        assert_bit_exact(_np(opt.mu[k]), m2, f"reset mu {k}")
        assert_bit_exact(_np(opt.nu[k]), n2, f"reset nu {k}")


def test_adam_rejects_bad_groups():
    x = torch.zeros((4, 3), device="cuda")
    with pytest.raises(ValueError):
        optim.Adam({"a": x}, {"b": 1e-3})
    opt = optim.Adam({"a": x}, {"a": 1e-3})
    with pytest.raises(ValueError):
        opt.step({"a": torch.zeros((4, 2), device="cuda")})


def test_compute_relocation_within_one_ulp():
    _case("compute_relocation")
    rng = np.random.default_rng(0)
    n = 5000
    opac = rng.uniform(0.005, 0.999, n).astype(np.float32)
    scales = rng.uniform(0.001, 0.5, (n, 3)).astype(np.float32)
    ratios = rng.integers(1, 60, n).astype(np.float32)
    ratios[:10] = [0.4, 1.5, 2.5, 50.5, 51.0, 52.0, 1e9, -3.0, float("nan"), 1.0]
    ro, rs = T.compute_relocation(opac, scales, ratios, n_max=51)
    go, gs = mcmc.compute_relocation(_t(opac), _t(scales), _t(ratios), mcmc.make_binoms(51))
    assert _max_ulp(_np(go), ro) <= 1
    assert _max_ulp(_np(gs), rs) <= 1


def _scene(n, dead_frac, seed):
    rng = np.random.default_rng(seed)
    means = rng.uniform(-3, 3, (n, 3)).astype(np.float32)
    log_scales = rng.normal(-5, 0.7, (n, 3)).astype(np.float32)
    quats = rng.normal(size=(n, 4)).astype(np.float32)
    colors = rng.normal(size=(n, 3)).astype(np.float32)
    logit = rng.normal(1.0, 1.5, n).astype(np.float32)
    dead = rng.uniform(size=n) < dead_frac
    logit[dead] = rng.uniform(-25.0, -5.3, int(dead.sum())).astype(np.float32)
    logit[:8] = [-5.2933, -5.2932, -5.29, -5.3, -30.0, -100.0, 0.0, 12.0]  # near the threshold
    return means, log_scales, quats, colors, logit


def _relocate_gpu(seed, arrays, n_max=51, min_opacity=0.005):
    dev = [_t(a) for a in arrays]
    reset, source = mcmc.relocate_(seed, *dev, mcmc.make_binoms(n_max), min_opacity,
                                   return_source=True)
    torch.cuda.synchronize()
    return [_np(d) for d in dev], _np(source), _np(reset)


@pytest.mark.parametrize("n,dead_frac,seed", [(1, 0.0, 0), (7, 1.0, 1), (4096, 0.05, 2),
                                              (50000, 0.2, 3), (50000, 0.97, 4)])
def test_relocate_matches_oracle(n, dead_frac, seed):
    _case(f"relocate n={n} dead={dead_frac} seed={seed}")
    arrays = tuple(np.ascontiguousarray(a[:n]) for a in _scene(max(n, 8), dead_frac, seed))
    if dead_frac == 1.0:
        arrays[4][:] = -40.0  # nothing alive: every row draws row 0
    key = 0x9E3779B97F4A7C15 ^ seed
    rm, rls, rq, rc, rl, rsrc, rreset = T.relocate(key, *arrays, n_max=51)
    (gm, gls, gq, gc, gl), gsrc, greset = _relocate_gpu(key, arrays)
    assert_bit_exact(gsrc, rsrc, "source")
    assert np.array_equal(greset, rreset), "reset rows"
    assert_bit_exact(gm, rm, "means")
    assert_bit_exact(gq, rq, "quats")
    assert_bit_exact(gc, rc, "logit_colors")
    assert _max_ulp(gl, rl) <= 1, "logit_opacities"
    assert _max_ulp(gls, rls) <= 1, "log_scales"


def test_relocate_functional_equals_in_place_and_validates():
    arrays = _scene(3000, 0.3, 9)
    dev = [_t(a) for a in arrays]
    binoms = mcmc.make_binoms(51)
    new, reset = mcmc.relocate(5, *dev, binoms)
    for d, a in zip(dev, arrays):  # inputs untouched
        assert_bit_exact(_np(d), a, "relocate input")
    (gm, gls, gq, gc, gl), _, greset = _relocate_gpu(5, arrays)
    for x, y in zip(new, (gm, gls, gq, gc, gl)):
        assert_bit_exact(_np(x), y, "functional vs in place")
    assert np.array_equal(_np(reset), greset)
    with pytest.raises(ValueError):
        mcmc.relocate_(1, dev[0], dev[1], dev[2][:, :3].contiguous(), dev[3], dev[4], binoms)
    with pytest.raises(ValueError):
        mcmc.relocate_(1, *dev, mcmc.make_binoms(70))
    ref = [[math.comb(i, k) if k <= i else 0 for k in range(6)] for i in range(6)]
    assert mcmc.make_binoms(6).tolist() == ref


def test_relocate_config4_size_properties():
    """3M gaussians (config 4) with 5% dead: size-independent properties of the result."""
    n = 3_000_000
    _case(f"relocate properties n={n}")
    arrays = _scene(n, 0.05, 11)
    (gm, gls, gq, gc, gl), src, reset = _relocate_gpu(77, arrays)
    (gm2, gls2, gq2, gc2, gl2), src2, reset2 = _relocate_gpu(77, arrays)
    for x, y in zip((gm, gls, gq, gc, gl, src, reset), (gm2, gls2, gq2, gc2, gl2, src2, reset2)):
        assert np.array_equal(x, y), "relocation is deterministic"
    means, log_scales, quats, colors, logit = arrays
    opac = T.sigmoid(logit)
    dead = opac <= np.float32(0.005)
    idx = np.arange(n)
    assert np.array_equal(src[~dead], idx[~dead])
    d = idx[dead]
    s = src[dead]
    assert (~dead[s]).all(), "sources are alive"
    assert np.array_equal(gm[d], means[s]) and np.array_equal(gq[d], quats[s])
    assert np.array_equal(gc[d], colors[s])
    counts = np.bincount(s, minlength=n)
    assert np.array_equal(reset, dead | (counts > 0))
    keep = ~reset
    for x, y in zip((gm, gls, gq, gc, gl), arrays):
        assert np.array_equal(x[keep], y[keep])
    assert np.array_equal(gl[d], gl[s]) and np.array_equal(gls[d], gls[s])
    # r = counts + 1 copies at the new opacity composite to the old opacity
    srcs = np.nonzero(counts)[0]
    r = np.minimum(counts[srcs] + 1, 51).astype(np.float64)
    new_o = 1.0 / (1.0 + np.exp(-gl[srcs].astype(np.float64)))
    unclipped = new_o > 0.0051
    comp = 1.0 - (1.0 - new_o) ** r
    np.testing.assert_allclose(comp[unclipped], opac[srcs][unclipped], rtol=2e-5)
    # draw frequencies by opacity decile of the alive rows follow the decile's opacity mass
    alive = idx[~dead]
    order = alive[np.argsort(opac[alive], kind="stable")]
    bins = np.array_split(order, 10)
    which = np.empty(n, np.int64)
    for b, rows in enumerate(bins):
        which[rows] = b
    hist = np.bincount(which[s], minlength=10)
    mass = np.array([opac[rows].astype(np.float64).sum() for rows in bins])
    exp = mass / mass.sum() * d.size
    chi2 = float(((hist - exp) ** 2 / exp).sum())
    assert chi2 < 27.9, (hist, exp, chi2)  # p = 0.001 at 9 degrees of freedom
    assert _lib.check_device() == 0


def _noise_inputs(n, seed):
    rng = np.random.default_rng(seed)
    means = rng.normal(scale=2.0, size=(n, 3)).astype(np.float32)
    ls = rng.normal(loc=-2.0, scale=0.8, size=(n, 3)).astype(np.float32)
    q = (rng.normal(size=(n, 4)) * rng.uniform(0.3, 2.0, size=(n, 1))).astype(np.float32)
    logit = rng.normal(loc=-3.0, scale=3.0, size=(n, 1)).astype(np.float32)
    return means, ls, q, logit


def _assert_displacement(got, ref, means, label):
    """got = fl32(means + d) against ref = means + d_ref in double: the final rounding costs at
    most half an ulp of the sum (2^-24 |ref| up to the ulp's own rounding); what exceeds it is
    the displacement's error, held to 1e-5 relative Frobenius and per element to 1e-5 of the
    largest displacement."""
    got = np.asarray(got, np.float64)
    d_ref = np.asarray(ref, np.float64) - means
    excess = np.maximum(np.abs(got - ref) - 2.0**-24 * (1.0 + 2.0**-20) * np.abs(ref), 0.0)
    err = np.linalg.norm(excess) / max(np.linalg.norm(d_ref), 1e-30)
    assert err < 1e-5, (label, err)
    assert (excess <= 1e-5 * np.abs(d_ref).max()).all(), label


@pytest.mark.parametrize("n,seed", [(1, 0), (1000, 1), (65_537, 2)])
def test_inject_noise_given_normals(n, seed):
    _case(f"inject_noise given normals n={n} seed={seed}")
    means, ls, q, logit = _noise_inputs(n, seed)
    z = np.random.default_rng(seed + 100).normal(size=(n, 3)).astype(np.float32)
    got = _np(mcmc.inject_noise(0, _t(means), _t(ls), _t(q), _t(logit), 0.05, 0.01,
                                noise=_t(z)))
    ref = T.inject_noise(means, ls, q, logit, 0.05, z, 0.01)
    assert got.shape == (n, 3)
    _assert_displacement(got, ref, means.astype(np.float64), f"n={n}")
    assert _lib.check_device() == 0


@pytest.mark.parametrize("n,key", [(1, 5), (4099, 0x0123_4567_89AB_CDEF)])
def test_inject_noise_drawn_normals_follow_the_philox_stream(n, key):
    _case(f"inject_noise drawn normals n={n} key={key:#x}")
    means, ls, q, logit = _noise_inputs(n, 7)
    got = _np(mcmc.inject_noise(key, _t(means), _t(ls), _t(q), _t(logit), 0.5))
    ref = T.inject_noise(means, ls, q, logit, 0.5, T.noise_normals(key, n))
    _assert_displacement(got, ref, means.astype(np.float64), f"n={n}")


def test_inject_noise_normals_law_at_1m():
    """Identity rotation and unit scales: the displacement is z * gate * scaler exactly up to
    float32 rounding, so z is recovered and tested against the standard normal law."""
    from scipy import stats

    _case("inject_noise normal law n=1M")
    n = 1 << 20
    means = torch.zeros((n, 3), device="cuda")
    ls = torch.zeros((n, 3), device="cuda")
    q = torch.tensor([1.0, 0.0, 0.0, 0.0], device="cuda").repeat(n, 1)
    logit = torch.full((n, 1), -40.0, device="cuda")
    out = _np(mcmc.inject_noise(11, means, ls, q, logit, 1.0, min_opacity=0.5))
    gate = 1.0 / (1.0 + math.exp(-100.0 * (0.5 - 1.0 / (1.0 + math.exp(40.0)))))
    z = out.astype(np.float64) / gate
    # float32 log / sqrt / cos / sin of the same exact uniforms: 1.7e-6 at most, measured
    np.testing.assert_allclose(z, T.noise_normals(11, n), rtol=1e-5, atol=5e-6)
    assert np.abs(z.mean(axis=0)).max() < 5 * n ** -0.5
    assert np.abs(z.var(axis=0) - 1.0).max() < 5 * (2.0 / n) ** 0.5
    assert np.abs(np.corrcoef(z.T) - np.eye(3)).max() < 5 * n ** -0.5
    for k in range(3):
        assert stats.kstest(z[:, k], "norm").pvalue > 1e-3, k
    assert np.isfinite(z).all() and np.abs(z).max() < 5.8  # u >= 2^-24 bounds |z| by 5.77


def test_inject_noise_determinism_in_place_and_opacity():
    _case("inject_noise determinism / in place / opacity")
    n = 400
    means = torch.zeros((n, 3), device="cuda")
    ls = torch.full((n, 3), math.log(0.1), device="cuda")
    q = torch.tensor([1.0, 0.0, 0.0, 0.0], device="cuda").repeat(n, 1)
    logit = torch.cat([torch.full((200, 1), -5.0), torch.full((200, 1), 8.0)]).cuda()
    a = mcmc.inject_noise(2, means, ls, q, logit, scaler=100.0)
    b = mcmc.inject_noise(2, means, ls, q, logit, scaler=100.0)
    c = mcmc.inject_noise(3, means, ls, q, logit, scaler=100.0)
    assert torch.equal(a, b) and not torch.equal(a, c)
    disp = np.linalg.norm(_np(a), axis=1)
    assert disp[:200].mean() > 10 * disp[200:].mean() + 1e-6  # tests/test_mcmc.py:102-114
    m2 = means.clone()
    r = mcmc.inject_noise(2, m2, ls, q, logit, scaler=100.0, out=m2)
    assert r.data_ptr() == m2.data_ptr() and torch.equal(m2, a)
    empty = torch.zeros((0, 3), device="cuda")
    assert mcmc.inject_noise(0, empty, empty, torch.zeros((0, 4), device="cuda"),
                             torch.zeros((0, 1), device="cuda"), 1.0).shape == (0, 3)
    assert _lib.check_device() == 0


def test_train_step_noise_equals_the_call():
    """TrainStep(noise_lr > 0) adds inject_noise at means-lr(step) * noise_lr after the Adam
    update and relocation (scripts/train_lego.py:277-284): one step with noise equals one step
    without, followed by the call with the trainer's key."""
    from splax_amd.scenes import make_scene
    from splax_amd.train import TrainStep, params_from_scene

    _case("train step with noise n=20000")
    scene = make_scene(4, n=20_000)
    kw = dict(viewmats=_t(scene.viewmats), targets=_t(scene.targets),
              background=_t(scene.background), img_shape=scene.img_shape, f=scene.f, seed=9)
    noisy = TrainStep(params_from_scene(scene), noise_lr=5e5, **kw)
    plain = TrainStep(params_from_scene(scene), **kw)
    noisy()
    plain()
    p = plain.params
    want = mcmc.inject_noise((9 << 32) ^ 1, p["means"], p["log_scales"], p["quats"],
                             p["opac_logit"], plain.means_lr(1) * 5e5, plain.min_opacity)
    for k in p:
        if k != "means":
            assert torch.equal(noisy.params[k], p[k]), k
    assert torch.equal(noisy.params["means"], want)
    assert not torch.equal(want, p["means"])
    assert _lib.check_device() == 0


def test_train_step_config4_small():
    """The config-4 step end to end at 20k gaussians: finite loss, every group updated, dead
    rows relocated and their moments zeroed, and the loss falls over a few steps."""
    from splax_amd.scenes import make_scene
    from splax_amd.train import TrainStep, params_from_scene

    _case("train step config4 n=20000")
    scene = make_scene(4, n=20_000)
    params = params_from_scene(scene)
    params["opac_logit"][:500] = -12.0  # dead rows to relocate
    before = {k: v.clone() for k, v in params.items()}
    train = TrainStep(params, viewmats=_t(scene.viewmats), targets=_t(scene.targets),
                      background=_t(scene.background), img_shape=scene.img_shape, f=scene.f,
                      antialiased=True, lrs={"means": 1e-3, "log_scales": 5e-3, "quats": 1e-3,
                                             "colors_logit": 5e-2, "opac_logit": 5e-2})
    losses = [float(train()) for _ in range(6)]
    torch.cuda.synchronize()
    assert all(np.isfinite(losses)) and losses[-1] < losses[0], losses
    for k in params:
        assert not torch.equal(train.params[k], before[k]), k
    opac = torch.sigmoid(train.params["opac_logit"][:500])
    assert bool((opac > 0.005).all()), "dead rows were relocated"
    assert train.opt.count == 6
    assert _lib.check_device() == 0


@pytest.mark.parametrize("n", [1, 333, 20000])
def test_mapped_adam_equals_log_params_bwd_then_adam(n):
    """splat_adam_step_mapped (render_log's map applied in reverse inside the update) equals
    splat_log_params_bwd followed by splat_adam_step bit for bit: parameters, mu and nu over
    three steps of mapped-space gradients of mixed scales, with an unmapped group beside."""
    _case(f"mapped adam n={n}")
    rng = np.random.default_rng(n)
    raw = {"means": rng.normal(size=(n, 3)), "log_scales": rng.normal(-4, 1, size=(n, 3)),
           "quats": rng.normal(size=(n, 4)), "colors_logit": rng.normal(0, 2, size=(n, 3)),
           "opac_logit": rng.normal(0, 3, size=(n, 1))}
    raw["quats"][0] = 0.0  # a zero quaternion: the rule's 0.5 / |q| gives inf / NaN in both
    mk = lambda: {k: _t(v.astype(np.float32)) for k, v in raw.items()}  # noqa: E731
    pa, pb = mk(), mk()
    lrs = {"means": 1e-3, "log_scales": 5e-3, "quats": 1e-3, "colors_logit": 1e-2,
           "opac_logit": 5e-2}
    adam_a, adam_b = optim.Adam(pa, lrs), optim.Adam(pb, lrs)
    maps = {"log_scales": optim.MAP_EXP, "quats": optim.MAP_QUAT,
            "colors_logit": optim.MAP_SIGMOID, "opac_logit": optim.MAP_SIGMOID}
    for step in range(3):
        g = {k: _t((rng.normal(size=v.shape) * 10.0 ** rng.integers(-6, 2, size=v.shape))
                   .astype(np.float32)) for k, v in raw.items()}
        # path A: the map's backward as its own launch, then the plain update
        ins = [pa[k].contiguous() for k in ("log_scales", "quats", "colors_logit", "opac_logit")]
        outs = [torch.empty_like(t) for t in ins]
        vs = [g[k] for k in ("log_scales", "quats", "colors_logit", "opac_logit")]
        st = _lib.lib().splat_log_params_bwd(_lib.stream_handle(ins[0].device),
                                             *map(_lib.ptr, ins), n, *map(_lib.ptr, vs),
                                             *map(_lib.ptr, outs))
        _lib.check(st, "log_params_bwd")
        ga = {"means": g["means"], **dict(zip(("log_scales", "quats", "colors_logit",
                                                "opac_logit"), outs))}
        adam_a.step(ga)
        # path B: one launch
        adam_b.step(g, maps=maps)
        torch.cuda.synchronize()
        for k in raw:
            assert_bit_exact(_np(pb[k]), _np(pa[k]), f"step {step} {k}")
            assert_bit_exact(_np(adam_b.mu[k]), _np(adam_a.mu[k]), f"step {step} mu {k}")
            assert_bit_exact(_np(adam_b.nu[k]), _np(adam_a.nu[k]), f"step {step} nu {k}")
    assert not bool(torch.isfinite(pb["quats"][0]).all())  # the zero quaternion, as in path A
    with pytest.raises(ValueError):
        adam_b.step(g, maps={"nope": optim.MAP_EXP})
    assert _lib.check_device() == 0


def test_train_step_fused_map_equals_unfused():
    """TrainStep's step (the render on the mapped values, the map's backward inside Adam) equals
    the autograd chain through render_log (loss_and_grads) followed by the plain update, bit for
    bit over three steps with relocation."""
    from splax_amd.scenes import make_scene
    from splax_amd.train import TrainStep, params_from_scene

    _case("train step fused map vs unfused n=20000")
    scene = make_scene(4, n=20_000)
    kw = dict(viewmats=_t(scene.viewmats), targets=_t(scene.targets),
              background=_t(scene.background), img_shape=scene.img_shape, f=scene.f, seed=3)
    p0 = params_from_scene(scene)
    p0["opac_logit"][:300] = -12.0  # dead rows to relocate
    fused = TrainStep({k: v.clone() for k, v in p0.items()}, **kw)
    plain = TrainStep({k: v.clone() for k, v in p0.items()}, **kw)
    for _ in range(3):
        lf = fused()
        lp, grads = plain.loss_and_grads()
        plain.opt.step(grads)
        plain.step_idx += 1
        key = (plain.seed << 32) ^ plain.step_idx
        reset = mcmc.relocate_(key, *plain.params.values(), plain.binoms, plain.min_opacity)
        plain.opt.reset_rows(reset)
        torch.cuda.synchronize()
        assert_bit_exact(_np(lf), _np(lp), "loss")
        for k in fused.params:
            assert_bit_exact(_np(fused.params[k]), _np(plain.params[k]), k)
            assert_bit_exact(_np(fused.opt.mu[k]), _np(plain.opt.mu[k]), f"mu {k}")
    assert _lib.check_device() == 0


@pytest.mark.parametrize("n", [1, 777, 20000])
def test_log_params_bit_exact(n):
    """render_log's parameter map and its reverse mode, one library pass each, against the
    oracle; a missing cotangent is a zero one."""
    from splax_amd._render import _LogParamsFn

    _case(f"log_params n={n}")
    rng = np.random.default_rng(n)
    ins = [rng.normal(-4, 1, (n, 3)), rng.normal(size=(n, 4)), rng.normal(0, 2, (n, 3)),
           rng.normal(0, 3, (n, 1))]
    ins = [a.astype(np.float32) for a in ins]
    ref = T.log_params_fwd(*ins)
    leaves = [_t(a).requires_grad_(True) for a in ins]
    outs = _LogParamsFn.apply(*leaves)
    for label, g, r in zip(("scales", "quats", "colors", "opacities"), outs, ref):
        assert_bit_exact(_np(g).reshape(r.shape), r, f"log_params {label}")
    cots = [rng.normal(size=np.shape(r)).astype(np.float32) for r in ref]
    cots[2] = np.zeros_like(cots[2])
    torch.autograd.backward([outs[0], outs[1], outs[3]],
                            [_t(cots[0]), _t(cots[1]), _t(cots[3]).reshape(n, 1)])
    back = T.log_params_bwd(*ins, *cots)
    for label, x, r in zip(("v_log_scales", "v_quats", "v_logit_colors", "v_logit_opac"),
                           leaves, back):
        assert_bit_exact(_np(x.grad).reshape(r.shape), r, f"log_params {label}")


@pytest.mark.parametrize("count", [1, 4095, 4097, 16383, 16385, 3 * 1060 * 1600 * 4])
def test_l1_loss(count):
    from splax_amd.train import l1_loss

    _case(f"l1 count={count}")
    rng = np.random.default_rng(count)
    img = rng.uniform(size=count).astype(np.float32)
    tgt = rng.uniform(size=count).astype(np.float32)
    tgt[: count // 7] = img[: count // 7]  # exact ties: zero cotangent
    ref_loss, ref_v = T.l1_loss(img, tgt, g=3.0)
    x = _t(img).requires_grad_(True)
    loss = l1_loss(x, _t(tgt))
    (loss * 3.0).backward()
    assert abs(float(loss.detach()) - float(ref_loss)) <= 1e-6 * float(ref_loss)
    assert_bit_exact(_np(x.grad), ref_v, "l1 cotangent")


@pytest.mark.parametrize("count", [1, 4095, 4097, 16383, 16385, 3 * 1080 * 1920])
def test_mse_loss(count):
    from splax_amd.train import mse_loss

    _case(f"mse count={count}")
    rng = np.random.default_rng(count + 1)
    img = rng.uniform(size=count).astype(np.float32)
    tgt = rng.uniform(size=count).astype(np.float32)
    ref_loss, ref_v = T.mse_loss(img, tgt, g=3.0)
    x = _t(img).requires_grad_(True)
    loss = mse_loss(x, _t(tgt))
    (loss * 3.0).backward()
    assert abs(float(loss.detach()) - float(ref_loss)) <= 1e-6 * float(ref_loss)
    assert_bit_exact(_np(x.grad), ref_v, "mse cotangent")
