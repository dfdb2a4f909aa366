"""Pins the training-step oracle (oracle/train_oracle.py) without a GPU.

- Philox4x32-10 against the known-answer vectors published with the Random123 library.
- The exact 64x64 high product against Python integers.
- Adam against torch.optim.Adam in float64 (an independent implementation of the same update:
  optax's mu / bc1 / (sqrt(nu / bc2) + eps) equals torch's (lr / bc1) mu / (sqrt(nu) /
  sqrt(bc2) + eps) in exact arithmetic), and the first step's closed form.
- compute_relocation against a float64 transcription of the double sum of gsplat's relocation
  kernel (Eq. 9 of Kheradmand et al., the form tests/test_mcmc.py:21-40 of the reference checks
  against), its closed forms at ratio 1 and 2, and the invariant that r copies of the new opacity
  compose to the old one.
- relocate: the reference's invariants (tests/test_mcmc.py:63-99: dead rows reset, new opacity
  above the threshold, relocated means on alive sources), a draw brute-forced with Python
  integers, and a chi-square test of the draw frequencies against opacity.
- noise_normals: the uniforms brute-forced with Python integers, the Box-Muller identity
  z0^2 + z1^2 = -2 ln u0, and the moments, cross-correlations and Kolmogorov-Smirnov distance of
  the normals against the standard normal law.
- inject_noise: the covariance against scipy's Rotation (an independent quaternion routine),
  the closed forms of the identity rotation and of the opacity gate (1/2 at the threshold), the
  symmetry of Sigma, and the reference's own check that transparent gaussians move at least ten
  times as far as opaque ones (tests/test_mcmc.py:102-114).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import train_oracle as T


def test_philox_known_answers():
    cases = [
        ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
        ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
        ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
         (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
    ]
    for ctr, key, want in cases:
        got = tuple(int(x) for x in T.philox4x32_10(ctr, key))
        assert got == want, (ctr, key, [hex(x) for x in got])


def test_mulhi64_exact():
    rng = np.random.default_rng(3)
    r = rng.integers(0, 2**63, 2000, dtype=np.uint64) * np.uint64(2) + \
        rng.integers(0, 2, 2000, dtype=np.uint64)
    for t in (1, 3, 2**32 - 1, 2**32 + 7, 12345678901234567, 2**64 - 1):
        got = T.mulhi64(r, t)
        want = np.array([(int(x) * t) >> 64 for x in r], dtype=np.uint64)
        assert np.array_equal(got, want), t


def test_adam_matches_torch_adam_float64():
    rng = np.random.default_rng(5)
    p0 = rng.normal(size=(257, 3)).astype(np.float32)
    grads = [rng.normal(scale=10.0 ** rng.uniform(-4, 1), size=p0.shape).astype(np.float32)
             for _ in range(6)]
    lr = 3e-3
    p, mu, nu = p0.copy(), np.zeros_like(p0), np.zeros_like(p0)
    tp = torch.tensor(p0, dtype=torch.float64, requires_grad=True)
    opt = torch.optim.Adam([tp], lr=lr, betas=(0.9, 0.999), eps=1e-8)
    for step, g in enumerate(grads, start=1):
        p, mu, nu = T.adam_step(p, g, mu, nu, lr=lr, count=step)
        tp.grad = torch.tensor(g, dtype=torch.float64)
        opt.step()
        ref = tp.detach().numpy()
        np.testing.assert_allclose(p, ref, rtol=2e-6, atol=1e-7)
    st = opt.state[tp]
    # the moments are sums over steps of different gradient scales: float32 rounding is relative
    # to the largest term, not to the (possibly cancelled) total
    m_ref, v_ref = st["exp_avg"].numpy(), st["exp_avg_sq"].numpy()
    np.testing.assert_allclose(mu, m_ref, rtol=1e-5, atol=1e-6 * np.abs(m_ref).max())
    np.testing.assert_allclose(nu, v_ref, rtol=1e-5, atol=1e-6 * np.abs(v_ref).max())


def test_adam_first_step_closed_form():
    """count 1: mu_hat = g and nu_hat = g^2 up to rounding, so p' = p - lr g / (|g| + eps)."""
    g = np.array([1.0, -2.5, 1e-3, -7e-9, 0.0], np.float32)
    p = np.zeros_like(g)
    out, mu, nu = T.adam_step(p, g, np.zeros_like(g), np.zeros_like(g), lr=0.1, count=1)
    want = -0.1 * g.astype(np.float64) / (np.abs(g.astype(np.float64)) + 1e-8)
    np.testing.assert_allclose(out, want, rtol=1e-6, atol=1e-9)
    assert out[-1] == 0.0


def test_reset_rows():
    mu = np.ones((4, 3), np.float32)
    nu = np.full((4, 3), 2.0, np.float32)
    m2, n2 = T.reset_rows(mu, nu, [True, False, True, False])
    assert (m2[[0, 2]] == 0).all() and (m2[[1, 3]] == 1).all() and (n2[[1, 3]] == 2).all()


def _eq9_double_loop(o: float, n: int) -> tuple[float, float]:
    """Float64 double sum over i = 1..n, k = 0..i-1 of C(i-1, k) (-1)^k / sqrt(k+1) o'^(k+1)."""
    no = 1.0 - (1.0 - o) ** (1.0 / n)
    denom = 0.0
    for i in range(1, n + 1):
        for k in range(i):
            denom += math.comb(i - 1, k) * (-1.0) ** k / math.sqrt(k + 1.0) * no ** (k + 1)
    return no, o / denom


def test_compute_relocation_matches_double_loop():
    rng = np.random.default_rng(0)
    n = 300
    opac = rng.uniform(0.01, 0.99, n).astype(np.float32)
    scales = rng.uniform(0.01, 0.5, (n, 3)).astype(np.float32)
    ratios = rng.integers(1, 40, n).astype(np.float32)
    got_o, got_s = T.compute_relocation(opac, scales, ratios, n_max=51)
    for i in range(n):
        no, coeff = _eq9_double_loop(float(opac[i]), int(ratios[i]))
        assert abs(float(got_o[i]) - no) <= 1e-7 * abs(no) + 1e-12, i
        np.testing.assert_allclose(got_s[i], coeff * scales[i].astype(np.float64), rtol=1e-6)


def test_compute_relocation_closed_forms_and_invariant():
    opac = np.array([0.1, 0.5, 0.9, 0.3], np.float32)
    scales = np.array([[0.1, 0.2, 0.3], [0.4, 0.4, 0.4], [0.05, 0.1, 0.2], [1, 2, 3]],
                      np.float32)
    o1, s1 = T.compute_relocation(opac, scales, np.ones(4, np.float32), n_max=51)
    assert np.array_equal(o1, opac)
    np.testing.assert_allclose(s1, scales, rtol=1e-7)
    o2, s2 = T.compute_relocation(opac, scales, np.full(4, 2.0, np.float32), n_max=51)
    for i, o in enumerate(opac.astype(np.float64)):
        no = 1.0 - math.sqrt(1.0 - o)
        coeff = o / (2.0 * no - no * no / math.sqrt(2.0))
        assert abs(float(o2[i]) - no) <= 1e-7 * no
        np.testing.assert_allclose(s2[i], coeff * scales[i].astype(np.float64), rtol=1e-6)
    # r copies at the new opacity composite to the old one; ratios beyond n_max are clipped
    o7, _ = T.compute_relocation(opac, scales, np.full(4, 7.0, np.float32), n_max=51)
    np.testing.assert_allclose(1.0 - (1.0 - o7.astype(np.float64)) ** 7, opac, rtol=1e-6)
    oc, _ = T.compute_relocation(opac, scales, np.full(4, 90.0, np.float32), n_max=5)
    o5, _ = T.compute_relocation(opac, scales, np.full(4, 5.0, np.float32), n_max=51)
    assert np.array_equal(oc, o5)


def _scene(n, n_dead, seed):
    rng = np.random.default_rng(seed)
    means = rng.uniform(-1, 1, (n, 3)).astype(np.float32)
    log_scales = np.full((n, 3), math.log(0.05), np.float32) + \
        rng.normal(0, 0.1, (n, 3)).astype(np.float32)
    quats = rng.normal(size=(n, 4)).astype(np.float32)
    colors = rng.normal(size=(n, 3)).astype(np.float32)
    logit = rng.normal(0.85, 1.0, n).astype(np.float32)
    logit[:n_dead] = -20.0
    return means, log_scales, quats, colors, logit


def test_relocate_invariants():
    """The reference's test_relocate_teleports_dead_onto_alive (tests/test_mcmc.py:63-99)."""
    means, ls, q, c, logit = _scene(500, 100, 1)
    nm, nls, nq, nc, nl, src, reset = T.relocate(7, means, ls, q, c, logit, n_max=51)
    assert nm.shape == (500, 3) and nl.shape == (500,)
    assert reset[:100].all()
    new_opac = T.sigmoid(nl)
    assert (new_opac[:100] > 0.005).all()
    for i in range(100):
        s = src[i]
        assert s >= 100 and np.array_equal(nm[i], means[s]) and np.array_equal(nq[i], q[s])
        assert np.array_equal(nc[i], c[s])
    # untouched rows keep every parameter; drawn sources keep mean, rotation and colour
    keep = ~reset
    assert np.array_equal(nm[keep], means[keep]) and np.array_equal(nl[keep], logit[keep])
    drawn = np.unique(src[:100])
    assert reset[drawn].all() and np.array_equal(nm[drawn], means[drawn])
    # every row sharing a source carries the source's corrected values
    for i in range(100):
        assert nl[i] == nl[src[i]] and np.array_equal(nls[i], nls[src[i]])


def test_relocate_draw_brute_force():
    """The vectorized draw equals the same definition evaluated with Python integers."""
    means, ls, q, c, logit = _scene(60, 25, 2)
    seed = 0x1234_5678_9ABC_DEF0
    src = T.relocate(seed, means, ls, q, c, logit, n_max=51)[5]
    opac = T.sigmoid(logit)
    w = [0 if o <= np.float32(0.005) else int(np.float32(o) * np.float32(2.0**32)) for o in opac]
    total = sum(w)
    for i in range(25):
        c4 = T.philox4x32_10((i, 0, T.RELOCATE_TAG, 0), (seed & 0xFFFFFFFF, seed >> 32))
        r = (int(c4[0]) << 32) | int(c4[1])
        u = (r * total) >> 64
        acc, pick = 0, None
        for j, wj in enumerate(w):
            acc += wj
            if acc > u:
                pick = j
                break
        assert src[i] == pick, i


def test_relocate_draw_distribution():
    """4000 dead rows draw among 5 alive rows with probability proportional to opacity."""
    n_alive, n_dead = 5, 4000
    logit = np.concatenate([np.full(n_dead, -30.0), np.array([-2.0, -0.5, 0.0, 1.0, 3.0])])
    logit = logit.astype(np.float32)
    n = logit.size
    z3 = np.zeros((n, 3), np.float32)
    src = T.relocate(99, z3, z3, np.zeros((n, 4), np.float32), z3, logit, n_max=51)[5]
    hist = np.bincount(src[:n_dead] - n_dead, minlength=n_alive)
    p = T.sigmoid(logit[n_dead:]).astype(np.float64)
    p /= p.sum()
    exp = p * n_dead
    chi2 = float(((hist - exp) ** 2 / exp).sum())
    assert chi2 < 18.5, (hist, exp, chi2)  # p = 0.001 at 4 degrees of freedom


def test_relocate_nothing_alive_draws_row_zero():
    means, ls, q, c, logit = _scene(8, 8, 4)
    src = T.relocate(1, means, ls, q, c, logit, n_max=51)[5]
    assert (src == 0).all()


@pytest.mark.parametrize("seed", [0, 1, 2**40 + 5])
def test_relocate_deterministic(seed):
    a = T.relocate(seed, *_scene(200, 50, 6), n_max=51)
    b = T.relocate(seed, *_scene(200, 50, 6), n_max=51)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)


def test_log_params_match_float64_autograd():
    """render_log's parameter map and its reverse mode against float64 torch autograd of the
    reference expression (splax/_render.py:161-164)."""
    rng = np.random.default_rng(12)
    n = 400
    ls = rng.normal(-4, 1, (n, 3)).astype(np.float32)
    q = rng.normal(size=(n, 4)).astype(np.float32)
    lc = rng.normal(0, 2, (n, 3)).astype(np.float32)
    lo = rng.normal(0, 3, n).astype(np.float32)
    got = T.log_params_fwd(ls, q, lc, lo)
    t = [torch.tensor(a, dtype=torch.float64, requires_grad=True) for a in (ls, q, lc, lo)]
    want = (torch.exp(t[0]), t[1] / (torch.linalg.norm(t[1], dim=-1, keepdim=True) + 1e-8),
            torch.sigmoid(t[2]), torch.sigmoid(t[3]))
    for g, w in zip(got, want):
        np.testing.assert_allclose(g, w.detach().numpy(), rtol=2e-6, atol=1e-9)
    cots = [rng.normal(size=a.shape).astype(np.float32) for a in got]
    back = T.log_params_bwd(ls, q, lc, lo, *cots)
    torch.autograd.backward(want, [torch.tensor(c, dtype=torch.float64) for c in cots])
    for b, x in zip(back, t):
        np.testing.assert_allclose(b, x.grad.numpy(), rtol=2e-5, atol=1e-7)
    # the normalized quaternion's gradient is orthogonal to it
    u = got[1].astype(np.float64)
    assert np.abs((back[1] * u).sum(1)).max() < 1e-4 * np.abs(back[1]).max()


def test_l1_loss_closed_form():
    img = np.array([0.5, 0.25, 1.0, 0.75], np.float32)
    tgt = np.array([0.25, 0.25, 0.0, 1.0], np.float32)
    loss, v = T.l1_loss(img, tgt)
    assert loss == np.float32((0.25 + 0 + 1.0 + 0.25) / 4)
    assert v.tolist() == [0.25, 0.0, 0.25, -0.25]


def test_mse_loss_closed_form_and_torch():
    img = np.array([0.5, 0.25, 1.0, 0.75], np.float32)
    tgt = np.array([0.25, 0.25, 0.0, 1.0], np.float32)
    loss, v = T.mse_loss(img, tgt)
    assert loss == np.float32((0.0625 + 0 + 1.0 + 0.0625) / 4)
    assert v.tolist() == [0.125, 0.0, 0.5, -0.125]
    # against torch's own mse_loss and its gradient (float64, random inputs)
    import torch

    rng = np.random.default_rng(3)
    a = rng.uniform(size=10_000).astype(np.float32)
    b = rng.uniform(size=10_000).astype(np.float32)
    loss, v = T.mse_loss(a, b, g=2.0)
    x = torch.tensor(a, dtype=torch.float64, requires_grad=True)
    ref = torch.nn.functional.mse_loss(x, torch.tensor(b, dtype=torch.float64))
    (2.0 * ref).backward()
    assert abs(float(loss) - ref.item()) <= 1e-6 * ref.item()
    np.testing.assert_allclose(v, x.grad.numpy(), rtol=1e-6, atol=0)


def test_noise_uniforms_brute_force():
    seed = 0x1234_5678_9ABC_DEF0
    u = T.noise_uniforms(seed, 5)
    for i in range(5):
        c = T.philox4x32_10((i, 0, T.NOISE_TAG, 0), (seed & 0xFFFFFFFF, seed >> 32))
        want = [((int(w) >> 9) + 0.5) / 2**23 for w in c]
        assert list(u[i]) == want
    assert (u > 0).all() and (u < 1).all()
    assert (u.astype(np.float32).astype(np.float64) == u).all()  # exact in float32


def test_noise_normals_box_muller_identity_and_law():
    from scipy import stats

    n = 400_000
    z = T.noise_normals(7, n)
    u = T.noise_uniforms(7, n)
    np.testing.assert_allclose(z[:, 0] ** 2 + z[:, 1] ** 2, -2.0 * np.log(u[:, 0]), rtol=1e-12)
    assert np.abs(z.mean(axis=0)).max() < 5 * n ** -0.5
    assert np.abs(z.var(axis=0) - 1.0).max() < 5 * (2.0 / n) ** 0.5
    c = np.corrcoef(z.T)
    assert np.abs(c - np.eye(3)).max() < 5 * n ** -0.5
    for k in range(3):
        assert stats.kstest(z[:, k], "norm").pvalue > 1e-3, k
    # a planted mistake: the same uniform for radius and angle is visibly not normal
    bad = np.sqrt(-2.0 * np.log(u[:, 0])) * np.cos(2.0 * np.pi * u[:, 0])
    assert stats.kstest(bad, "norm").pvalue < 1e-6


def test_inject_noise_covariance_matches_scipy():
    from scipy.spatial.transform import Rotation

    rng = np.random.default_rng(3)
    n = 64
    means = rng.normal(size=(n, 3))
    ls = rng.normal(scale=0.7, size=(n, 3))
    q = rng.normal(size=(n, 4)) * rng.uniform(0.2, 3.0, size=(n, 1))  # not unit on purpose
    logit = rng.normal(scale=4.0, size=(n, 1))
    z = rng.normal(size=(n, 3))
    scaler, mo = 0.37, 0.01
    got = T.inject_noise(means, ls, q, logit, scaler, z, mo)
    R = Rotation.from_quat(q, scalar_first=True).as_matrix()
    s2 = np.exp(2.0 * ls)
    o = 1.0 / (1.0 + np.exp(-logit[:, 0]))
    gate = 1.0 / (1.0 + np.exp(-100.0 * (mo - o)))
    want = np.empty_like(means)
    for i in range(n):
        sigma = R[i] @ np.diag(s2[i]) @ R[i].T
        assert np.allclose(sigma, sigma.T)
        want[i] = means[i] + sigma @ (z[i] * gate[i] * scaler)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
    # planted mistakes: m^T m in place of m m^T, and the conjugate rotation, both differ
    m = T.quat_wxyz_to_rot(q) * np.exp(ls)[:, None, :]
    wrong = means + np.einsum("nji,njk,nk->ni", m, m, z * (gate * scaler)[:, None])
    assert np.abs(wrong - want).max() > 1e-3
    qc = q * np.array([1.0, -1.0, -1.0, -1.0])
    assert np.abs(T.inject_noise(means, ls, qc, logit, scaler, z, mo) - want).max() > 1e-3


def test_inject_noise_closed_forms():
    n = 6
    means = np.arange(3 * n, dtype=np.float64).reshape(n, 3)
    ls = np.log(np.array([[0.5, 2.0, 3.0]] * n))
    q = np.tile([2.0, 0.0, 0.0, 0.0], (n, 1))  # identity after normalization
    mo = 0.2
    logit = np.full((n, 1), np.log(mo / (1.0 - mo)))  # opacity exactly at the threshold
    z = np.ones((n, 3))
    got = T.inject_noise(means, ls, q, logit, 4.0, z, mo)
    np.testing.assert_allclose(got - means, np.tile([0.25 * 2.0, 4.0 * 2.0, 9.0 * 2.0], (n, 1)),
                               rtol=1e-12)
    # a rotation by 90 degrees about z swaps the x and y variances
    q90 = np.tile([np.cos(np.pi / 4), 0.0, 0.0, np.sin(np.pi / 4)], (n, 1))
    got = T.inject_noise(means, ls, q90, logit, 4.0, z, mo)
    np.testing.assert_allclose(got - means, np.tile([4.0 * 2.0, 0.25 * 2.0, 9.0 * 2.0], (n, 1)),
                               rtol=1e-12)


def test_inject_noise_respects_opacity():
    """The reference's check (tests/test_mcmc.py:102-114) on the oracle with its own normals."""
    n = 400
    means = np.zeros((n, 3))
    ls = np.full((n, 3), np.log(0.1))
    q = np.tile([1.0, 0.0, 0.0, 0.0], (n, 1))
    logit = np.concatenate([np.full((200, 1), -5.0), np.full((200, 1), 8.0)])
    moved = T.inject_noise(means, ls, q, logit, 100.0, T.noise_normals(2, n))
    disp = np.linalg.norm(moved, axis=1)
    assert disp[:200].mean() > 10 * disp[200:].mean() + 1e-6
