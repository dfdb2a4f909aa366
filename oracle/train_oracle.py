"""CPU restatement of the training-step operations (test infrastructure only).

Only ``tests/`` and ``bench.py``'s ``cpu_baseline`` leg import this module, as the checker of
the GPU library; the product package never does.

- ``adam_step``: optax 0.2.8 ``adam`` (a dependency of the reference's trainers, pinned in
  pixi.lock, not vendored in the reference) as called at scripts/train_lego.py:203-211:
  ``scale_by_adam`` (mu = (1-b1) g + b1 mu, nu = (1-b2) g^2 + b2 nu, bias corrections
  1 - b^count at the incremented count, u = mu_hat / (sqrt(nu_hat + eps_root) + eps)), then
  ``scale_by_learning_rate`` (u * -lr) and ``apply_updates`` (p + u), in float32.
- ``reset_rows``: _reset_opt_state, scripts/train_lego.py:136-146.
- ``philox4x32_10``: the counter-based generator of Salmon et al., "Parallel random numbers:
  as easy as 1, 2, 3" (SC'11), 10 rounds, as the library's relocation draw uses it.
- ``compute_relocation``: splax/mcmc.py:44-71 in double with exact binomials.
- ``relocate``: splax/mcmc.py:74-131 with the library's exact draw (integer weights
  opacity * 2^32, inclusive uint64 prefix, u = floor(r * total / 2^64) from a Philox draw at
  counter (i, 0, tag, 0), first index whose prefix exceeds u).
- ``noise_normals``: the library's standard normals for ``inject_noise``: Philox at counter
  (i_lo, i_hi, NOISE_TAG, 0), each word's top 23 bits as u = (k + 1/2) 2^-23, and Box-Muller
  (z0, z1) = sqrt(-2 ln u0) (cos, sin)(2 pi u1), z2 = sqrt(-2 ln u2) cos(2 pi u3), in double.
- ``inject_noise``: splax/mcmc.py:134-169 in double: means + R diag(s)^2 R^T (z gate scaler)
  with s = exp(log_scales), R the rotation of the normalized wxyz quaternion and
  gate = sigmoid(100 (min_opacity - sigmoid(logit))).
"""

from __future__ import annotations

import math

import numpy as np

from oracle import oracle as O

PHILOX_M = (0xD2511F53, 0xCD9E8D57)
PHILOX_W = (0x9E3779B9, 0xBB67AE85)
RELOCATE_TAG = 0x4D434D43
NOISE_TAG = 0x4E4F4953
_M32 = np.uint64(0xFFFFFFFF)


# ---------------------------------------------------------------- Adam

def adam_step(p, g, mu, nu, *, lr, count, b1=0.9, b2=0.999, eps=1e-8, eps_root=0.0):
    """One optax adam update of one parameter group; returns new (p, mu, nu) as float32."""
    f = np.float32
    p, g, mu, nu = (np.asarray(a, np.float32) for a in (p, g, mu, nu))
    c1, c2 = f(1.0 - b1), f(1.0 - b2)  # Python-float constants, rounded once to float32
    bc1 = f(1.0 - math.pow(b1, count))
    bc2 = f(1.0 - math.pow(b2, count))
    mu = c1 * g + f(b1) * mu
    nu = c2 * (g * g) + f(b2) * nu
    u = (mu / bc1) / (np.sqrt(nu / bc2 + f(eps_root)) + f(eps))
    p = p + f(-lr) * u
    return p.astype(np.float32), mu.astype(np.float32), nu.astype(np.float32)


def reset_rows(mu, nu, reset):
    """Zero the moment rows flagged in reset (leading axis = rows)."""
    keep = ~np.asarray(reset, bool)
    shape = (-1,) + (1,) * (np.ndim(mu) - 1)
    return mu * keep.reshape(shape), nu * keep.reshape(shape)


# ---------------------------------------------------------------- Philox4x32-10

def philox4x32_10(ctr, key):
    """ctr: four uint32 arrays (or scalars), key: two uint32 -> four uint32 arrays."""
    c = [np.asarray(x, np.uint64) & _M32 for x in ctr]
    k0, k1 = int(key[0]) & 0xFFFFFFFF, int(key[1]) & 0xFFFFFFFF
    for r in range(10):
        if r:
            k0 = (k0 + PHILOX_W[0]) & 0xFFFFFFFF
            k1 = (k1 + PHILOX_W[1]) & 0xFFFFFFFF
        p0 = np.uint64(PHILOX_M[0]) * c[0]
        p1 = np.uint64(PHILOX_M[1]) * c[2]
        c = [(p1 >> np.uint64(32)) ^ c[1] ^ np.uint64(k0), p1 & _M32,
             (p0 >> np.uint64(32)) ^ c[3] ^ np.uint64(k1), p0 & _M32]
    return [x.astype(np.uint32) for x in c]


def mulhi64(r: np.ndarray, t: int) -> np.ndarray:
    """floor(r * t / 2^64) for uint64 r and 0 <= t < 2^64, exactly."""
    r = np.asarray(r, np.uint64)
    rh, rl = r >> np.uint64(32), r & _M32
    th, tl = np.uint64(t >> 32), np.uint64(t & 0xFFFFFFFF)
    ll, lh, hl = rl * tl, rl * th, rh * tl
    mid = (ll >> np.uint64(32)) + (lh & _M32) + (hl & _M32)
    return rh * th + (lh >> np.uint64(32)) + (hl >> np.uint64(32)) + (mid >> np.uint64(32))


# ---------------------------------------------------------------- relocation

def sigmoid(x) -> np.ndarray:
    """1 / (1 + e^-x) in float32 with the library's fixed-sequence exp."""
    x = np.asarray(x, np.float32)
    return (np.float32(1.0) / (np.float32(1.0) + O.expf(-x))).astype(np.float32)


def relocation_values(o: float, r: int) -> tuple[float, float]:
    """(new opacity, scale factor) for one source of multiplicity r (splax/mcmc.py:44-71).
    IEEE double throughout: an opacity too small to change 1 - o gives o / 0 = inf, as in the
    reference's float32 evaluation."""
    no = 1.0 - (1.0 - o) ** (1.0 / r)
    denom, pw = 0.0, 1.0
    for k in range(r):
        pw = pw * no
        term = float(math.comb(r, k + 1)) * pw / math.sqrt(k + 1)
        denom = denom - term if k & 1 else denom + term
    with np.errstate(divide="ignore", invalid="ignore"):
        coeff = float(np.float64(o) / np.float64(denom))
    return no, coeff


def compute_relocation(opacities, scales, ratios, n_max: int):
    """splax/mcmc.py:44-71 -> (new_opac [n] f32, new_scales [n,3] f32)."""
    opac = np.asarray(opacities, np.float32).reshape(-1)
    sc = np.asarray(scales, np.float32).reshape(-1, 3)
    rr = np.rint(np.asarray(ratios, np.float32).reshape(-1))
    new_o = np.empty_like(opac)
    new_s = np.empty_like(sc)
    for i in range(opac.size):
        r = 1 if not rr[i] >= 1 else (n_max if rr[i] >= n_max else int(rr[i]))
        no, coeff = relocation_values(float(opac[i]), r)
        new_o[i] = np.float32(no)
        with np.errstate(invalid="ignore", over="ignore"):
            new_s[i] = (coeff * sc[i].astype(np.float64)).astype(np.float32)
    return new_o, new_s


def relocate(seed: int, means, log_scales, quats, logit_colors, logit_opacities, n_max: int,
             min_opacity: float = 0.005):
    """splax/mcmc.py:74-131 with the library's draw; returns (means, log_scales, quats,
    logit_colors, logit_opacities, source int32, reset bool) as new arrays."""
    means = np.array(means, np.float32).reshape(-1, 3)
    log_scales = np.array(log_scales, np.float32).reshape(-1, 3)
    quats = np.array(quats, np.float32).reshape(-1, 4)
    colors = np.array(logit_colors, np.float32).reshape(-1, 3)
    logit = np.array(logit_opacities, np.float32).reshape(-1)
    n = logit.size
    mo = np.float32(min_opacity)
    opac = sigmoid(logit)
    dead = opac <= mo
    w = np.where(dead, np.uint64(0), (opac * np.float32(2.0**32)).astype(np.uint64))
    cdf = np.cumsum(w, dtype=np.uint64)
    total = int(cdf[-1]) if n else 0
    idx = np.arange(n, dtype=np.int64)
    src = idx.copy()
    d = np.nonzero(dead)[0]
    if d.size:
        if total == 0:
            src[d] = 0
        else:
            c = philox4x32_10((d & 0xFFFFFFFF, d >> 32, np.full(d.size, RELOCATE_TAG),
                               np.zeros(d.size)), (seed & 0xFFFFFFFF, seed >> 32))
            r = (c[0].astype(np.uint64) << np.uint64(32)) | c[1].astype(np.uint64)
            u = mulhi64(r, total)
            src[d] = np.searchsorted(cdf, u, side="right")
    counts = np.bincount(src[d], minlength=n).astype(np.int64)
    reset = dead | (counts > 0)
    newv = {}
    lo_clip, hi_clip = float(mo), 1.0 - 2.0**-23
    for s in np.nonzero(counts)[0]:
        r = min(int(counts[s]) + 1, n_max)
        no, coeff = relocation_values(float(opac[s]), r)
        no = min(max(no, lo_clip), hi_clip)
        sc = O.expf(log_scales[s]).astype(np.float64)
        with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
            newv[s] = (np.float32(np.log(no / (1.0 - no))),
                       np.log(coeff * sc).astype(np.float32))
    out_means, out_ls, out_q, out_c, out_l = (a.copy() for a in (means, log_scales, quats,
                                                                   colors, logit))
    for i in np.nonzero(reset)[0]:
        s = int(src[i]) if dead[i] else int(i)
        if dead[i]:
            out_means[i], out_q[i], out_c[i] = means[s], quats[s], colors[s]
        out_l[i], out_ls[i] = newv[s]
    return out_means, out_ls, out_q, out_c, out_l, src.astype(np.int32), reset


# ---------------------------------------------------------------- noise on the means

def noise_uniforms(seed: int, n: int) -> np.ndarray:
    """(n, 4) uniforms (k + 1/2) 2^-23 from the top 23 bits of each Philox word."""
    i = np.arange(n, dtype=np.uint64)
    c = philox4x32_10((i & _M32, i >> np.uint64(32), np.full(n, NOISE_TAG, np.uint64),
                       np.zeros(n, np.uint64)), (seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF))
    return np.stack([((np.asarray(w, np.uint64) >> np.uint64(9)).astype(np.float64) + 0.5)
                     * 2.0**-23 for w in c], axis=1)


def noise_normals(seed: int, n: int) -> np.ndarray:
    """(n, 3) standard normals by Box-Muller on noise_uniforms, in double."""
    u = noise_uniforms(seed, n)
    r0, r1 = np.sqrt(-2.0 * np.log(u[:, 0])), np.sqrt(-2.0 * np.log(u[:, 2]))
    t0, t1 = 2.0 * np.pi * u[:, 1], 2.0 * np.pi * u[:, 3]
    return np.stack([r0 * np.cos(t0), r0 * np.sin(t0), r1 * np.cos(t1)], axis=1)


def quat_wxyz_to_rot(q) -> np.ndarray:
    """Rotation matrices (n, 3, 3) of the normalized wxyz quaternions, in double."""
    q = np.asarray(q, np.float64).reshape(-1, 4)
    w, x, y, z = (q / np.linalg.norm(q, axis=1, keepdims=True)).T
    return np.stack([
        np.stack([1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)], -1),
        np.stack([2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)], -1),
        np.stack([2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)], -1),
    ], axis=1)


def inject_noise(means, log_scales, quats, logit_opacities, scaler: float, noise,
                 min_opacity: float = 0.005) -> np.ndarray:
    """splax/mcmc.py:134-169 in double with the given standard normals noise (n, 3)."""
    means = np.asarray(means, np.float64).reshape(-1, 3)
    s = np.exp(np.asarray(log_scales, np.float64).reshape(-1, 3))
    o = 1.0 / (1.0 + np.exp(-np.asarray(logit_opacities, np.float64).reshape(-1)))
    gate = 1.0 / (1.0 + np.exp(-100.0 * (float(min_opacity) - o)))
    w = np.asarray(noise, np.float64).reshape(-1, 3) * (gate * float(scaler))[:, None]
    m = quat_wxyz_to_rot(quats) * s[:, None, :]  # R diag(s), Sigma = m m^T
    return means + np.einsum("nij,nkj,nk->ni", m, m, w)


# ---------------------------------------------------------------- render_log map and L1 loss

_QUAT_EPS = np.float32(1e-8)  # splax/_render.py:162


def _qnorm(q):
    return np.sqrt(((q[:, 0] * q[:, 0] + q[:, 1] * q[:, 1]) + q[:, 2] * q[:, 2])
                   + q[:, 3] * q[:, 3])


def log_params_fwd(log_scales, quats, logit_colors, logit_opacities):
    """render_log's parameter map (splax/_render.py:161-164) in float32 with the library's exp;
    returns (scales, quats / (|quats| + 1e-8), colors, opacities)."""
    ls = np.asarray(log_scales, np.float32).reshape(-1, 3)
    q = np.asarray(quats, np.float32).reshape(-1, 4)
    s = (_qnorm(q) + _QUAT_EPS)[:, None]
    scales = O.expf(ls).reshape(ls.shape)
    colors = sigmoid(logit_colors).reshape(-1, 3)
    opac = sigmoid(logit_opacities).reshape(-1)
    return scales, (q / s).astype(np.float32), colors, opac


def log_params_bwd(log_scales, quats, logit_colors, logit_opacities, v_scales, v_quats,
                   v_colors, v_opac):
    """Reverse mode of log_params_fwd: exp' = exp, logistic' = s (1 - s), and for
    q / (sqrt(sum q^2) + eps) the direct term g / s plus 2 q v_ss with
    v_ss = (sum_k -(g_k q_k) / s^2) * 0.5 / |q|, in float32."""
    f = np.float32
    ls = np.asarray(log_scales, np.float32).reshape(-1, 3)
    q = np.asarray(quats, np.float32).reshape(-1, 4)
    sc = sigmoid(logit_colors).reshape(-1, 3)
    so = sigmoid(logit_opacities).reshape(-1)
    v_ls = np.asarray(v_scales, np.float32).reshape(-1, 3) * O.expf(ls).reshape(ls.shape)
    v_lc = np.asarray(v_colors, np.float32).reshape(-1, 3) * (sc * (f(1) - sc))
    v_lo = np.asarray(v_opac, np.float32).reshape(-1) * (so * (f(1) - so))
    vy = np.asarray(v_quats, np.float32).reshape(-1, 4)
    nrm = _qnorm(q)
    s = nrm + _QUAT_EPS
    inv_s2 = f(1) / (s * s)
    v_s = np.zeros_like(s)
    for k in range(4):
        v_s = v_s + (-(vy[:, k] * q[:, k])) * inv_s2
    with np.errstate(divide="ignore", invalid="ignore"):
        v_ss = v_s * (f(0.5) / nrm)
    vq = vy / s[:, None] + (v_ss[:, None] * q + v_ss[:, None] * q)
    return (v_ls.astype(np.float32), vq.astype(np.float32), v_lc.astype(np.float32),
            v_lo.astype(np.float32))


def l1_loss(img, target, g=1.0):
    """mean |img - target| (scripts/train_lego.py:111): float32 differences, summed in double,
    rounded once; returns (loss, img cotangent sign(d) * (g / count) for loss cotangent g)."""
    d = np.asarray(img, np.float32).reshape(-1) - np.asarray(target, np.float32).reshape(-1)
    loss = np.float32(np.abs(d).astype(np.float64).sum() / d.size)
    scale = np.float32(g) / np.float32(d.size)
    sg = np.where(d > 0, np.float32(1), np.where(d < 0, np.float32(-1), d))
    return loss, (sg * scale).astype(np.float32)


def mse_loss(img, target, g=1.0):
    """mean (img - target)^2, the benchmark workloads' loss (configs 0-3 take the MSE to a
    seeded target; the reference library has no loss of its own): float32 differences, squared
    and summed in double, rounded once; returns (loss, img cotangent 2 d * (g / count) for loss
    cotangent g, with 2 d formed as d + d)."""
    d = np.asarray(img, np.float32).reshape(-1) - np.asarray(target, np.float32).reshape(-1)
    d64 = d.astype(np.float64)
    loss = np.float32((d64 * d64).sum() / d.size)
    scale = np.float32(g) / np.float32(d.size)
    return loss, ((d + d) * scale).astype(np.float32)
