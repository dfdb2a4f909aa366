"""Helpers of the full-size timed-path tests (test infrastructure, no tests of its own).

``gpu_run`` drives the exact calls bench.py times: ``splax_amd.render_loss`` (MSE; configs 2 and
3) and the training step's ``render_log_loss`` (L1, antialiased; config 4), then their backward.
``oracle_chain`` evaluates the same workload through the float32 oracle, chained as the
reference's custom_vjp rules chain its kernels (splax/_render.py:94-115, splax/_rasterize/
_rasterize.py:191-231, splax/_project/_project.py:236-275): project_fwd -> (opacity
compensation) -> rasterize_fwd -> the loss's image cotangent -> rasterize_bwd ->
(compensation_vjp) -> project_bwd (-> render_log's parameter map), and with ``truth`` the same
chain with every backward step in float64 at the float32 forward's decisions
(oracle.rasterize_bwd_f64, oracle/truth64.py).
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import oracle as O
from oracle import train_oracle as TO
from oracle import truth64

BANDS = ((0.0, 1e2), (1e2, 1e3), (1e3, 1e4), (1e4, np.inf))


def _t(a, grad=False):
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return t.requires_grad_(True) if grad else t


def _np(t):
    return t.detach().cpu().numpy()


def log_params(s):
    """The config-4 parameters in render_log's parameterization (splax_amd.train)."""
    from splax_amd.train import params_from_scene

    return {k: v.cpu().numpy() for k, v in params_from_scene(s, "cpu").items()}


def gpu_run(s, config: int):
    """The benchmark's timed call and its backward on the GPU. Returns (loss, image, grads,
    (final_Ts, final_idx, M)); grads keyed as the call's leaves (plus "viewmat" when the call
    asks for it); the final buffers come from the same library forward (splat_render_fwd with
    the fused loss) through the tensor wrapper."""
    import splax_amd
    from splax_amd import _ops

    B = s.B
    vm_np = s.viewmats if B > 1 else s.viewmats[0]
    tgt = s.targets if B > 1 else s.targets[0]
    want_vm = config == 3
    vm = _t(vm_np, grad=want_vm)
    bg = _t(s.background)
    cam = dict(img_shape=s.img_shape, f=s.f, c=s.c)
    if config == 4:
        lp = log_params(s)
        leaves = {k: _t(v, grad=True) for k, v in lp.items()}
        loss, img = splax_amd.render_log_loss(*leaves.values(), target=_t(tgt), loss="l1",
                                              viewmat=vm, background=bg, antialiased=True,
                                              **cam)
    else:
        leaves = {k: _t(v, grad=True) for k, v in (("means", s.means), ("scales", s.scales),
                                                    ("quats", s.quats), ("colors", s.colors),
                                                    ("opac", s.opacities))}
        loss, img = splax_amd.render_loss(*leaves.values(), target=_t(tgt), loss="mse",
                                          viewmat=vm, background=bg, **cam)
    loss.backward()
    torch.cuda.synchronize()
    grads = {k: _np(v.grad) for k, v in leaves.items()}
    if want_vm:
        grads["viewmat"] = _np(vm.grad)
    out = (float(loss.item()), _np(img))
    del leaves, loss, img
    # the final buffers of the same forward call
    with torch.no_grad():
        if config == 4:
            sc, q, col, op = TO.log_params_fwd(lp["log_scales"], lp["quats"],
                                               lp["colors_logit"], lp["opac_logit"])
            geo = (s.means, sc, q, col, op)
        else:
            geo = (s.means, s.scales, s.quats, s.colors, s.opacities)
        tf = torch.zeros((1, 4, 4), device="cuda")
        tids = torch.full((1,), -1, device="cuda", dtype=torch.int32)
        loss_out = torch.empty((), device="cuda", dtype=torch.float32)
        g = [_t(a) for a in geo]
        _, Ts, fidx, kept, _ = _ops.render_fwd(
            g[0], g[1], g[2], g[3], g[4].reshape(-1), _t(s.viewmats.reshape(-1, 4)), bg, tf,
            tids, n=s.n, B=B, num_transforms=1, has_transforms=False, img_shape=s.img_shape,
            f=s.f, c=s.c, glob_scale=1.0, clip_thresh=0.01, compensate=config == 4,
            loss_kind=_ops.LOSS_L1 if config == 4 else _ops.LOSS_MSE,
            loss_target=_t(tgt).reshape(-1, s.img_shape[1], 3), loss_out=loss_out)
        torch.cuda.synchronize()
        fin = (_np(Ts), _np(fidx), kept.sort.M)
    return out[0], out[1], grads, fin


def _fold(a, B, n):
    a = np.asarray(a)
    return a.reshape(B, n, -1).astype(np.float64).sum(0) if B > 1 else a.reshape(n, -1)


def oracle_chain(s, config: int, truth: bool = False):
    """The oracle's forward (float32) and chained backward: float32, or with truth the float64
    truth of every backward step. Returns dict(loss, img, Ts, fidx, M, grads, cond) with grads
    keyed as gpu_run's and cond the largest conic condition number of each gaussian over the
    cameras that see it."""
    n, B = s.n, s.B
    H, W = s.img_shape
    aa = config == 4
    if config == 4:
        lp = log_params(s)
        scales, quats, colors, opac = TO.log_params_fwd(lp["log_scales"], lp["quats"],
                                                        lp["colors_logit"], lp["opac_logit"])
    else:
        scales, quats, colors, opac = s.scales, s.quats, s.colors, s.opacities.reshape(-1)
    q = np.roll(quats, -1, axis=-1)
    vms = s.viewmats.reshape(-1, 4)
    xys, depths, radii, conics, nth, cum = O.project_fwd(
        s.means, scales, q, vms, opac, n=n, total=B * n, img_shape=s.img_shape, f=s.f, c=s.c)
    vis = radii.reshape(-1) > 0
    ob = np.tile(np.asarray(opac, np.float32).reshape(-1), B)
    if aa:
        rho, _ = O.compensation_rho(conics)
        ob = (ob * np.where(vis, rho, np.float32(1))).astype(np.float32)
    img, Ts, fidx, _, M = O.rasterize_fwd(colors, ob, opac, s.background, xys, depths, radii,
                                          conics, cum, n=n, B=B, img_shape=s.img_shape)
    tgt = s.targets.reshape(img.shape)
    loss, vimg = (TO.l1_loss if config == 4 else TO.mse_loss)(img, tgt)
    vimg = vimg.reshape(-1, 3)
    args = (colors, ob, opac, s.background, xys, depths, radii, conics, cum, Ts, fidx, vimg)
    kw = dict(n=n, B_out=B, B_geom=B, img_shape=s.img_shape)
    if truth:
        v_colors, v_ob, v_xy, v_conic = O.rasterize_bwd_f64(*args, **kw)
    else:
        v_colors, v_ob, v_xy, v_conic, _ = O.rasterize_bwd(*args, **kw)
    if aa:
        opac_b = np.tile(np.asarray(opac, np.float32).reshape(-1), B)
        if truth:
            v_op, v_c = truth64.compensation_vjp_f64(v_ob, opac_b, conics)
        else:
            v_op, v_c = O.compensation_vjp(v_ob, opac_b, conics)
        v_op = np.where(vis, v_op, 0)  # culled items: rho = 1 in the reference, no blend terms
        v_conic = v_conic + np.where(vis[:, None], v_c, 0)
    else:
        v_op = v_ob
    zeros = np.zeros(B * n, np.float64 if truth else np.float32)
    if truth:
        vmean, vscale, vquat, vview = truth64.project_bwd_f64(
            s.means, scales, q, s.viewmats, radii, conics, v_xy, zeros, v_conic, n=n, B=B,
            f=s.f)
    else:
        vmean, vscale, vquat, vview, _ = O.project_bwd(
            s.means, scales, q, vms, radii, conics, v_xy.astype(np.float32), zeros,
            np.asarray(v_conic, np.float32), n=n, B=B, f=s.f)
    g = dict(means=_fold(vmean, B, n), scales=_fold(vscale, B, n),
             quats=np.roll(_fold(vquat, B, n), 1, axis=-1), colors=_fold(v_colors, B, n),
             opac=_fold(v_op, B, n))
    if config == 4:
        g = _log_params_bwd(lp, scales, g, truth)
    if config == 3:
        g["viewmat"] = np.asarray(vview, np.float64).reshape(B, 4, 4)
    ca, cb, cc = (conics[:, k].astype(np.float64) for k in range(3))
    cond = np.where(vis, (ca + cc) ** 2 / np.maximum(ca * cc - cb * cb, 1e-300), 0.0)
    return dict(loss=loss, img=img, Ts=Ts, fidx=fidx, M=M, grads=g,
                cond=cond.reshape(B, n).max(0))


def _log_params_bwd(lp, scales, g, truth):
    """render_log's parameter map backward (splax/_render.py:161-164): float32 through the
    oracle, or float64 from the same float32 inputs."""
    if not truth:
        v_ls, v_q, v_lc, v_lo = TO.log_params_bwd(
            lp["log_scales"], lp["quats"], lp["colors_logit"], lp["opac_logit"],
            g["scales"].astype(np.float32), g["quats"].astype(np.float32),
            g["colors"].astype(np.float32),
            g["opac"].astype(np.float32).reshape(-1))
        return dict(means=g["means"], log_scales=v_ls, quats=v_q, colors_logit=v_lc,
                    opac_logit=v_lo.reshape(-1, 1))
    d = np.float64
    ls = lp["log_scales"].astype(d)
    qr = lp["quats"].astype(d)
    sc = 1.0 / (1.0 + np.exp(-lp["colors_logit"].astype(d)))
    so = 1.0 / (1.0 + np.exp(-lp["opac_logit"].astype(d).reshape(-1)))
    v_ls = g["scales"] * np.exp(ls)
    v_lc = g["colors"] * sc * (1.0 - sc)
    v_lo = g["opac"].reshape(-1) * so * (1.0 - so)
    nrm = np.sqrt((qr * qr).sum(1))
    s_ = nrm + float(np.float32(1e-8))
    vy = g["quats"]  # wxyz, the normalized quaternion's cotangent
    v_s = -(vy * qr).sum(1) / (s_ * s_)
    vq = vy / s_[:, None] + qr * (v_s / nrm)[:, None]
    return dict(means=g["means"], log_scales=v_ls, quats=vq, colors_logit=v_lc,
                opac_logit=v_lo.reshape(-1, 1))


def rel_err(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / (np.linalg.norm(b) + 1e-300))


def band_errors(got, ref, truth, cond):
    """Per condition band: (items, relative error of got against truth, of ref against
    truth)."""
    rows = []
    for lo, hi in BANDS:
        m = (cond >= lo) & (cond < hi)
        if m.sum() == 0:
            rows.append((0, 0.0, 0.0))
            continue
        rows.append((int(m.sum()), rel_err(got[m], truth[m]), rel_err(ref[m], truth[m])))
    return rows


def weighted_chain(sc, w, vm=None, truth=False, antialiased=False, wd=None):
    """The oracle's forward and chained backward of sum(img * w) for a random_scene-style
    dictionary (conftest.random_scene), float32 or the float64 truth; with B stacked viewmats
    (vm of shape (B, 4, 4), w of shape (B, H, W, 3)) the per-camera item gradients are summed.
    With antialiased, the blend takes the compensated opacities o * rho(conic) of the visible
    items and the tile intersection the raw ones, and the backward adds the compensation's VJP
    (splax/_render.py:105-110, as oracle_chain does). With wd (shaped like the image without its
    channel axis) the objective adds sum(depth * wd) over the expected-depth channel, whose
    cotangent reaches the projection's depth input (splax/_render.py:112-114). Returns (image,
    grads keyed means / scales / quats (wxyz) / colors / opac / viewmat, cond), the image being
    (image, depth image) with wd."""
    H, W = sc["img_shape"]
    n = len(sc["means"])
    vm = sc["vm"] if vm is None else vm
    B = vm.size // 16
    q = np.roll(sc["quats"], -1, axis=-1)
    xys, depths, radii, conics, nth, cum = O.project_fwd(
        sc["means"], sc["scales"], q, vm.reshape(-1, 4), sc["opac"], n=n, total=B * n,
        img_shape=(H, W), f=sc["f"], c=sc["c"])
    vis = radii.reshape(-1) > 0
    opac_b = np.tile(np.asarray(sc["opac"], np.float32).reshape(-1), B)
    ob = sc["opac"]
    if antialiased:
        rho, _ = O.compensation_rho(conics)
        ob = (opac_b * np.where(vis, rho, np.float32(1))).astype(np.float32).reshape(-1, 1)
    fw = O.rasterize_fwd(sc["colors"], ob, sc["opac"], sc["bg"], xys, depths, radii, conics, cum,
                         n=n, B=B, img_shape=(H, W), render_depth=wd is not None)
    img, Ts, fidx = fw[0], fw[1], fw[2]
    dkw = {} if wd is None else dict(v_out_depth=np.asarray(wd, np.float32).reshape(-1))
    args = (sc["colors"], ob, sc["opac"], sc["bg"], xys, depths, radii, conics, cum, Ts, fidx,
            np.asarray(w, np.float32).reshape(-1, 3))
    kw = dict(n=n, B_out=B, B_geom=B, img_shape=(H, W), **dkw)
    vdep = np.zeros(B * n, np.float64 if truth else np.float32)
    if truth:
        out = O.rasterize_bwd_f64(*args, **kw)
        vc, vo, vxy, vcon = out[:4]
    else:
        out = O.rasterize_bwd(*args, **kw)
        vc, vo, vxy, vcon = out[:4]
    if wd is not None:
        vdep = out[-1]
    if antialiased:
        if truth:
            v_op, v_c = truth64.compensation_vjp_f64(vo, opac_b, conics)
        else:
            v_op, v_c = O.compensation_vjp(vo, opac_b, conics)
        vo = np.where(vis, v_op, 0)  # culled items: rho = 1 in the reference, no blend terms
        vcon = vcon + np.where(vis[:, None], v_c, 0)
    if truth:
        vm_, vs_, vq_, vv_ = truth64.project_bwd_f64(
            sc["means"], sc["scales"], q, vm.reshape(B, 4, 4), radii, conics, vxy,
            np.asarray(vdep, np.float64).reshape(-1), vcon, n=n, B=B, f=sc["f"])
    else:
        vm_, vs_, vq_, vv_, _ = O.project_bwd(sc["means"], sc["scales"], q, vm.reshape(-1, 4),
                                              radii, conics, vxy,
                                              np.asarray(vdep, np.float32).reshape(-1),
                                              np.asarray(vcon, np.float32), n=n, B=B,
                                              f=sc["f"])
    g = dict(means=_fold(vm_, B, n), scales=_fold(vs_, B, n),
             quats=np.roll(_fold(vq_, B, n), 1, axis=-1), colors=_fold(vc, B, n),
             opac=_fold(np.asarray(vo).reshape(-1, 1), B, n),
             viewmat=np.asarray(vv_, np.float64).reshape(B, 4, 4))
    ca, cb, cc = (conics[:, k].astype(np.float64) for k in range(3))
    cond = np.where(vis, (ca + cc) ** 2 / np.maximum(ca * cc - cb * cb, 1e-300), 0.0)
    if antialiased:
        # The compensation's own condition. rho2 = 1 - eps (a + c) + eps^2 (a c - b^2) cancels
        # to nearly zero for a gaussian far below a pixel (the 0.3 px^2 dilation then dominates
        # its covariance), keeping rho2 / (1 + eps (a + c) + eps^2 (|a c| + b^2)) of its terms'
        # magnitude, and sqrt's VJP divides by rho: the conic's rounding reaches the gradients
        # amplified by the inverse ratio. Where the float32 rho2 is <= 0 the reference's VJP is
        # NaN (0.5 / sqrt(0) times clip's zero slope) and the condition infinite.
        eps = 0.3
        r2 = 1.0 - eps * (ca + cc) + eps * eps * (ca * cc - cb * cb)
        mag = 1.0 + eps * (ca + cc) + eps * eps * (np.abs(ca * cc) + cb * cb)
        _, r2f = O.compensation_rho(conics)
        cond_rho = np.where(r2f > 0, mag / np.maximum(r2, 1e-300), np.inf)
        cond = np.where(vis, np.maximum(cond, cond_rho), cond)
    return (img if wd is None else (img, fw[-1])), g, cond.reshape(B, n).max(0)


# The bar's factor. The float32 oracle rounds each per-pixel term once and sums the terms in
# double; the GPU rounds the same terms and sums a record's 64 lanes in a six-level float32
# pairwise tree (then two more float adds across the tile's waves). For terms of random sign a
# pairwise tree of depth L rounds about sqrt(L) times as much as the terms themselves, so where
# the pixel sums dominate (the cond^2-amplified v_conic of needle-thin items) the GPU's error is
# expected near sqrt(1 + 6 + 2) = 3 times the oracle's, and where the projection VJP's own float32
# rounding dominates (common to both) near 1. Measured: at most 2.7 on the benchmark workloads and
# the extremes scene.
FACTOR = 4.0


def assert_bands(got, ref, truth, cond, label, floor=1e-5):
    """The principled bar on ill-conditioned items: per conic-condition band, got's relative
    error against the float64 truth at most FACTOR times the float32 oracle's (ref), or below
    floor (the gradient bar); the whole array likewise."""
    got, ref, truth = (np.asarray(a, np.float64) for a in (got, ref, truth))
    eg, eo = rel_err(got, truth), rel_err(ref, truth)
    print(f"    {label}: vs truth {eg:.2e} (oracle {eo:.2e})", flush=True)
    assert eg <= max(FACTOR * eo, floor), (label, "whole array", eg, eo)
    for (lo, hi), (cnt, eg, eo) in zip(BANDS, band_errors(got, ref, truth, cond)):
        if cnt:
            assert eg <= max(FACTOR * eo, floor), (label, (lo, hi), cnt, eg, eo)
