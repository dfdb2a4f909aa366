"""The config-4 training step on the gfx950 library.

One step is the reference trainer's step (scripts/train_lego.py:101-131,217-229) at a fixed
gaussian budget with the loss reduced to L1:
  1. ``render_log`` of the log / logit parameters from B cameras in one batched launch, with the
     antialiasing opacity compensation (splax/_render.py:118-168, splax/_project/_project.py:95-117);
  2. L1 = mean |img - target| and its gradient through the render's custom backward, the loss
     fused into the blends (``render_log_loss``);
  3. one fused Adam update of the five parameter groups (optax.adam per group,
     scripts/train_lego.py:203-211, exponential decay on the means' learning rate);
  4. one MCMC relocation (splax/mcmc.py:74-131) and the moment reset of the relocated rows
     (scripts/train_lego.py:136-146, 217-222);
  5. with ``noise_lr > 0`` (off by default, as config 4 times it), the means' noise of the
     reference trainer (scripts/train_lego.py:224-229,277-284): ``inject_noise`` at strength
     means-learning-rate(step) * noise_lr.
"""

from __future__ import annotations

from collections.abc import Mapping

import numpy as np
import torch

from splax_amd import _lib, mcmc
from splax_amd._render import _LogParamsFn, render_log_loss, render_loss
from splax_amd.optim import MAP_EXP, MAP_QUAT, MAP_SIGMOID, Adam, exponential_decay
from splax_amd.scenes import Scene

SPLAT_KEYS = ("means", "log_scales", "quats", "colors_logit", "opac_logit")

# render_log's map of each parameter group (splax/_render.py:161-164), applied in reverse by the
# fused Adam update
PARAM_MAPS = {"log_scales": MAP_EXP, "quats": MAP_QUAT, "colors_logit": MAP_SIGMOID,
              "opac_logit": MAP_SIGMOID}

# scripts/train_lego.py:407-411 (defaults of the reference trainer)
DEFAULT_LRS = {"means": 1.5e-3, "log_scales": 5e-3, "quats": 1e-3, "colors_logit": 1e-2,
               "opac_logit": 5e-2}


def _logit(x: np.ndarray, eps: float = 1e-4) -> np.ndarray:
    x = np.clip(x.astype(np.float64), eps, 1.0 - eps)
    return np.log(x / (1.0 - x)).astype(np.float32)


def params_from_scene(scene: Scene, device: torch.device | str = "cuda") -> dict[str, torch.Tensor]:
    """Log / logit parameters (render_log's parameterization) of a synthetic scene."""
    arrays = {
        "means": scene.means.astype(np.float32),
        "log_scales": np.log(scene.scales.astype(np.float64)).astype(np.float32),
        "quats": scene.quats.astype(np.float32),
        "colors_logit": _logit(scene.colors),
        "opac_logit": _logit(scene.opacities.reshape(-1, 1)),
    }
    return {k: torch.from_numpy(np.ascontiguousarray(v)).to(device) for k, v in arrays.items()}


class _PixelLossFn(torch.autograd.Function):
    """Mean of |img - target| ("l1") or (img - target)^2 ("mse"): one library pass each way."""

    @staticmethod
    def forward(ctx, img, target, kind):
        if img.shape != target.shape or img.dtype != torch.float32 or \
                target.dtype != torch.float32:
            raise ValueError(f"{kind}_loss: img and target must be float32 of one shape")
        img, target = img.contiguous(), target.contiguous()
        dev = _lib.require_gpu(img, target)
        count = img.numel()
        partials = torch.empty(((count + 4095) // 4096,), device=dev, dtype=torch.float64)
        loss = torch.empty((), device=dev, dtype=torch.float32)
        fwd = getattr(_lib.lib(), f"splat_{kind}_loss_fwd")
        with torch.cuda.device(dev):
            st = fwd(_lib.stream_handle(dev), img.data_ptr(), target.data_ptr(), count,
                     partials.data_ptr(), loss.data_ptr())
        _lib.check(st, f"{kind}_loss_fwd")
        ctx.save_for_backward(img, target)
        ctx.kind = kind
        return loss

    @staticmethod
    def backward(ctx, v_loss):
        img, target = ctx.saved_tensors
        v_loss = v_loss.to(torch.float32).contiguous()
        v_img = torch.empty_like(img)
        bwd = getattr(_lib.lib(), f"splat_{ctx.kind}_loss_bwd")
        with torch.cuda.device(img.device):
            st = bwd(_lib.stream_handle(img.device), img.data_ptr(), target.data_ptr(),
                     img.numel(), v_loss.data_ptr(), v_img.data_ptr())
        _lib.check(st, f"{ctx.kind}_loss_bwd")
        return v_img, None, None


def l1_loss(img: torch.Tensor, target: torch.Tensor) -> torch.Tensor:
    """mean |img - target| (scripts/train_lego.py:111), one library pass each way; the target
    receives no gradient."""
    return _PixelLossFn.apply(img, target, "l1")


def mse_loss(img: torch.Tensor, target: torch.Tensor) -> torch.Tensor:
    """mean (img - target)^2, one library pass each way (torch's mse_loss runs four kernels and
    a fill); the target receives no gradient."""
    return _PixelLossFn.apply(img, target, "mse")


class TrainStep:
    """Fixed-budget training step over B cameras; ``params`` are updated in place."""

    def __init__(self, params: Mapping[str, torch.Tensor], *, viewmats: torch.Tensor,
                 targets: torch.Tensor, background: torch.Tensor, img_shape: tuple[int, int],
                 f: tuple[float, float], c: tuple[float, float] | None = None,
                 antialiased: bool = True, steps: int = 30_000,
                 lrs: Mapping[str, float] | None = None, min_opacity: float = 0.005,
                 n_max: int = 51, relocate_every: int = 1, seed: int = 0,
                 noise_lr: float = 0.0):
        if tuple(params) != SPLAT_KEYS:
            raise ValueError(f"params must hold {SPLAT_KEYS} in this order")
        self.params = {k: p.detach().contiguous() for k, p in params.items()}
        lr = dict(DEFAULT_LRS if lrs is None else lrs)
        sched = dict(lr)
        sched["means"] = exponential_decay(lr["means"], steps, 0.01)  # train_lego.py:203
        self.opt = Adam(self.params, sched)
        self.means_lr = sched["means"]
        self.noise_lr = float(noise_lr)
        self.viewmats = viewmats
        self.targets = targets
        self.background = background
        self.camera = dict(img_shape=img_shape, f=f, c=c, antialiased=antialiased)
        self.binoms = mcmc.make_binoms(n_max)
        self.min_opacity = min_opacity
        self.relocate_every = relocate_every
        self.seed = seed
        self.step_idx = 0

    def loss_and_grads(self) -> tuple[torch.Tensor, dict[str, torch.Tensor]]:
        leaves = [p.requires_grad_(True) for p in self.params.values()]
        try:
            # the L1 loss fused into the blends (render_log then l1_loss, without the loss's own
            # passes over the images)
            loss, _ = render_log_loss(*leaves, target=self.targets, loss="l1",
                                      viewmat=self.viewmats, background=self.background,
                                      **self.camera)
            grads = torch.autograd.grad(loss, leaves)
        finally:
            for p in leaves:
                p.requires_grad_(False)
        return loss.detach(), dict(zip(SPLAT_KEYS, grads))

    def mapped_loss_and_grads(self) -> tuple[torch.Tensor, dict[str, torch.Tensor]]:
        """The loss and its gradients with respect to the means and the mapped values (scales,
        normalized quaternions, colours, opacities) of render_log's map, which the fused Adam
        update (PARAM_MAPS) turns into the log / logit parameters' gradients."""
        p = self.params
        with torch.no_grad():
            mapped = _LogParamsFn.apply(p["log_scales"], p["quats"], p["colors_logit"],
                                        p["opac_logit"])
        leaves = [p["means"].requires_grad_(True), *(t.requires_grad_(True) for t in mapped)]
        try:
            loss, _ = render_loss(*leaves, target=self.targets, loss="l1",
                                  viewmat=self.viewmats, background=self.background,
                                  **self.camera)
            grads = torch.autograd.grad(loss, leaves)
        finally:
            p["means"].requires_grad_(False)
        return loss.detach(), dict(zip(SPLAT_KEYS, grads))

    def __call__(self) -> torch.Tensor:
        """One step; returns the L1 loss before the update (a device scalar). The map's backward
        runs inside the Adam launch (bit for bit loss_and_grads followed by opt.step)."""
        loss, grads = self.mapped_loss_and_grads()
        self.opt.step(grads, maps=PARAM_MAPS)
        self.step_idx += 1
        if self.relocate_every and self.step_idx % self.relocate_every == 0:
            key = (self.seed << 32) ^ self.step_idx
            reset = mcmc.relocate_(key, *self.params.values(), self.binoms, self.min_opacity)
            self.opt.reset_rows(reset)
        if self.noise_lr > 0:
            key = (self.seed << 32) ^ self.step_idx
            p = self.params
            mcmc.inject_noise(key, p["means"], p["log_scales"], p["quats"], p["opac_logit"],
                              self.means_lr(self.step_idx) * self.noise_lr, self.min_opacity,
                              out=p["means"])
        return loss
