"""Per-parameter-group Adam on the gfx950 library.

The reference's trainers build ``optax.multi_transform`` over one ``optax.adam`` per parameter
group (scripts/train_lego.py:203-211), with an ``optax.exponential_decay`` schedule on the means,
and zero the moments of relocated rows (scripts/train_lego.py:136-146). ``Adam`` keeps the same
state (per-group mu, nu and a step count) and applies all groups in one fused launch
(``splat_adam_step``); ``reset_rows`` is one launch over every group's moments.
"""

from __future__ import annotations

import ctypes
from collections.abc import Callable, Mapping

import torch

from splax_amd import _lib

Schedule = Callable[[int], float]

# Parameter maps of Adam.step (include/splat_hip.h SPLAT_MAP_*): the gradient given for the group
# is the cotangent of the mapped value of render_log (splax/_render.py:161-164), and the update
# applies the map's reverse-mode rule first.
MAP_NONE, MAP_EXP, MAP_SIGMOID, MAP_QUAT = 0, 1, 2, 3


def exponential_decay(init_value: float, transition_steps: int,
                      decay_rate: float) -> Schedule:
    """optax.exponential_decay without staircase or delay: init * rate ** (count / steps)."""
    if transition_steps <= 0:
        return lambda count: float(init_value)
    return lambda count: float(init_value) * float(decay_rate) ** (count / transition_steps)


class Adam:
    """optax.adam(lr_k, b1, b2, eps, eps_root) per named group, updated in place."""

    def __init__(self, params: Mapping[str, torch.Tensor],
                 lr: Mapping[str, float | Schedule], *, b1: float = 0.9, b2: float = 0.999,
                 eps: float = 1e-8, eps_root: float = 0.0):
        if set(lr) != set(params):
            raise ValueError(f"learning rates {sorted(lr)} do not match groups {sorted(params)}")
        if len(params) > 8:
            raise ValueError("at most 8 parameter groups")
        for k, p in params.items():
            if p.dtype != torch.float32 or not p.is_contiguous():
                raise ValueError(f"group {k!r} must be a contiguous float32 tensor")
        self.params = dict(params)
        self.lr = dict(lr)
        self.b1, self.b2, self.eps, self.eps_root = b1, b2, eps, eps_root
        self.mu = {k: torch.zeros_like(p) for k, p in self.params.items()}
        self.nu = {k: torch.zeros_like(p) for k, p in self.params.items()}
        self.count = 0
        self._dev = _lib.require_gpu(*self.params.values())

    def _groups(self, grads: Mapping[str, torch.Tensor] | None, count: int):
        keys = list(self.params)
        arr = (_lib.AdamGroup * len(keys))()
        keep = []
        for i, k in enumerate(keys):
            p = self.params[k]
            g = None
            if grads is not None:
                g = grads[k]
                if g.shape != p.shape or g.dtype != torch.float32:
                    raise ValueError(f"gradient of {k!r} must be float32 of shape "
                                     f"{tuple(p.shape)}, got {g.dtype} {tuple(g.shape)}")
                g = g.contiguous()
                keep.append(g)
            lr = self.lr[k]
            lr = lr(count) if callable(lr) else lr
            arr[i] = _lib.AdamGroup(p.data_ptr(), 0 if g is None else g.data_ptr(),
                                    self.mu[k].data_ptr(), self.nu[k].data_ptr(), p.numel(),
                                    float(lr))
        return arr, keep

    def step(self, grads: Mapping[str, torch.Tensor],
             maps: Mapping[str, int] | None = None) -> None:
        """One update of every group (learning-rate schedules see the pre-increment count).

        ``maps`` names, per group, the parameter map whose output ``grads`` differentiates
        (MAP_EXP, MAP_SIGMOID, MAP_QUAT; groups not named take MAP_NONE): the update then applies
        the map's reverse-mode rule at the parameters before the update, bit for bit as
        render_log's own backward does, in the same launch."""
        arr, keep = self._groups(grads, self.count)
        self.count += 1
        map_arr = None
        if maps is not None:
            unknown = set(maps) - set(self.params)
            if unknown:
                raise ValueError(f"maps name groups {sorted(unknown)} that do not exist")
            map_arr = (ctypes.c_int32 * len(arr))(*[int(maps.get(k, MAP_NONE))
                                                    for k in self.params])
        with torch.cuda.device(self._dev):
            st = _lib.lib().splat_adam_step_mapped(
                _lib.stream_handle(self._dev), ctypes.addressof(arr), len(arr),
                None if map_arr is None else ctypes.addressof(map_arr), self.b1, self.b2,
                self.eps, self.eps_root, self.count)
        _lib.check(st, "adam_step")
        del keep

    def reset_rows(self, reset: torch.Tensor) -> None:
        """Zero mu and nu of the rows flagged in ``reset`` (bool or uint8, one per row)."""
        rows = reset.numel()
        # a bool tensor holds one byte per row, 0 or 1: read as uint8 without a cast kernel
        mask = reset.contiguous()
        mask = mask.view(torch.uint8) if mask.dtype == torch.bool else mask.to(torch.uint8)
        arr, _ = self._groups(None, self.count)
        with torch.cuda.device(self._dev):
            st = _lib.lib().splat_adam_reset_rows(
                _lib.stream_handle(self._dev), ctypes.addressof(arr), len(arr), mask.data_ptr(), rows)
        _lib.check(st, "adam_reset_rows")
