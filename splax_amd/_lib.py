"""ctypes binding of ``libsplat_hip.so`` (the C ABI in ``include/splat_hip.h``).

The library is loaded from this package directory only (built in-tree by ``splax_amd._build``).
There is no fallback: a missing library, or a call without a ROCm GPU, raises.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libsplat_hip.so"

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_f32 = ctypes.c_float
_f64 = ctypes.c_double
_u64 = ctypes.c_uint64


class AdamGroup(ctypes.Structure):
    """splat_adam_group (include/splat_hip.h)."""
    _fields_ = [("params", _vp), ("grads", _vp), ("mu", _vp), ("nu", _vp), ("size", _i64),
                ("lr", _f64)]


# name -> argtypes, in the order of include/splat_hip.h
_SIGS = {
    "splat_project_fwd": [_vp] + [_vp, _i64] * 6 + [_vp, _i32, _i32, _i32, _i64, _i32, _i32]
    + [_f32] * 6 + [_vp] * 6 + [_i32],
    "splat_project_fwd_noalloc": [_vp] + [_vp, _i64] * 6 + [_vp, _i32, _i32, _i32, _i64, _i32,
                                                         _i32] + [_f32] * 6 + [_vp] * 6 + [_i32],
    "splat_project_bwd": [_vp] + [_vp, _i64] * 10 + [_vp, _i32, _i32, _i32, _i32, _f32, _f32,
                                                     _f32] + [_vp] * 5 + [_i32, _i32],
    "splat_rasterize_fwd": [_vp] + [_vp, _i64] * 4 + [_vp] * 5 + [_i32] * 4 + [_vp] * 4,
    "splat_rasterize_depth_fwd": [_vp] + [_vp, _i64] * 4 + [_vp] * 5 + [_i32] * 4 + [_vp] * 5,
    "splat_rasterize_bwd": [_vp] + [_vp, _i64] * 4 + [_vp] * 5 + [_vp, _vp, _vp, _i64]
    + [_i32] * 5 + [_vp] * 4,
    "splat_rasterize_depth_bwd": [_vp] + [_vp, _i64] * 4 + [_vp] * 5 + [_vp, _vp, _vp, _i64]
    + [_vp, _i64] + [_i32] * 5 + [_vp] * 5,
    "splat_rasterize_fwd_keep": [_vp] + [_vp, _i64] * 4 + [_vp] * 5 + [_i32] * 4 + [_i64]
    + [_vp] * 10 + [_i32],
    "splat_rasterize_bwd_sorted": [_vp] + [_vp, _i64] * 3 + [_vp] * 9 + [_i64]
    + [_vp, _vp, _vp, _i64] + [_vp, _i64] + [_i32] * 5 + [_vp] * 5 + [_i32, _i32],
    "splat_sort_and_bin": [_vp] + [_vp] * 4 + [_vp, _i64, _vp] + [_i32] * 4
    + [_vp, _vp, _i64, _vp, _vp],
    "splat_set_wide_keys": [_i32],
    "splat_render_fwd": [_vp] + [_vp, _i64] * 8 + [_vp] + [_i32] * 6 + [_f32] * 6
    + [_i32, _i32] + [_vp] * 6 + [_i64] + [_vp] * 10 + [_vp, _i32, _vp],
    "splat_render_bwd": [_vp] + [_vp, _i64] * 8 + [_vp] + [_i32] * 6 + [_f32] * 3
    + [_i32, _i32] + [_vp] * 10 + [_i64] + [_vp] * 3 + [_i64, _vp, _i64] + [_vp] * 7 + [_i32]
    + [_vp, _i32, _vp, _vp],
    "splat_adam_step": [_vp, _vp, _i32, _f64, _f64, _f64, _f64, _i64],
    "splat_adam_step_mapped": [_vp, _vp, _i32, _vp, _f64, _f64, _f64, _f64, _i64],
    "splat_adam_reset_rows": [_vp, _vp, _i32, _vp, _i64],
    "splat_mcmc_relocate": [_vp] + [_vp] * 5 + [_i64, _i32, _f32, _u64, _vp, _vp],
    "splat_mcmc_compute_relocation": [_vp, _vp, _vp, _vp, _i64, _i32, _vp, _vp],
    "splat_mcmc_inject_noise": [_vp] + [_vp] * 4 + [_i64, _f32, _f32, _u64, _vp, _vp],
    "splat_log_params_fwd": [_vp] + [_vp] * 4 + [_i64] + [_vp] * 4,
    "splat_log_params_bwd": [_vp] + [_vp] * 4 + [_i64] + [_vp] * 8,
    "splat_l1_loss_fwd": [_vp, _vp, _vp, _i64, _vp, _vp],
    "splat_l1_loss_bwd": [_vp, _vp, _vp, _i64, _vp, _vp],
    "splat_mse_loss_fwd": [_vp, _vp, _vp, _i64, _vp, _vp],
    "splat_mse_loss_bwd": [_vp, _vp, _vp, _i64, _vp, _vp],
    "splat_clear_cache": [],
    "splat_last_error": [],
    "splat_set_stage_timing": [_i32],
    "splat_get_stage_times": [_vp, _vp, _i32],
    "splat_check_device": [],
    "splat_abi_version": [],
}

STAGES = ("project", "minmax", "emit", "sort", "bins", "blend_fwd", "blend_bwd", "project_bwd",
          "blend_fwd_kernel", "blend_bwd_kernel")

# splat_abi_version() of the library this binding was written for (include/splat_hip.h)
ABI_VERSION = 17

# status codes (splax_amd/csrc/splat_internal.hpp)
ERR_ARGS, ERR_KEY_OVERFLOW, ERR_TOO_MANY = 1, 2, 6


class SplatError(RuntimeError):
    pass


def lib() -> ctypes.CDLL:
    """Load the gfx950 library (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise ImportError(
                    f"{LIB_PATH} is missing: build it with `python -m splax_amd._build` "
                    "(or __graft_entry__.build())")
            handle = ctypes.CDLL(str(LIB_PATH))
            for name, args in _SIGS.items():
                fn = getattr(handle, name)
                fn.argtypes = args
                fn.restype = ctypes.c_int
            handle.splat_last_error.restype = ctypes.c_char_p
            handle.splat_clear_cache.restype = None
            version = handle.splat_abi_version()
            if version != ABI_VERSION:
                raise ImportError(
                    f"{LIB_PATH} has ABI version {version}, this binding expects "
                    f"{ABI_VERSION}: rebuild it with `python -m splax_amd._build`")
            _lib = handle
    return _lib


def check(status: int, what: str) -> None:
    if status == 0:
        return
    msg = lib().splat_last_error().decode(errors="replace")
    if status in (ERR_ARGS, ERR_KEY_OVERFLOW):
        raise ValueError(f"{what}: {msg}")
    raise SplatError(f"{what} failed (status {status}): {msg}")


def require_gpu(*tensors: torch.Tensor) -> torch.device:
    """All tensors must live on one ROCm device; returns it."""
    if not torch.cuda.is_available():
        raise RuntimeError("splax_amd needs a ROCm GPU (torch.cuda.is_available() is False)")
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise ValueError(f"expected a GPU tensor, got one on {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    if dev is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    return dev


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def set_stage_timing(stages=None) -> None:
    """Bracket the named stages (all when True, none when False/empty) with HIP events."""
    if stages is True:
        stages = STAGES
    mask = 0
    for name in (stages or ()):
        mask |= 1 << STAGES.index(name)
    lib().splat_set_stage_timing(mask)


def stage_times() -> dict[str, tuple[float, int]]:
    """Summed milliseconds and call counts per stage since the last query (then reset)."""
    ms = (ctypes.c_double * len(STAGES))()
    calls = (ctypes.c_int64 * len(STAGES))()
    check(lib().splat_get_stage_times(ms, calls, len(STAGES)), "stage_times")
    return {s: (ms[i], calls[i]) for i, s in enumerate(STAGES)}


def set_wide_keys(force: bool) -> None:
    """Make every sort take the 64-bit key (the reference's tests patch _use_32bit_keys,
    splax/_rasterize/_sort/_sort.py:23-26, the same way)."""
    lib().splat_set_wide_keys(int(bool(force)))


def check_device() -> int:
    """Wait for the current device; return (and clear) its device error word (0 = healthy)."""
    return int(lib().splat_check_device())


def clear_cache() -> None:
    """Release the library's persistent per-device scratch (splax/_cache.py:158-164)."""
    if LIB_PATH.exists():
        lib().splat_clear_cache()
