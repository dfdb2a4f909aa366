"""Build recipe of the gfx950 library ``splax_amd/libsplat_hip.so``.

Compiles every ``csrc/*.hip`` with hipcc for gfx950 only and links one shared library exporting
the C ABI declared in ``include/splat_hip.h``. Flags:
- ``-ffp-contract=off``: no implicit FMA; results follow the written arithmetic exactly.
- ``-munsafe-fp-atomics``: float atomicAdd lowers to the native global / LDS add instructions.
- ``-target-feature -packed-fp32-ops``: no packed-FP32 instructions are generated.
"""

from __future__ import annotations

import os
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "libsplat_hip.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

CXXFLAGS = [
    "-O3", "-fPIC", "-std=c++17", f"--offload-arch={ARCH}", "-ffp-contract=off",
    "-munsafe-fp-atomics", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-command-line-argument",
]


# Per-file additions. blend.hip: its LDS adds come from a few lanes at known-distinct or
# single-lane addresses, where the atomic optimizer's lane-by-lane readlane loop only adds VALU
# work to a VALU-bound kernel.
EXTRA_FLAGS = {
    "blend.hip": ["-mllvm", "-amdgpu-atomic-optimizer-strategy=None"],
}


def build(verbose: bool = False) -> Path:
    """Compile and link the library (always rebuilds)."""
    sources = sorted(CSRC.glob("*.hip"))
    objdir = PKG / "_obj"
    objdir.mkdir(exist_ok=True)

    def compile_one(src: Path) -> Path:
        obj = objdir / (src.stem + ".o")
        cmd = [HIPCC, *CXXFLAGS, *EXTRA_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr}")
        noise = [ln for ln in res.stderr.splitlines() if "packed-fp32-ops" not in ln]
        if verbose and any(noise):
            print("\n".join(noise))
        return obj

    workers = min(len(sources), int(os.environ.get("MAX_JOBS", "8")))
    with ThreadPoolExecutor(max_workers=max(1, workers)) as ex:
        objs = list(ex.map(compile_one, sources))
    tmp = LIB.with_suffix(f".so.tmp{os.getpid()}")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    tmp.replace(LIB)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
