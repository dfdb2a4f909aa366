"""Build recipe for the CPU oracle (test infrastructure only).

Compiles ``oracle/splat_oracle.c`` into ``oracle/liboracle.so`` with strict IEEE float semantics
(no FMA contraction, no fast-math), the arithmetic contract the GPU library is compared against.

The reference (amacati/splax) is pure Python over NVIDIA Warp and jaxlib wheels; none of its
render-path code is C/C++ source, so there is nothing to compile into ``oracle/_ref`` and the
oracle is pinned by closed forms, brute force, autograd and finite differences instead.
"""

from __future__ import annotations

import os
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "splat_oracle.c"
LIB = HERE / "liboracle.so"


def _has_fma() -> bool:
    try:
        return " fma " in Path("/proc/cpuinfo").read_text()
    except OSError:
        return False


def build(verbose: bool = False) -> Path:
    """Compile the oracle shared library (always recompiles)."""
    flags = ["-O3", "-fPIC", "-shared", "-std=c11", "-ffp-contract=off", "-fno-fast-math"]
    flags += ["-fopenmp", "-Wall", "-Wno-unused-function", "-Wno-unknown-pragmas"]
    if _has_fma():
        flags.append("-mfma")  # explicit fmaf() becomes one instruction; no contraction otherwise
    tmp = LIB.with_suffix(f".so.tmp{os.getpid()}")
    cmd = ["gcc", *flags, "-o", str(tmp), str(SRC), "-lm"]
    if verbose:
        print(" ".join(cmd))
    subprocess.run(cmd, check=True)
    tmp.replace(LIB)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
