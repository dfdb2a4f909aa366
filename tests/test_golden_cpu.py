"""The oracle still reproduces the committed golden fixture bit for bit (regression guard)."""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

from conftest import assert_bit_exact

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
import make_golden  # noqa: E402

FIXTURE = Path(__file__).resolve().parent / "golden" / "tiny_render.npz"


def test_oracle_reproduces_golden_fixture():
    ref = np.load(FIXTURE)
    got = make_golden.make()
    for k in ref.files:
        if k in ("v_colors", "v_opac", "v_xy", "v_conic", "v_viewmat"):
            # double accumulation in a thread-dependent order: equal to the float32 rounding
            np.testing.assert_allclose(got[k], ref[k], rtol=1e-6, atol=1e-9, err_msg=k)
        else:
            assert_bit_exact(np.asarray(got[k]), ref[k], k)
    assert int(ref["cum"][-1]) == ref["keys"].size > 0
