"""The DeltaNet state's device layout: the library's nmx_state_index (host code, no GPU needed)
equals the restatement in tests/refmath.py, which is a bijection onto [0, heads dk dv) for every
supported dk and for value widths that leave a partial group of 16 columns."""
from __future__ import annotations

import numpy as np
import pytest

from nibblemac_amd import nmx
from tests.refmath import state_from_dev, state_offsets, state_to_dev


@pytest.mark.parametrize("dk", [32, 64, 128, 256])
@pytest.mark.parametrize("dv", [1, 8, 16, 20, 32, 48, 128])
def test_layout_matches_library_and_is_a_permutation(dk, dv):
    heads = 3
    off = state_offsets(heads, dk, dv)
    assert np.array_equal(np.sort(off.ravel()), np.arange(heads * dk * dv))
    lib = nmx.load_library()
    for h in range(heads):
        for j in range(dv):
            for i in range(0, dk, max(1, dk // 16)):
                assert lib.nmx_state_index(h, j, i, dk, dv) == off[h, j, i], (h, j, i)


def test_round_trip():
    rng = np.random.default_rng(3)
    S = rng.standard_normal((4, 128, 20)).astype(np.float32)
    assert np.array_equal(state_from_dev(state_to_dev(S, 4, 128, 20), 4, 128, 20), S)


def test_wave_slot_is_contiguous():
    """a wave (16 full columns, 64 lanes) reads slot k of every lane as one 1 KB run"""
    off = state_offsets(1, 128, 128)
    for k in range(8):
        lanes = [off[0, j, 32 * c + 4 * k] for j in range(16) for c in range(4)]
        assert lanes == [k * 256 + 4 * l for l in range(64)]
