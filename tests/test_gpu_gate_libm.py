"""GPU parity of the DeltaNet gates' exp / log1p (engine/src/forward_lin.c:18-19,59-66: the
reference calls the C library) against this host's C library itself, on every binary32 input.

The device functions (nibblemac_amd/csrc/hip/nmx_math.h: nmx_gate_expf, nmx_gate_log1pf, the
ones the mixer kernels call) run through nmx_gate_eval over all 2^32 bit patterns, 2^26 per
launch; the host values come from expf / log1pf themselves (oracle.orc_libm_eval, on this
box's glibc). Bar: bit-exact, NaN results matching NaN results.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

CHUNK = 1 << 26


@pytest.mark.parametrize("which,name", [(0, "expf"), (1, "log1pf")])
def test_device_gate_equals_host_libm_on_every_input(dev, which, name):
    print(f"[case] device {name} over 2^32 inputs", flush=True)
    L = oracle.lib()
    thr = max(1, min(16, len(os.sched_getaffinity(0))))
    y = dev.empty((CHUNK,), np.float32)
    ref = np.empty(CHUNK, np.float32)
    bad = 0
    try:
        for c in range((1 << 32) // CHUNK):
            first = c * CHUNK
            dev.gate_eval(which, first, CHUNK, y)
            L.orc_libm_eval(which, first, CHUNK, ref.ctypes.data_as(ctypes.c_void_p), thr)
            got = y.numpy()
            diff = got.view(np.uint32) != ref.view(np.uint32)
            if diff.any():
                diff &= ~(np.isnan(got) & np.isnan(ref))
                if diff.any() and not bad:
                    i = int(np.flatnonzero(diff)[0])
                    print(f"first mismatch: bits {first + i:08x}: {got[i]!r} vs {ref[i]!r}")
                bad += int(diff.sum())
    finally:
        y.free()
    assert bad == 0, f"{name}: {bad} inputs differ from the host C library"
