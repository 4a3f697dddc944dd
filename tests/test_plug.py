"""Host part of the reference-engine operator plug (nibblemac_amd/csrc/plug/matvec_nmx.c, built
with the reference's engine objects into oracle/_ref/libpinfer_nmxplug.so): its Q4K embedding
row decoder, pf_get_row (kern_get_row_q, engine/src/kern_act.c:53-88), against the oracle's, on
quantized random rows and on hand-set fp16 scales (subnormal, negative, largest finite,
infinite, NaN). Bar: bit-exact (NaN where the oracle gives NaN). The device parts of the plug
are in test_gpu_plug.py."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle
from oracle import HERE as ORACLE_DIR

PLUG = ORACLE_DIR / "_ref" / "libpinfer_nmxplug.so"
pytestmark = pytest.mark.skipif(not PLUG.exists(), reason="oracle/_ref not built (reference "
                                "absent when the tree was built)")

PQ_Q4K_G32 = 4


class PfMat(ctypes.Structure):
    """Mirror of pf_mat (engine/src/ops.h:16-20)."""

    _fields_ = [("dtype", ctypes.c_uint32), ("rows", ctypes.c_int), ("cols", ctypes.c_int),
                ("data", ctypes.c_void_p)]


def plug_get_row(W: np.ndarray, rows: int, cols: int, row: int) -> np.ndarray:
    L = ctypes.CDLL(str(PLUG))
    L.pf_get_row.restype = None
    L.pf_get_row.argtypes = [ctypes.POINTER(PfMat), ctypes.c_int, ctypes.c_void_p]
    m = PfMat(PQ_Q4K_G32, rows, cols, W.ctypes.data)
    out = np.empty(cols, np.float32)
    L.pf_get_row(ctypes.byref(m), row, out.ctypes.data)
    return out


def same_bits(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    nan = np.isnan(b)
    assert np.array_equal(np.isnan(a), nan)
    assert np.array_equal(a.view(np.uint32)[~nan], b.view(np.uint32)[~nan])


def test_get_row_quantized():
    rng = np.random.default_rng(21)
    rows, cols = 12, 768
    W = oracle.q4k_quantize(rng.standard_normal((rows, cols)).astype(np.float32) * 0.05)
    for r in range(rows):
        same_bits(plug_get_row(W, rows, cols, r), oracle.q4k_get_row(W, rows, cols, r))


def test_get_row_special_scales():
    """Each superblock's D (bytes 2r..2r+1) and M (8+2r..) of every row r set to fp16 patterns
    the quantizer never writes."""
    rng = np.random.default_rng(22)
    rows, cols = 8, 1024
    W = oracle.q4k_quantize(rng.standard_normal((rows, cols)).astype(np.float32))
    pats = np.array([0x0001, 0x03FF, 0x8001, 0x7BFF, 0xFBFF, 0x7C00, 0xFC00, 0x7E00, 0x0000,
                     0x8000, 0x3C00, 0x0400], np.uint16)
    sb = W.reshape(-1, 576)
    for i in range(sb.shape[0]):
        h = sb[i, :16].view(np.uint16)
        h[:] = pats[rng.integers(0, pats.size, 8)]
    for r in range(rows):
        same_bits(plug_get_row(W, rows, cols, r), oracle.q4k_get_row(W, rows, cols, r))
