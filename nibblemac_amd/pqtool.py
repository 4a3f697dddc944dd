"""ctypes binding of the .pq tools in libpqtool.so (include/pqtool.h): seeded Gaussian weights
and the Q4K_G32 packer for synthetic random-init models."""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

LIB = Path(__file__).resolve().parent / "lib" / "libpqtool.so"
_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            raise RuntimeError(f"{LIB} is missing: run `python -m nibblemac_amd.build` first")
        L = ctypes.CDLL(str(LIB))
        u64, i, f, vp, sz = ctypes.c_uint64, ctypes.c_int, ctypes.c_float, ctypes.c_void_p, ctypes.c_size_t
        L.pqt_gauss.restype, L.pqt_gauss.argtypes = None, [u64, u64, u64, f, vp, sz]
        L.pqt_quantize_q4k.restype, L.pqt_quantize_q4k.argtypes = i, [vp, i, i, vp]
        L.pqt_gauss_q4k.restype, L.pqt_gauss_q4k.argtypes = i, [u64, u64, i, i, f, vp, i]
        _lib = L
    return _lib


def q4k_nbytes(rows: int, cols: int) -> int:
    return rows // 4 * (cols // 256) * 576


def gauss(seed: int, stream: int, n: int, std: float = 1.0, first: int = 0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().pqt_gauss(seed, stream, first, std, out.ctypes.data, n)
    return out


def quantize_q4k(w: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    out = np.empty(q4k_nbytes(rows, cols), np.uint8)
    if lib().pqt_quantize_q4k(w.ctypes.data, rows, cols, out.ctypes.data) != 0:
        raise ValueError(f"bad Q4K shape {w.shape}")
    return out


def gauss_q4k(seed: int, stream: int, rows: int, cols: int, std: float = 0.02,
              threads: int | None = None) -> np.ndarray:
    out = np.empty(q4k_nbytes(rows, cols), np.uint8)
    threads = threads or min(16, len(os.sched_getaffinity(0)))
    if lib().pqt_gauss_q4k(seed, stream, rows, cols, std, out.ctypes.data, threads) != 0:
        raise ValueError(f"bad Q4K shape {rows}x{cols}")
    return out
