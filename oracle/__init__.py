"""ORACLE — test infrastructure only.

ctypes loader of the scalar C restatement (oracle/lib/liboracle.so) and, when it was built,
of the reference engine's own portable sources (oracle/_ref/libpinfer_ref.so). Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package, and only as
the checker or the timed CPU baseline. The product never imports it.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "lib" / "liboracle.so"
REF = HERE / "_ref" / "libpinfer_ref.so"

_vp, _i, _f = ctypes.c_void_p, ctypes.c_int, ctypes.c_float


class LinArgs(ctypes.Structure):
    """Mirror of orc_lin_args (oracle.h)."""

    _fields_ = [("n", _i), ("heads", _i), ("rep", _i), ("dk", _i), ("dv", _i),
                ("qkv_stride", _i), ("o_stride", _i), ("qkv", _vp), ("decay", _vp),
                ("beta", _vp), ("S", _vp), ("o", _vp), ("log", _vp), ("pend", _vp),
                ("keep", _i), ("log0", _i)]


class RefLinArgs(ctypes.Structure):
    """Mirror of the reference's pf_lin_args (engine/src/ops.h:69-82)."""

    _fields_ = [("n", _i), ("heads", _i), ("rep", _i), ("dk", _i), ("dv", _i),
                ("qkv_stride", _i), ("o_stride", _i), ("qkv", _vp), ("decay", _vp),
                ("beta", _vp), ("S", _vp), ("o", _vp), ("log", _vp), ("pend", _vp),
                ("keep", _i), ("work", _vp)]


_SIGS = {
    "orc_f32_to_f16": (ctypes.c_uint16, [_f]),
    "orc_f16_to_f32": (_f, [ctypes.c_uint16]),
    "orc_q4k_nbytes": (ctypes.c_size_t, [_i, _i]),
    "orc_get6": (_i, [_vp, _i]),
    "orc_q4k_get_row": (None, [_vp, _i, _i, _i, _vp]),
    "orc_q4k_quantize": (None, [_vp, _i, _i, _vp]),
    "orc_quant_a8": (None, [_vp, _i, _i, _vp, _vp, _vp]),
    "orc_q4k_matmul": (None, [_vp, _i, _i, _vp, _vp, _vp, _i, _vp, _vp]),
    "orc_q4k_matmul_mt": (None, [_vp, _i, _i, _vp, _vp, _vp, _i, _vp, _i]),
    "orc_lin_rule": (None, [ctypes.POINTER(LinArgs)]),
    "orc_lin_apply": (None, [_vp, _vp, _i, _i, _i, _i]),
    "orc_argmax": (_i, [_vp, _i]),
    "orc_accept": (_i, [_vp, _i, _vp, _i, _vp, _vp]),
    "orc_expf_cephes": (_f, [_f]),
    "orc_top1_prob": (_f, [_vp, _i]),
    "orc_gate_expf": (_f, [_f]),
    "orc_gate_log1pf": (_f, [_f]),
    "orc_libm_mismatches": (ctypes.c_longlong, [_i, _i]),
    "orc_libm_eval": (None, [_i, ctypes.c_uint32, ctypes.c_long, _vp, _i]),
    "orc_exp2_tab": (ctypes.c_uint64, [_i]),
}

_lib = None
_ref = None


def build() -> None:
    """make -C oracle (and the reference build when its sources are present)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    if Path("/root/reference/engine/src").is_dir():
        subprocess.run(["make", "-s", "-C", str(HERE), "ref"], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = ctypes.CDLL(str(LIB))
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args
        _lib = L
    return _lib


def ref_lib() -> ctypes.CDLL | None:
    """The reference's own portable engine, or None where it was not built."""
    global _ref
    if _ref is None and REF.exists():
        R = ctypes.CDLL(str(REF))
        R.pf_lin_rule.restype, R.pf_lin_rule.argtypes = None, [_vp, ctypes.POINTER(RefLinArgs)]
        R.pf_lin_apply.restype, R.pf_lin_apply.argtypes = None, [_vp, _vp, _vp, _i, _i, _i, _i]
        R.pf_expf.restype, R.pf_expf.argtypes = _f, [_f]
        R.pf_argmax.restype, R.pf_argmax.argtypes = _i, [_vp, _i]
        R.pf_softmax_max.restype, R.pf_softmax_max.argtypes = _f, [_vp, _i]
        R.pf_softmax_exp.restype, R.pf_softmax_exp.argtypes = _f, [_vp, _i, _f]
        _ref = R
    return _ref


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


# ---- numpy-facing helpers --------------------------------------------------------------
def q4k_nbytes(rows: int, cols: int) -> int:
    return int(lib().orc_q4k_nbytes(rows, cols))


def q4k_quantize(w: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    out = np.zeros(q4k_nbytes(rows, cols), np.uint8)
    lib().orc_q4k_quantize(_ptr(w), rows, cols, _ptr(out))
    return out


def q4k_get_row(W: np.ndarray, rows: int, cols: int, row: int) -> np.ndarray:
    out = np.empty(cols, np.float32)
    lib().orc_q4k_get_row(_ptr(W), rows, cols, row, _ptr(out))
    return out


def quant_a8(X: np.ndarray):
    X = np.ascontiguousarray(X, np.float32)
    n, cols = X.shape
    q = np.empty((cols // 32, n, 32), np.int8)
    d = np.empty((cols // 32, n), np.float32)
    fs = np.empty((cols // 32, n), np.float32)
    lib().orc_quant_a8(_ptr(X), n, cols, _ptr(q), _ptr(d), _ptr(fs))
    return q, d, fs


def q4k_matmul(W: np.ndarray, rows: int, cols: int, q, d, fs, n: int, want_dots=False,
               threads: int = 0):
    Y = np.empty((n, rows), np.float32)
    dots = np.empty((n, rows, cols // 32), np.int32) if want_dots else None
    if threads:
        lib().orc_q4k_matmul_mt(_ptr(W), rows, cols, _ptr(q), _ptr(d), _ptr(fs), n, _ptr(Y),
                                threads)
    else:
        lib().orc_q4k_matmul(_ptr(W), rows, cols, _ptr(q), _ptr(d), _ptr(fs), n, _ptr(Y),
                             _ptr(dots))
    return (Y, dots) if want_dots else Y


def lin_rule(qkv, decay, beta, S, *, n, heads, rep, dk, dv, log=False, pend=None, keep=0,
             log0=False):
    """Returns (S_after, o, log) as new arrays; inputs are not modified."""
    S = np.array(S, np.float32, copy=True)
    qkv = np.ascontiguousarray(qkv, np.float32)
    decay = np.ascontiguousarray(decay, np.float32)
    beta = np.ascontiguousarray(beta, np.float32)
    o = np.zeros((n, heads * dv), np.float32)
    lg = np.zeros((n, heads, dk + dv + 1), np.float32) if log else None
    pend = None if pend is None else np.ascontiguousarray(pend, np.float32)
    a = LinArgs(n, heads, rep, dk, dv, qkv.shape[1], heads * dv, _ptr(qkv), _ptr(decay),
                _ptr(beta), _ptr(S), _ptr(o), _ptr(lg), _ptr(pend), keep, int(log0))
    lib().orc_lin_rule(ctypes.byref(a))
    return S, o, lg


def lin_apply(S, log, keep, heads, dk, dv):
    S = np.array(S, np.float32, copy=True)
    log = np.ascontiguousarray(log, np.float32)
    lib().orc_lin_apply(_ptr(S), _ptr(log), keep, heads, dk, dv)
    return S


def top1_prob(logits: np.ndarray) -> np.float32:
    l = np.ascontiguousarray(logits, np.float32)
    return np.float32(lib().orc_top1_prob(_ptr(l), l.size))


def argmax(v: np.ndarray) -> int:
    v = np.ascontiguousarray(v, np.float32)
    return int(lib().orc_argmax(_ptr(v), v.size))


def accept(logits: np.ndarray, drafts: np.ndarray):
    logits = np.ascontiguousarray(logits, np.float32)
    k = logits.shape[0] - 1
    drafts = np.ascontiguousarray(drafts, np.int32)
    bonus = ctypes.c_int32()
    rows = np.empty(k + 1, np.int32)
    a = lib().orc_accept(_ptr(logits), logits.shape[1], _ptr(drafts), k, ctypes.byref(bonus),
                         _ptr(rows))
    return int(a), int(bonus.value), rows
