"""ctypes binding of libpinfer.so (include/pinfer.h), with the struct mirrors and symbol table
of the reference's Python binding (python/pinfer/_lib.py:34-170), so code written against the
reference's `pinfer` package finds the same names.

Search order: the `path` argument, PINFER_LIB, then nibblemac_amd/lib/libpinfer.so.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path
from typing import Any

_PKG_LIB = Path(__file__).resolve().parent.parent / "lib" / "libpinfer.so"


class Params(ctypes.Structure):
    """pinfer_params: n_threads, max_ctx, kv_dtype, gpu_split."""
    _fields_ = [("n_threads", ctypes.c_int), ("max_ctx", ctypes.c_int),
                ("kv_dtype", ctypes.c_int), ("gpu_split", ctypes.c_float)]


class SpecParams(ctypes.Structure):
    """pinfer_spec_params: k, draft_vocab, adaptive, ngram."""
    _fields_ = [("k", ctypes.c_int), ("draft_vocab", ctypes.c_int), ("adaptive", ctypes.c_int),
                ("ngram", ctypes.c_int)]


class SpecStats(ctypes.Structure):
    """pinfer_spec_stats."""
    _fields_ = [("rounds", ctypes.c_int64), ("drafted", ctypes.c_int64),
                ("accepted", ctypes.c_int64), ("ngram_rounds", ctypes.c_int64),
                ("ngram_drafted", ctypes.c_int64), ("ngram_accepted", ctypes.c_int64)]


_c_float_p = ctypes.POINTER(ctypes.c_float)
_c_int32_p = ctypes.POINTER(ctypes.c_int32)
_c_int_p = ctypes.POINTER(ctypes.c_int)
ON_TOKEN = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_int32, ctypes.c_void_p)


class GenOpts(ctypes.Structure):
    """pinfer_gen_opts: stop_ids, n_stop, on_token, user."""
    _fields_ = [("stop_ids", _c_int32_p), ("n_stop", ctypes.c_int), ("on_token", ON_TOKEN),
                ("user", ctypes.c_void_p)]


_REQUIRED = {
    "pinfer_default_params": (Params, []),
    "pinfer_load": (ctypes.c_void_p, [ctypes.c_char_p, ctypes.POINTER(Params), _c_int_p]),
    "pinfer_free": (None, [ctypes.c_void_p]),
    "pinfer_reset": (None, [ctypes.c_void_p]),
    "pinfer_eval": (ctypes.c_int, [ctypes.c_void_p, _c_int32_p, ctypes.c_int, _c_float_p]),
    "pinfer_n_vocab": (ctypes.c_int, [ctypes.c_void_p]),
    "pinfer_n_past": (ctypes.c_int, [ctypes.c_void_p]),
    "pinfer_eos_id": (ctypes.c_int, [ctypes.c_void_p]),
    "pinfer_argmax": (ctypes.c_int, [_c_float_p, ctypes.c_int]),
    "pinfer_version": (ctypes.c_char_p, []),
}
_GEN_EX = [ctypes.c_void_p, _c_int32_p, ctypes.c_int, _c_int32_p, ctypes.c_int,
           ctypes.POINTER(SpecParams), ctypes.POINTER(GenOpts), ctypes.POINTER(SpecStats), _c_int_p]
_OPTIONAL = {
    "pinfer_has_mtp": (ctypes.c_int, [ctypes.c_void_p]),
    "pinfer_default_spec_params": (SpecParams, []),
    "pinfer_generate_greedy": (ctypes.c_int, [ctypes.c_void_p, _c_int32_p, ctypes.c_int, _c_int32_p,
                                              ctypes.c_int, ctypes.POINTER(SpecParams),
                                              ctypes.POINTER(SpecStats)]),
    "pinfer_generate_greedy_ex": (ctypes.c_int, _GEN_EX),
    "pinfer_generate_greedy_cont": (ctypes.c_int, _GEN_EX),
    "pinfer_eval_select": (ctypes.c_int, [ctypes.c_void_p, _c_int32_p, ctypes.c_int, _c_int32_p,
                                          ctypes.c_int, _c_float_p]),
    "pinfer_state_size": (ctypes.c_size_t, [ctypes.c_void_p]),
    "pinfer_state_save": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]),
    "pinfer_state_load": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]),
    "pinfer_checkpoint": (ctypes.c_int, [ctypes.c_void_p]),
    "pinfer_rewind": (ctypes.c_int, [ctypes.c_void_p]),
    "pinfer_checkpoint_clear": (None, [ctypes.c_void_p]),
    "pinfer_checkpoint_n_past": (ctypes.c_int, [ctypes.c_void_p]),
    "pinfer_bench_generate": (ctypes.c_int, [ctypes.c_void_p, _c_int32_p, ctypes.c_int, _c_int32_p,
                                             ctypes.c_int, ctypes.POINTER(SpecParams),
                                             ctypes.POINTER(SpecStats),
                                             ctypes.POINTER(ctypes.c_double),
                                             ctypes.POINTER(ctypes.c_double)]),
}


class LibraryNotFoundError(OSError):
    pass


class Lib:
    """A loaded libpinfer.so with typed entry points (None for optional ones it lacks)."""

    def __init__(self, path: str, cdll: ctypes.CDLL) -> None:
        self.path, self.cdll = path, cdll
        for name, (res, args) in _REQUIRED.items():
            try:
                fn = getattr(cdll, name)
            except AttributeError as e:
                raise LibraryNotFoundError(f"{path}: missing symbol {name}") from e
            fn.restype, fn.argtypes = res, args
            setattr(self, name, fn)
        for name, (res, args) in _OPTIONAL.items():
            fn = getattr(cdll, name, None)
            if fn is not None:
                fn.restype, fn.argtypes = res, args
            setattr(self, name, fn)
        self.version: str = self.pinfer_version().decode()

    def has(self, name: str) -> bool:
        return hasattr(self.cdll, name)


_cache: dict[str, Lib] = {}


def load_library(path: str | os.PathLike[str] | None = None) -> Lib:
    cands = [os.fspath(path)] if path else [p for p in (os.environ.get("PINFER_LIB"),
                                                        str(_PKG_LIB)) if p]
    errors = []
    for cand in cands:
        if not os.path.exists(cand):
            errors.append(f"{cand}: not found")
            continue
        key = os.path.realpath(cand)
        if key not in _cache:
            _cache[key] = Lib(cand, ctypes.CDLL(cand))
        return _cache[key]
    raise LibraryNotFoundError("cannot load libpinfer.so: " + "; ".join(errors) +
                               " (build with `python -m nibblemac_amd.build`)")


