"""ORACLE — test infrastructure only.

The reference engine's benchmark sequence on the checker build (oracle/_ref/libpinfer_refq4k.so:
the reference's own engine sources with the oracle's Q4K operators). Used by tests/ as the
end-to-end checker and by bench.py's cpu_baseline leg as the timed CPU baseline; the product
never imports it.

bench_generate follows engine/tools/pinfer_run.c:384-430: pf_spec_prefill of the prompt, then
pf_spec_decode of exactly n_gen tokens with EOS disabled (engine/src/spec.h:86-105), each phase
timed with the host clock.
"""
from __future__ import annotations

import ctypes
import time
from dataclasses import dataclass
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REFQ4K = HERE / "_ref" / "libpinfer_refq4k.so"


class _Params(ctypes.Structure):
    """pinfer_params (engine/include/pinfer.h:40-48)."""
    _fields_ = [("n_threads", ctypes.c_int), ("max_ctx", ctypes.c_int),
                ("kv_dtype", ctypes.c_int), ("gpu_split", ctypes.c_float)]


class _SpecParams(ctypes.Structure):
    """pinfer_spec_params (engine/include/pinfer.h:76-93)."""
    _fields_ = [("k", ctypes.c_int), ("draft_vocab", ctypes.c_int), ("adaptive", ctypes.c_int),
                ("ngram", ctypes.c_int)]


class _SpecStats(ctypes.Structure):
    """pinfer_spec_stats (engine/include/pinfer.h:95-102)."""
    _fields_ = [(f, ctypes.c_int64) for f in ("rounds", "drafted", "accepted", "ngram_rounds",
                                              "ngram_drafted", "ngram_accepted")]


class _Stop(ctypes.Structure):
    """pf_stop (engine/src/spec.h:89-96)."""
    _fields_ = [("eos", ctypes.c_int), ("stop_ids", ctypes.c_void_p), ("n_stop", ctypes.c_int),
                ("on_token", ctypes.c_void_p), ("user", ctypes.c_void_p)]


@dataclass
class RefRun:
    tokens: list[int]
    rounds: int
    drafted: int
    accepted: int
    prefill_s: float
    decode_s: float
    state: bytes | None
    next_logits: np.ndarray | None = None


def _lib(path: Path = REFQ4K) -> ctypes.CDLL:
    if not path.exists():
        raise FileNotFoundError(f"{path} not built (make -C oracle ref)")
    L = ctypes.CDLL(str(path))
    vp, i = ctypes.c_void_p, ctypes.c_int
    L.pinfer_default_params.restype = _Params
    L.pinfer_load.restype, L.pinfer_load.argtypes = vp, [ctypes.c_char_p, vp, vp]
    L.pinfer_free.restype, L.pinfer_free.argtypes = None, [vp]
    L.pf_spec_prefill.restype, L.pf_spec_prefill.argtypes = i, [vp, vp, i, vp, i]
    L.pf_spec_decode.restype, L.pf_spec_decode.argtypes = i, [vp] * 8
    L.pinfer_state_size.restype, L.pinfer_state_size.argtypes = ctypes.c_size_t, [vp]
    L.pinfer_state_save.restype, L.pinfer_state_save.argtypes = i, [vp, vp, ctypes.c_size_t]
    L.pinfer_eval.restype, L.pinfer_eval.argtypes = i, [vp, vp, i, vp]
    L.pinfer_n_vocab.restype, L.pinfer_n_vocab.argtypes = i, [vp]
    return L


def bench_generate(path: str | Path, prompt: np.ndarray, n_gen: int, k: int, draft_vocab: int,
                   threads: int, max_ctx: int = 1024, want_state: bool = False,
                   lib: Path = REFQ4K, next_logits: bool = False) -> RefRun:
    """Prefill `prompt`, then exactly n_gen tokens at draft count k (EOS ignored) on `threads`
    host threads; with want_state, the state blob (pinfer_state_save) after the decode; with
    next_logits, then the logits of feeding the last generated token (pinfer_eval)."""
    L = _lib(lib)
    p = L.pinfer_default_params()
    p.max_ctx, p.n_threads = max_ctx, threads
    err = ctypes.c_int(0)
    ctx = L.pinfer_load(str(path).encode(), ctypes.byref(p), ctypes.byref(err))
    if not ctx:
        raise RuntimeError(f"reference pinfer_load failed: {err.value}")
    try:
        prompt = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(n_gen, np.int32)
        sp, st = _SpecParams(k, draft_vocab, 0, 0), _SpecStats()
        stop, status = _Stop(-1, None, 0, None, None), ctypes.c_int(0)
        t0 = time.perf_counter()
        rc = L.pf_spec_prefill(ctx, prompt.ctypes.data, prompt.size, ctypes.byref(sp), 0)
        t1 = time.perf_counter()
        if rc < 0:
            raise RuntimeError(f"reference prefill failed: {rc}")
        n = L.pf_spec_decode(ctx, out.ctypes.data, n_gen, ctypes.byref(sp), ctypes.byref(stop),
                             ctypes.byref(st), None, ctypes.byref(status))
        t2 = time.perf_counter()
        if n != n_gen or status.value != 0:
            raise RuntimeError(f"reference decode failed: {n} tokens, status {status.value}")
        blob = None
        if want_state:
            size = L.pinfer_state_size(ctx)
            buf = ctypes.create_string_buffer(size)
            if L.pinfer_state_save(ctx, buf, size) != 0:
                raise RuntimeError("reference pinfer_state_save failed")
            blob = buf.raw
        logits = None
        if next_logits:
            logits = np.zeros(L.pinfer_n_vocab(ctx), np.float32)
            last = np.array([out[-1]], np.int32)
            if L.pinfer_eval(ctx, last.ctypes.data, 1, logits.ctypes.data) != 0:
                raise RuntimeError("reference pinfer_eval failed")
        return RefRun([int(x) for x in out], st.rounds, st.drafted, st.accepted, t1 - t0,
                      t2 - t1, blob, logits)
    finally:
        L.pinfer_free(ctx)
