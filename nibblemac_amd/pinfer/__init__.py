"""Python face of the MI355X engine: the ctypes binding of libpinfer.so (see _lib) and a small
`Model` wrapper with eval / generate, mirroring the reference package's calls
(python/pinfer/model.py:229-244, :445-510; speculative.py:115-141)."""
from __future__ import annotations

import ctypes

import numpy as np

from ._lib import (GenOpts, Lib, LibraryNotFoundError, ON_TOKEN, Params, SpecParams,  # noqa: F401
                   SpecStats, load_library)

ERRORS = {-1: "E_IO", -2: "E_FORMAT", -3: "E_NOMEM", -4: "E_ARG", -5: "E_CTX_FULL"}


class PinferError(RuntimeError):
    def __init__(self, code: int, what: str):
        super().__init__(f"{what}: PINFER_{ERRORS.get(code, code)}")
        self.code = code


class Model:
    """A loaded .pq model on the MI355X."""

    def __init__(self, path: str, max_ctx: int = 4096, lib: Lib | None = None,
                 lib_path: str | None = None, n_threads: int | None = None, kv_dtype: int = 0):
        self.lib = lib or load_library(lib_path)
        p = self.lib.pinfer_default_params()
        p.max_ctx = max_ctx
        p.kv_dtype = kv_dtype  # PINFER_KV_F32 / F16 / I8
        if n_threads is not None:
            p.n_threads = n_threads
        err = ctypes.c_int(0)
        self.ctx = self.lib.pinfer_load(str(path).encode(), ctypes.byref(p), ctypes.byref(err))
        if not self.ctx:
            raise PinferError(err.value, f"pinfer_load({path})")
        self.n_vocab = self.lib.pinfer_n_vocab(self.ctx)

    def close(self) -> None:
        if self.ctx:
            self.lib.pinfer_free(self.ctx)
            self.ctx = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def n_past(self) -> int:
        return self.lib.pinfer_n_past(self.ctx)

    def reset(self) -> None:
        self.lib.pinfer_reset(self.ctx)

    def eval(self, tokens, logits: bool = True) -> np.ndarray | None:
        t = np.ascontiguousarray(tokens, np.int32)
        out = np.empty(self.n_vocab, np.float32) if logits else None
        rc = self.lib.pinfer_eval(self.ctx, t.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
                                  t.size, out.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
                                  if logits else None)
        if rc != 0:
            raise PinferError(rc, "pinfer_eval")
        return out

    def generate(self, prompt, n_max: int, k: int = 0, draft_vocab: int = 32768,
                 cont: bool = False, stop_ids=(), adaptive: int = 0,
                 ngram: int = 0) -> tuple[list[int], SpecStats]:
        """Greedy generation (pinfer_generate_greedy_ex, or _cont with cont=True): k MTP drafts
        per verify pass (0 = plain), prompt-lookup drafts of up to `ngram` tokens, the adaptive
        policy flag; returns the tokens and the speculative statistics."""
        t = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(n_max, np.int32)
        sp = SpecParams(k, draft_vocab, adaptive, ngram)
        st = SpecStats()
        status = ctypes.c_int(0)
        stops = np.ascontiguousarray(stop_ids, np.int32)
        opts = GenOpts(stops.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)) if stops.size else None,
                       int(stops.size), ON_TOKEN(0), None)
        fn = self.lib.pinfer_generate_greedy_cont if cont else self.lib.pinfer_generate_greedy_ex
        n = fn(self.ctx, t.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), t.size,
               out.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), n_max, ctypes.byref(sp),
               ctypes.byref(opts), ctypes.byref(st), ctypes.byref(status))
        if n < 0 or (status.value != 0 and n == 0):
            raise PinferError(status.value or n, "pinfer_generate_greedy")
        return [int(x) for x in out[:n]], st

    def default_spec_params(self) -> dict:
        """pinfer_default_spec_params() as a dict (k, draft_vocab, adaptive, ngram)."""
        sp = self.lib.pinfer_default_spec_params()
        return {"k": sp.k, "draft_vocab": sp.draft_vocab, "adaptive": sp.adaptive,
                "ngram": sp.ngram}

    def state_save(self) -> bytes:
        """The context state as a blob (pinfer_state_save)."""
        n = self.lib.pinfer_state_size(self.ctx)
        buf = ctypes.create_string_buffer(n)
        rc = self.lib.pinfer_state_save(self.ctx, buf, n)
        if rc != 0:
            raise PinferError(rc, "pinfer_state_save")
        return buf.raw

    def state_load(self, blob: bytes) -> None:
        rc = self.lib.pinfer_state_load(self.ctx, blob, len(blob))
        if rc != 0:
            raise PinferError(rc, "pinfer_state_load")

    def checkpoint(self) -> None:
        rc = self.lib.pinfer_checkpoint(self.ctx)
        if rc != 0:
            raise PinferError(rc, "pinfer_checkpoint")

    def rewind(self) -> None:
        rc = self.lib.pinfer_rewind(self.ctx)
        if rc != 0:
            raise PinferError(rc, "pinfer_rewind")

    @property
    def checkpoint_n_past(self) -> int:
        return self.lib.pinfer_checkpoint_n_past(self.ctx)

    def bench_generate(self, prompt, n_gen: int, k: int = 4, draft_vocab: int = 32768,
                       adaptive: int = 0, ngram: int = 0):
        """The reference CLI's benchmark timing (engine/tools/pinfer_run.c:384-430): reset,
        prefill, then exactly n_gen tokens with EOS ignored. Returns (tokens, stats, prefill
        seconds, decode seconds); decode tok/s is (n_gen - 1) / decode seconds."""
        if self.lib.pinfer_bench_generate is None:
            raise PinferError(-4, f"{self.lib.path} has no pinfer_bench_generate")
        t = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(n_gen, np.int32)
        sp, st = SpecParams(k, draft_vocab, adaptive, ngram), SpecStats()
        tp, td = ctypes.c_double(0.0), ctypes.c_double(0.0)
        n = self.lib.pinfer_bench_generate(
            self.ctx, t.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), t.size,
            out.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), n_gen, ctypes.byref(sp),
            ctypes.byref(st), ctypes.byref(tp), ctypes.byref(td))
        if n != n_gen:
            raise PinferError(n if n < 0 else -4, f"pinfer_bench_generate returned {n}")
        return [int(x) for x in out], st, tp.value, td.value
