"""ctypes binding of libnmx.so (include/nmx.h): the MI355X device layer.

Used by the Python tests and bench.py; the C host engine (libpinfer.so) links the same library
directly. There is no fallback: if libnmx.so is missing or no GPU is present the calls raise.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

LIB_DIR = Path(__file__).resolve().parent / "lib"

_vp = ctypes.c_void_p
_i = ctypes.c_int
_sz = ctypes.c_size_t
_fp = ctypes.POINTER(ctypes.c_float)

NMX_MAX_SEGS = 6


class NmxError(RuntimeError):
    pass


class LinArgs(ctypes.Structure):
    """Mirror of nmx_lin_args (include/nmx.h)."""

    _fields_ = [("n", _i), ("heads", _i), ("rep", _i), ("dk", _i), ("dv", _i),
                ("qkv_stride", _i), ("o_stride", _i), ("qkv", _vp), ("decay", _vp),
                ("beta", _vp), ("S", _vp), ("o", _vp), ("log", _vp), ("pend", _vp),
                ("keep", _i), ("log0", _i), ("keep_dev", _vp)]


class LinPreArgs(ctypes.Structure):
    """Mirror of nmx_lin_pre_args (include/nmx.h)."""

    _fields_ = [("n", _i), ("C", _i), ("conv_k", _i), ("dk", _i), ("kd", _i), ("raw", _vp),
                ("raw_stride", _i), ("out", _vp), ("state", _vp), ("conv_w", _vp), ("xin", _vp),
                ("qscale", ctypes.c_float), ("l2eps", ctypes.c_float), ("b_in", _vp),
                ("a_in", _vp), ("g_stride", _i), ("heads", _i), ("A_log", _vp), ("A", _vp),
                ("dt_bias", _vp), ("beta", _vp), ("decay", _vp)]


class A8(ctypes.Structure):
    """Mirror of nmx_a8: block-major int8 codes, per-block scale d and d * sum(codes)."""

    _fields_ = [("q", _vp), ("d", _vp), ("fs", _vp)]


class NormIn(ctypes.Structure):
    """Mirror of nmx_norm_in (the RMSNorm input of a fused matmul)."""

    _fields_ = [("x", _vp), ("x_stride", _i), ("add", _vp), ("add_stride", _i), ("x_out", _vp),
                ("xo_stride", _i), ("w", _vp), ("eps", ctypes.c_float)]


class LinMixArgs(ctypes.Structure):
    """Mirror of nmx_lin_mix_args."""

    _fields_ = [("pre", LinPreArgs), ("rule", LinArgs), ("z", _vp), ("z_stride", _i),
                ("norm_w", _vp), ("eps", ctypes.c_float), ("y", _vp), ("y_stride", _i),
                ("a8", A8)]


class CommitArgs(ctypes.Structure):
    """Mirror of nmx_commit_args (the rollback commit of every linear layer)."""

    _fields_ = [("layers", _i), ("C", _i), ("conv_k", _i), ("state", _vp), ("xin", _vp),
                ("log", _vp), ("pend", _vp), ("cap", _i), ("row", _i), ("ctl", _vp), ("vt", _vp),
                ("state_bak", _vp), ("redo", _i)]


class AcceptKeys(ctypes.Structure):
    """Mirror of nmx_accept_keys (the acceptance resolved from the head's partial keys)."""

    _fields_ = [("keys", _vp), ("nkeys", _i), ("n", _i), ("drafts", _vp), ("out", _vp),
                ("mailbox", _vp), ("nvt", _i)]


class AttnArgs(ctypes.Structure):
    """Mirror of nmx_attn_args (gated full attention over the KV caches)."""

    _fields_ = [("n", _i), ("nh", _i), ("nkv", _i), ("hd", _i), ("rot", _i), ("max_ctx", _i),
                ("q", _vp), ("k_in", _vp), ("v_in", _vp), ("q_norm", _vp), ("k_norm", _vp),
                ("eps", ctypes.c_float), ("scale", ctypes.c_float), ("rope_cos", _vp),
                ("rope_sin", _vp), ("kc", _vp), ("vc", _vp), ("pos", _vp), ("pos_off", _i),
                ("o", _vp), ("a8", A8), ("scores", _vp), ("kv_dtype", _i)]


_SIGS: dict[str, tuple[object, list[object]]] = {
    "nmx_create": (_vp, [_i]),
    "nmx_create_error": (ctypes.c_char_p, []),
    "nmx_destroy": (None, [_vp]),
    "nmx_error": (ctypes.c_char_p, [_vp]),
    "nmx_device_name": (ctypes.c_char_p, [_vp]),
    "nmx_device_count": (_i, []),
    "nmx_alloc": (_vp, [_vp, _sz]),
    "nmx_free": (_i, [_vp, _vp]),
    "nmx_upload": (_i, [_vp, _vp, _vp, _sz]),
    "nmx_download": (_i, [_vp, _vp, _vp, _sz]),
    "nmx_copy_d2d": (_i, [_vp, _vp, _vp, _sz]),
    "nmx_fill_zero": (_i, [_vp, _vp, _sz]),
    "nmx_sync": (_i, [_vp]),
    "nmx_event_create": (_vp, [_vp]),
    "nmx_event_destroy": (None, [_vp]),
    "nmx_event_record": (_i, [_vp, _vp]),
    "nmx_event_elapsed_ms": (_i, [_vp, _vp, _vp, _fp]),
    "nmx_graph_begin": (_i, [_vp]),
    "nmx_graph_end": (_vp, [_vp]),
    "nmx_graph_launch": (_i, [_vp, _vp]),
    "nmx_graph_destroy": (None, [_vp]),
    "nmx_quant_a8": (_i, [_vp, _vp, _i, _i, _vp, _vp, _vp]),
    "nmx_q4k_matmul": (_i, [_vp, _vp, _i, _i, _i, _vp, _vp, _vp, _vp, _i, _vp]),
    "nmx_q4k_matmul_multi": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _i, _i, _vp, _vp, _vp]),
    "nmx_lin_rule": (_i, [_vp, ctypes.POINTER(LinArgs)]),
    "nmx_lin_apply": (_i, [_vp, _vp, _vp, _i, _i, _i, _i]),
    "nmx_state_index": (_sz, [_i, _i, _i, _i, _i]),
    "nmx_head_work_bytes": (_sz, [_i, _i]),
    "nmx_head_accept": (_i, [_vp, _vp, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "nmx_head_accept_to": (_i, [_vp, _vp, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "nmx_head_row_accept_to": (_i, [_vp, _vp, _i, _i, _vp, _i, _vp, _i, _vp, ctypes.c_float, _vp,
                                    _i, _i, _vp, _vp, _vp, _vp, A8, _vp]),
    "nmx_head_accept_noalloc": (_i, [_vp, _vp, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp]),
    "nmx_head_accept_commit": (_i, [_vp, _vp, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                    _vp, _vp, _i]),
    "nmx_accept_commit": (_i, [_vp, _vp, _vp, _vp]),
    "nmx_head_nkeys": (_i, [_i, _i, _i]),
    "nmx_gate_eval": (_i, [_vp, _i, ctypes.c_uint32, ctypes.c_long, _vp]),
    "nmx_head_keys": (_i, [_vp, _vp, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp]),
    "nmx_lin_commit": (_i, [_vp, ctypes.POINTER(CommitArgs)]),
    "nmx_lin_commit_keys": (_i, [_vp, ctypes.POINTER(CommitArgs), ctypes.POINTER(AcceptKeys)]),
    "nmx_accept_commit_mb": (_i, [_vp, _vp, _vp, _vp, _vp, _i]),
    "nmx_host_alloc": (_vp, [_vp, _sz]),
    "nmx_embed_norm": (_i, [_vp, _vp, _i, _vp, _i, _i, ctypes.c_float, _vp, _vp, _i, _vp, _i, A8,
                            _vp, _i, _vp, _vp, _i, A8]),
    "nmx_host_free": (_i, [_vp, _vp]),
    "nmx_rmsnorm_row": (_i, [_vp, _vp, _i, _vp, _i, _vp, _i, ctypes.c_float, _vp, _i, _i, _vp,
                             A8]),
    "nmx_rmsnorm_xo": (_i, [_vp, _vp, _i, _vp, _i, _vp, _i, _vp, _i, _i, ctypes.c_float, _vp, _i,
                            A8]),
    "nmx_silu_mul": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp, A8]),
    "nmx_q4k_matmul_embed_norm": (_i, [_vp, _vp, _i, _vp, _i, _i, _i, _vp, _i, _vp, _vp, _vp,
                                       _i, _vp, ctypes.c_float, A8, _vp, _i]),
    "nmx_head_row_keys": (_i, [_vp, _vp, _i, _i, _vp, _i, _vp, _i, _vp, ctypes.c_float, _vp, _i,
                               _i, _vp, _vp]),
    "nmx_head_row_nkeys": (_i, [_i]),
    "nmx_embed_norm_keys": (_i, [_vp, _vp, _i, _vp, _i, _i, ctypes.c_float, _vp, _vp, _i, A8,
                                 _vp, _i]),
    "nmx_q4k_matmul_norm": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _i, _i, ctypes.POINTER(NormIn),
                                 A8]),
    "nmx_lin_pre": (_i, [_vp, ctypes.POINTER(LinPreArgs)]),
    "nmx_lin_post": (_i, [_vp, _vp, _i, _vp, _i, _vp, _i, _i, _i, ctypes.c_float, _vp, _i, A8]),
    "nmx_lin_mix": (_i, [_vp, ctypes.POINTER(LinMixArgs)]),
    "nmx_attn_prep": (_i, [_vp, ctypes.POINTER(AttnArgs)]),
    "nmx_attn": (_i, [_vp, ctypes.POINTER(AttnArgs)]),
    "nmx_attn_fused": (_i, [_vp, ctypes.POINTER(AttnArgs)]),
    "nmx_q4k_swiglu": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp, _vp, _vp, ctypes.POINTER(NormIn),
                            _vp, A8, A8, _vp, _vp]),
    "nmx_top1_gate": (_i, [_vp, _vp, _i, ctypes.c_float, _vp]),
    "nmx_kv_bytes": (_sz, [_i, _i, _i, _i]),
}

_lib: ctypes.CDLL | None = None


def library_path() -> Path:
    return LIB_DIR / "libnmx.so"


def load_library() -> ctypes.CDLL:
    """Load libnmx.so from the package (built by nibblemac_amd.build); raises if absent."""
    global _lib
    if _lib is not None:
        return _lib
    path = library_path()
    if not path.exists():
        raise NmxError(f"{path} is missing: run `python -m nibblemac_amd.build` first")
    lib = ctypes.CDLL(str(path))
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def exported_symbols() -> list[str]:
    return list(_SIGS)


class Buffer:
    """A device allocation: pointer, size, and an optional numpy dtype/shape."""

    def __init__(self, dev: "Device", ptr: int, nbytes: int, dtype=None, shape=None):
        self.dev, self.ptr, self.nbytes = dev, ptr, nbytes
        self.dtype, self.shape = dtype, shape

    def offset(self, nbytes: int) -> int:
        return self.ptr + nbytes

    def numpy(self) -> np.ndarray:
        return self.dev.download(self, self.dtype, self.shape)

    def free(self) -> None:
        if self.ptr:
            self.dev.free(self)
            self.ptr = 0


class Device:
    """One nmx context (device + stream)."""

    def __init__(self, device: int = 0):
        self.lib = load_library()
        self.ctx = self.lib.nmx_create(device)
        if not self.ctx:
            raise NmxError(self.lib.nmx_create_error().decode())
        self._bufs: list[Buffer] = []

    # ---- errors / lifetime
    def check(self, rc: int, what: str = "nmx call") -> None:
        if rc != 0:
            raise NmxError(f"{what}: {self.lib.nmx_error(self.ctx).decode()}")

    @property
    def name(self) -> str:
        return self.lib.nmx_device_name(self.ctx).decode()

    def close(self) -> None:
        if self.ctx:
            for b in self._bufs:
                if b.ptr:
                    self.lib.nmx_free(self.ctx, b.ptr)
                    b.ptr = 0
            self.lib.nmx_destroy(self.ctx)
            self.ctx = None

    def __enter__(self) -> "Device":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    # ---- memory
    def alloc(self, nbytes: int, dtype=None, shape=None) -> Buffer:
        p = self.lib.nmx_alloc(self.ctx, max(int(nbytes), 1))
        if not p:
            raise NmxError(f"nmx_alloc({nbytes}): {self.lib.nmx_error(self.ctx).decode()}")
        b = Buffer(self, p, int(nbytes), dtype, shape)
        self._bufs.append(b)
        return b

    def empty(self, shape, dtype) -> Buffer:
        dt = np.dtype(dtype)
        shape = tuple(int(s) for s in np.atleast_1d(shape)) if not isinstance(shape, tuple) else shape
        return self.alloc(int(np.prod(shape)) * dt.itemsize, dt, shape)

    def zeros(self, shape, dtype) -> Buffer:
        b = self.empty(shape, dtype)
        self.check(self.lib.nmx_fill_zero(self.ctx, b.ptr, b.nbytes), "fill_zero")
        return b

    def to_device(self, arr: np.ndarray) -> Buffer:
        arr = np.ascontiguousarray(arr)
        b = self.alloc(arr.nbytes, arr.dtype, arr.shape)
        if arr.nbytes:
            self.check(self.lib.nmx_upload(self.ctx, b.ptr, arr.ctypes.data, arr.nbytes), "upload")
        return b

    def upload(self, b: Buffer, arr: np.ndarray) -> None:
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= b.nbytes
        self.check(self.lib.nmx_upload(self.ctx, b.ptr, arr.ctypes.data, arr.nbytes), "upload")

    def download(self, b: Buffer, dtype=None, shape=None) -> np.ndarray:
        dtype = np.dtype(dtype if dtype is not None else b.dtype)
        shape = shape if shape is not None else b.shape
        out = np.empty(shape, dtype)
        self.check(self.lib.nmx_download(self.ctx, out.ctypes.data, b.ptr, out.nbytes), "download")
        return out

    def free(self, b: Buffer) -> None:
        self.check(self.lib.nmx_free(self.ctx, b.ptr), "free")

    def copy(self, dst, src, nbytes: int) -> None:
        """Device-to-device copy of nbytes on the context's stream."""
        self.check(self.lib.nmx_copy_d2d(self.ctx, _p(dst), _p(src), nbytes), "copy")

    def sync(self) -> None:
        self.check(self.lib.nmx_sync(self.ctx), "sync")

    # ---- timing / graphs
    def event(self) -> int:
        e = self.lib.nmx_event_create(self.ctx)
        if not e:
            raise NmxError("event create failed")
        return e

    def record(self, ev: int) -> None:
        self.check(self.lib.nmx_event_record(self.ctx, ev), "event record")

    def elapsed_ms(self, e0: int, e1: int) -> float:
        ms = ctypes.c_float()
        self.check(self.lib.nmx_event_elapsed_ms(self.ctx, e0, e1, ctypes.byref(ms)), "elapsed")
        return float(ms.value)

    def graph_begin(self) -> None:
        self.check(self.lib.nmx_graph_begin(self.ctx), "graph begin")

    def graph_end(self) -> int:
        g = self.lib.nmx_graph_end(self.ctx)
        if not g:
            raise NmxError(f"graph end: {self.lib.nmx_error(self.ctx).decode()}")
        return g

    def graph_destroy(self, g: int) -> None:
        self.lib.nmx_graph_destroy(g)

    def graph_launch(self, g: int) -> None:
        self.check(self.lib.nmx_graph_launch(self.ctx, g), "graph launch")

    # ---- kernels
    def quant_a8(self, X: Buffer | int, n: int, cols: int, q: Buffer | int, d: Buffer | int,
                 fs: Buffer | int) -> None:
        self.check(self.lib.nmx_quant_a8(self.ctx, _p(X), n, cols, _p(q), _p(d), _p(fs)),
                   "quant_a8")

    def q4k_matmul(self, W, rows: int, cols: int, n: int, q, d, fs, Y, y_stride: int | None = None,
                   dots=None) -> None:
        self.check(self.lib.nmx_q4k_matmul(self.ctx, _p(W), rows, cols, n, _p(q), _p(d), _p(fs),
                                           _p(Y), y_stride or rows, _p(dots) if dots else None),
                   "q4k_matmul")

    def q4k_matmul_multi(self, Ws, rows, Ys, y_strides, cols: int, n: int, q, d, fs) -> None:
        c = len(Ws)
        w = (ctypes.c_void_p * c)(*[_p(x) for x in Ws])
        r = (ctypes.c_int * c)(*rows)
        y = (ctypes.c_void_p * c)(*[_p(x) for x in Ys])
        s = (ctypes.c_int * c)(*y_strides)
        self.check(self.lib.nmx_q4k_matmul_multi(self.ctx, c, w, r, y, s, cols, n, _p(q), _p(d),
                                                 _p(fs)), "q4k_matmul_multi")


    def rmsnorm(self, x, n: int, cols: int, w, eps: float, *, add=None, xo=None, y=None,
                a8=(None, None, None)) -> None:
        """Rows [n][cols] (contiguous): xo = x + add (if given), y / a8 of rmsnorm(...) * w."""
        self.check(self.lib.nmx_rmsnorm_xo(self.ctx, _p(x), cols, _p(add), cols, _p(xo), cols,
                                           _p(w), n, cols, eps, _p(y), cols,
                                           A8(*[_p(t) for t in a8])), "rmsnorm")

    def rmsnorm_row(self, x, nrows: int, cols: int, w, eps: float, idx, off: int, *, add=None,
                    y=None, a8=(None, None, None)) -> None:
        """nmx_rmsnorm_row: the norm of row idx[0] + off (read on the device) of contiguous
        rows [nrows][cols] (+ add) into y [cols] and a one-vector A8."""
        self.check(self.lib.nmx_rmsnorm_row(self.ctx, _p(x), cols, _p(add), cols, _p(w), cols,
                                            eps, _p(idx), off, nrows, _p(y),
                                            A8(*[_p(t) for t in a8])), "rmsnorm_row")

    def embed_norm(self, E, vocab: int, tok, n: int, cols: int, eps: float, w0, *, xo0=None,
                   y0=None, a0=(None, None, None), x1=None, w1=None, y1=None,
                   a1=(None, None, None)) -> None:
        """nmx_embed_norm on contiguous rows: Q4K embedding rows tok -> xo0, norm -> y0 / a0,
        and an optional second norm of x1 -> y1 / a1."""
        self.check(self.lib.nmx_embed_norm(self.ctx, _p(E), vocab, _p(tok), n, cols, eps, _p(w0),
                                           _p(xo0), cols, _p(y0), cols, A8(*[_p(t) for t in a0]),
                                           _p(x1), cols, _p(w1), _p(y1), cols,
                                           A8(*[_p(t) for t in a1])), "embed_norm")

    def q4k_matmul_embed_norm(self, W, rows: int, Y, n: int, H: int, E, vocab: int, tok, w_emb,
                              h, w_hid, eps: float, a8_tmp=(None, None, None), tok_keys=None,
                              nkeys: int = 0) -> None:
        """nmx_q4k_matmul_embed_norm on contiguous rows: Y [n][rows] = W x A8 of
        [rmsnorm(embed(tok), w_emb) | rmsnorm(h, w_hid)]; with tok_keys (one row) the token is
        the argmax of the nkeys partial keys, written to tok[0]."""
        self.check(self.lib.nmx_q4k_matmul_embed_norm(self.ctx, _p(W), rows, _p(Y), rows, n, H,
                                                      _p(E), vocab, _p(tok), _p(w_emb), _p(h),
                                                      H, _p(w_hid), eps,
                                                      A8(*[_p(t) for t in a8_tmp]),
                                                      _p(tok_keys), nkeys),
                   "q4k_matmul_embed_norm")

    def head_row_keys(self, W, rows: int, cols: int, x, nrows: int, w, eps: float, idx, off: int,
                      keys, *, add=None, y=None) -> None:
        """nmx_head_row_keys: the one-row head's partial argmax keys (no reduction)."""
        self.check(self.lib.nmx_head_row_keys(self.ctx, _p(W), rows, cols, _p(x), cols, _p(add),
                                              cols, _p(w), eps, _p(idx), off, nrows, _p(y),
                                              _p(keys)), "head_row_keys")

    def head_row_nkeys(self, rows: int) -> int:
        return self.lib.nmx_head_row_nkeys(rows)

    def embed_norm_keys(self, E, vocab: int, tok, n: int, cols: int, eps: float, w, keys,
                        nkeys: int, *, xo=None, a8=(None, None, None)) -> None:
        """nmx_embed_norm_keys: nmx_embed_norm (one set) with row n - 1's token from keys."""
        self.check(self.lib.nmx_embed_norm_keys(self.ctx, _p(E), vocab, _p(tok), n, cols, eps,
                                                _p(w), _p(xo), cols, A8(*[_p(t) for t in a8]),
                                                _p(keys), nkeys), "embed_norm_keys")

    def silu_mul(self, gate, up, n: int, cols: int, y=None, a8=(None, None, None)) -> None:
        self.check(self.lib.nmx_silu_mul(self.ctx, _p(gate), _p(up), cols, n, cols, _p(y),
                                         A8(*[_p(t) for t in a8])), "silu_mul")

    def q4k_matmul_norm(self, Ws, rows, Ys, cols: int, n: int, x, w, eps: float, *, add=None,
                        xo=None, a8_tmp=(None, None, None)) -> None:
        c = len(Ws)
        arr = lambda t, xs: (t * c)(*xs)  # noqa: E731
        nin = NormIn(_p(x), cols, _p(add), cols, _p(xo), cols, _p(w), eps)
        self.check(self.lib.nmx_q4k_matmul_norm(
            self.ctx, c, arr(ctypes.c_void_p, [_p(t) for t in Ws]), arr(ctypes.c_int, rows),
            arr(ctypes.c_void_p, [_p(t) for t in Ys]), arr(ctypes.c_int, rows), cols, n,
            ctypes.byref(nin), A8(*[_p(t) for t in a8_tmp])), "q4k_matmul_norm")

    def q4k_swiglu(self, Wg, Wu, ffn: int, cols: int, n: int, out, *, a8=(None, None, None),
                   norm=None, y=None, a8_tmp=(None, None, None), gate_tmp=None,
                   up_tmp=None) -> None:
        """norm: (x, w, eps, add, xo) for the fused RMSNorm input, else the A8 input a8."""
        nin = None
        if norm is not None:
            x, w, eps, add, xo = norm
            nin = ctypes.byref(NormIn(_p(x), cols, _p(add), cols, _p(xo), cols, _p(w), eps))
        q, d, fs = [_p(t) for t in a8]
        self.check(self.lib.nmx_q4k_swiglu(self.ctx, _p(Wg), _p(Wu), ffn, cols, n, q, d, fs, nin,
                                           _p(y), A8(*[_p(t) for t in out]),
                                           A8(*[_p(t) for t in a8_tmp]), _p(gate_tmp),
                                           _p(up_tmp)), "q4k_swiglu")

    def lin_rule(self, *, n, heads, rep, dk, dv, qkv_stride, o_stride, qkv, decay, beta, S, o,
                 log=None, pend=None, keep=0, log0=False) -> None:
        a = LinArgs(n, heads, rep, dk, dv, qkv_stride, o_stride, _p(qkv), _p(decay), _p(beta),
                    _p(S), _p(o), _p(log), _p(pend), keep, int(log0), None)
        self.check(self.lib.nmx_lin_rule(self.ctx, ctypes.byref(a)), "lin_rule")

    def lin_pre(self, args: "LinPreArgs") -> None:
        self.check(self.lib.nmx_lin_pre(self.ctx, ctypes.byref(args)), "lin_pre")

    def lin_post(self, o, o_stride, z, z_stride, w, n, heads, dv, eps, y=None, y_stride=0,
                 a8=(None, None, None)) -> None:
        self.check(self.lib.nmx_lin_post(self.ctx, _p(o), o_stride, _p(z), z_stride, _p(w), n,
                                         heads, dv, eps, _p(y), y_stride,
                                         A8(*[_p(t) for t in a8])), "lin_post")

    def attn_prep(self, args: "AttnArgs") -> None:
        self.check(self.lib.nmx_attn_prep(self.ctx, ctypes.byref(args)), "attn_prep")

    def attn(self, args: "AttnArgs") -> None:
        self.check(self.lib.nmx_attn(self.ctx, ctypes.byref(args)), "attn")

    def attn_fused(self, args: "AttnArgs") -> None:
        """nmx_attn_fused: nmx_attn_prep + nmx_attn in two launches."""
        self.check(self.lib.nmx_attn_fused(self.ctx, ctypes.byref(args)), "attn_fused")

    def lin_mix(self, args: "LinMixArgs") -> None:
        self.check(self.lib.nmx_lin_mix(self.ctx, ctypes.byref(args)), "lin_mix")

    def lin_apply(self, S, log, keep: int, heads: int, dk: int, dv: int) -> None:
        self.check(self.lib.nmx_lin_apply(self.ctx, _p(S), _p(log), keep, heads, dk, dv),
                   "lin_apply")

    def head_work_bytes(self, rows: int, n: int) -> int:
        return int(self.lib.nmx_head_work_bytes(rows, n))

    def head_accept(self, W, rows: int, cols: int, n: int, q, d, fs, logits, drafts, work,
                    out, tok_dst=None) -> None:
        """nmx_head_accept, or nmx_head_accept_to when tok_dst (a device int32) is given."""
        if tok_dst is None:
            rc = self.lib.nmx_head_accept(self.ctx, _p(W), rows, cols, n, _p(q), _p(d), _p(fs),
                                          _p(logits), _p(drafts), _p(work), _p(out))
        else:
            rc = self.lib.nmx_head_accept_to(self.ctx, _p(W), rows, cols, n, _p(q), _p(d), _p(fs),
                                             _p(logits), _p(drafts), _p(work), _p(out), _p(tok_dst))
        self.check(rc, "head_accept")

    def head_row_accept_to(self, W, rows: int, cols: int, x, nrows: int, w, eps: float, idx,
                           off: int, work, out, tok_dst, *, add=None, y=None,
                           a8_tmp=(None, None, None), advance=None) -> None:
        """nmx_head_row_accept_to: the one-row head on the RMSNorm of row idx[0] + off of
        contiguous rows x [nrows][cols] (+ add), the norm inside the head's workgroups;
        advance (int32 control block): advance[0] += advance[1] after the head."""
        self.check(self.lib.nmx_head_row_accept_to(self.ctx, _p(W), rows, cols, _p(x), cols,
                                                   _p(add), cols, _p(w), eps, _p(idx), off, nrows,
                                                   _p(y), _p(work), _p(out), _p(tok_dst),
                                                   A8(*[_p(t) for t in a8_tmp]), _p(advance)),
                   "head_row_accept_to")

    def head_accept_noalloc(self, W, rows: int, cols: int, n: int, q, d, fs, logits, drafts,
                            out) -> None:
        """nmx_head_accept_noalloc: the head with its scratch in the library's static array."""
        self.check(self.lib.nmx_head_accept_noalloc(self.ctx, _p(W), rows, cols, n, _p(q), _p(d),
                                                    _p(fs), _p(logits), _p(drafts), _p(out)),
                   "head_accept_noalloc")

    def head_accept_commit(self, W, rows: int, cols: int, n: int, q, d, fs, drafts, work, out,
                           vt, ctl, mailbox=None, nvt: int = 0) -> None:
        """nmx_head_accept_commit: the head, the acceptance and the commit of the accepted run
        (vt, ctl and, when given, the host mailbox) in one launch sequence."""
        self.check(self.lib.nmx_head_accept_commit(self.ctx, _p(W), rows, cols, n, _p(q), _p(d),
                                                   _p(fs), _p(drafts), _p(work), _p(out), _p(vt),
                                                   _p(ctl), mailbox, nvt), "head_accept_commit")

    def gate_eval(self, which: int, first: int, n: int, y) -> None:
        """nmx_gate_eval: the device's gate exp (0) / log1p (1) of n consecutive bit patterns."""
        self.check(self.lib.nmx_gate_eval(self.ctx, which, first, n, _p(y)), "gate_eval")

    def head_nkeys(self, rows: int, cols: int, n: int) -> int:
        """nmx_head_nkeys: partial argmax keys per row of nmx_head_keys."""
        return int(self.lib.nmx_head_nkeys(rows, cols, n))

    def head_keys(self, W, rows: int, cols: int, n: int, q, d, fs, drafts, work,
                  drafts_copy) -> None:
        """nmx_head_keys: the verify head's dots and partial argmax keys, drafts copied."""
        self.check(self.lib.nmx_head_keys(self.ctx, _p(W), rows, cols, n, _p(q), _p(d), _p(fs),
                                          _p(drafts), _p(work), _p(drafts_copy)), "head_keys")

    def lin_commit(self, args: CommitArgs, keys: AcceptKeys | None = None) -> None:
        """nmx_lin_commit, or nmx_lin_commit_keys with the acceptance from keys."""
        if keys is None:
            rc = self.lib.nmx_lin_commit(self.ctx, ctypes.byref(args))
        else:
            rc = self.lib.nmx_lin_commit_keys(self.ctx, ctypes.byref(args), ctypes.byref(keys))
        self.check(rc, "lin_commit")

    def accept_commit(self, out, vt, ctl, mailbox=None, nvt: int = 0) -> None:
        """nmx_accept_commit, or nmx_accept_commit_mb writing the host mailbox."""
        if mailbox is None:
            rc = self.lib.nmx_accept_commit(self.ctx, _p(out), _p(vt), _p(ctl))
        else:
            rc = self.lib.nmx_accept_commit_mb(self.ctx, _p(out), _p(vt), _p(ctl), mailbox, nvt)
        self.check(rc, "accept_commit")

    def host_alloc(self, nbytes: int) -> int:
        """Page-locked host memory kernels may write (nmx_host_alloc); free with host_free."""
        p = self.lib.nmx_host_alloc(self.ctx, nbytes)
        if not p:
            raise NmxError(f"nmx_host_alloc({nbytes}): {self.lib.nmx_error(self.ctx).decode()}")
        return p

    def host_free(self, p: int) -> None:
        self.check(self.lib.nmx_host_free(self.ctx, p), "host_free")


    def top1_gate(self, logits, n: int, tau: float, flag) -> None:
        """flag[0] = top-1 softmax probability of logits[0, n) >= tau (nmx_top1_gate)."""
        self.check(self.lib.nmx_top1_gate(self.ctx, _p(logits), n, tau, _p(flag)), "top1_gate")


def _p(x) -> int | None:
    if x is None:
        return None
    return x.ptr if isinstance(x, Buffer) else int(x)
