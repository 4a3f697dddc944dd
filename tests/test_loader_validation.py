"""Loader validation of the .pq model file (libpinfer.so pinfer_load; the checks of the
reference loader, engine/src/model.c:60-202, tested the way tests/test_malformed.py tests the
reference): broken files made from a valid synthetic Q4K model by patching its header and
tensor directory (written as a sparse file of the real size, or a cut one) must be refused
with the right error code, and the loader's message must name the check that fired, so each
case proves its own check and not a later one.

Every check runs before any device call (pinfer_load validates the whole file first), so these
run on a host without a GPU: a refused file returns PINFER_E_FORMAT / PINFER_E_IO with no
device touched; the unpatched control passes every check and stops only at device creation
(PINFER_E_NOMEM here; it loads on a GPU host, where tests/test_gpu_e2e.py runs it)."""
from __future__ import annotations

import ctypes
import os
import struct
import tempfile
from pathlib import Path

import pytest

from nibblemac_amd import pqfile
from nibblemac_amd.pinfer import load_library

E_IO, E_FORMAT, E_NOMEM = -1, -2, -3
HDR = {"magic": (0, "8s"), "version": (8, "I"), "n_tensors": (12, "I"), "dir_offset": (16, "Q"),
       "data_offset": (24, "Q"), "arch": (32, "I"), "hidden": (36, "I"), "n_layers": (40, "I"),
       "vocab": (44, "I"), "ffn": (48, "I"), "n_heads": (52, "I"), "n_kv_heads": (56, "I"),
       "head_dim": (60, "I"), "rot_dim": (64, "I"), "lin_k_heads": (68, "I"),
       "lin_v_heads": (72, "I"), "lin_k_dim": (76, "I"), "lin_v_dim": (80, "I"),
       "conv_k": (84, "I"), "full_attn_mask": (88, "I"), "eos_id": (92, "I"),
       "tied_embeddings": (96, "I"), "has_mtp": (100, "I"), "rms_eps": (104, "f"),
       "rope_theta": (108, "f")}
ENT = {"dtype": (80, "I"), "ndim": (84, "I"), "offset": (104, "Q"), "nbytes": (112, "Q")}


class Pq:
    """The header + directory of a .pq file, patchable, written out as a sparse file."""

    def __init__(self, path: Path):
        self.size = path.stat().st_size
        with path.open("rb") as f:
            head = f.read(32)
            data_offset = struct.unpack_from("<Q", head, 24)[0]
            f.seek(0)
            self.buf = bytearray(f.read(data_offset))

    def copy(self):
        c = object.__new__(Pq)
        c.size, c.buf = self.size, bytearray(self.buf)
        return c

    def hdr(self, k):
        off, fmt = HDR[k]
        return struct.unpack_from("<" + fmt, self.buf, off)[0]

    def set_hdr(self, k, v):
        off, fmt = HDR[k]
        struct.pack_into("<" + fmt, self.buf, off, v)
        return self

    def at(self, name):
        base = self.hdr("dir_offset")
        for i in range(self.hdr("n_tensors")):
            o = base + 128 * i
            if bytes(self.buf[o:o + 80]).split(b"\0", 1)[0].decode() == name:
                return o
        raise KeyError(name)

    def get(self, name, k):
        off, fmt = ENT[k]
        return struct.unpack_from("<" + fmt, self.buf, self.at(name) + off)[0]

    def set(self, name, k, v):
        off, fmt = ENT[k]
        struct.pack_into("<" + fmt, self.buf, self.at(name) + off, v)
        return self

    def shape(self, name):
        return list(struct.unpack_from("<4I", self.buf, self.at(name) + 88))

    def set_shape(self, name, dims):
        struct.pack_into("<4I", self.buf, self.at(name) + 88, *(list(dims) + [0] * 4)[:4])
        return self

    def set_name(self, name, raw):
        o = self.at(name)
        self.buf[o:o + 80] = raw[:80].ljust(80, b"\0")
        return self

    def write(self, out: Path, size=None):
        with out.open("wb") as f:
            f.write(self.buf)
            f.truncate(self.size if size is None else size)
        return out


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    return Pq(pqfile.write_model(tmp_path_factory.mktemp("pq") / "small.pq", pqfile.SMALL, seed=3))


@pytest.fixture(scope="module")
def lib():
    return load_library(str(Path(__file__).resolve().parent.parent / "nibblemac_amd" / "lib" /
                            "libpinfer.so"))


def load(lib, path) -> tuple[int, str]:
    """pinfer_load's error code and what it wrote to stderr (fd 2)."""
    err = ctypes.c_int(0)
    p = lib.pinfer_default_params()
    p.max_ctx = 64
    with tempfile.TemporaryFile() as cap:
        saved = os.dup(2)
        os.dup2(cap.fileno(), 2)
        try:
            ctx = lib.pinfer_load(str(path).encode(), ctypes.byref(p), ctypes.byref(err))
        finally:
            os.dup2(saved, 2)
            os.close(saved)
        cap.seek(0)
        msg = cap.read().decode(errors="replace")
    if ctx:
        lib.pinfer_free(ctx)
    return err.value, msg


GATE = "layers.0.mlp.gate_proj.weight"
SB = 576


def cases():
    c = []

    def add(name, patch, code, text, size=None):
        c.append(pytest.param(patch, code, text, size, id=name))

    # file
    add("truncated", lambda p: p, E_FORMAT, "data out of bounds", lambda p: p.size - (1 << 16))
    add("truncated-header", lambda p: p, E_FORMAT, "too small", lambda p: 100)
    add("missing-file", None, E_IO, "No such file", None)
    add("bad-magic", lambda p: p.set_hdr("magic", b"PINFERX\0"), E_FORMAT, "bad magic")
    add("bad-version", lambda p: p.set_hdr("version", 2), E_FORMAT, "unsupported version 2")
    add("bad-arch", lambda p: p.set_hdr("arch", 7), E_FORMAT, "unsupported arch 7")
    # header bounds and uint32 wraps
    add("hdr-huge-hidden", lambda p: p.set_hdr("hidden", 0xFFFFFFFF), E_FORMAT,
        "bad model dimensions")
    add("hdr-layers-33", lambda p: p.set_hdr("n_layers", 33), E_FORMAT, "bad model dimensions")
    add("hdr-heads-wrap", lambda p: p.set_hdr("n_heads", (1 << 23) + 8), E_FORMAT,
        "bad attention dimensions")
    add("hdr-gqa", lambda p: p.set_hdr("n_kv_heads", 3), E_FORMAT, "bad attention dimensions")
    add("hdr-rot-odd", lambda p: p.set_hdr("rot_dim", 15), E_FORMAT, "bad attention dimensions")
    add("hdr-lin-wrap", lambda p: p.set_hdr("lin_k_heads", (1 << 25) + 2)
        .set_hdr("lin_v_heads", (1 << 25) + 4), E_FORMAT, "bad linear-attention dimensions")
    add("hdr-conv-k-9", lambda p: p.set_hdr("conv_k", 9), E_FORMAT,
        "bad linear-attention dimensions")
    add("hdr-eos", lambda p: p.set_hdr("eos_id", p.hdr("vocab")), E_FORMAT, "eos_id")
    add("hdr-tied-2", lambda p: p.set_hdr("tied_embeddings", 2), E_FORMAT, "bad tied_embeddings")
    add("hdr-theta-inf", lambda p: p.set_hdr("rope_theta", float("inf")), E_FORMAT,
        "bad eps / rope_theta")
    add("hdr-eps-nan", lambda p: p.set_hdr("rms_eps", float("nan")), E_FORMAT,
        "bad eps / rope_theta")
    add("hdr-eps-zero", lambda p: p.set_hdr("rms_eps", 0.0), E_FORMAT, "bad eps / rope_theta")
    # kernel limits (a header the format accepts that the MI355X kernels do not)
    add("lin-k-dim-96", lambda p: p.set_hdr("lin_k_dim", 96), E_FORMAT,
        "not supported by the MI355X kernels")
    add("vocab-odd", lambda p: p.set_hdr("vocab", p.hdr("vocab") - 1)
        .set_hdr("eos_id", 0), E_FORMAT, "not supported by the MI355X kernels")
    # directory
    add("dir-misaligned", lambda p: p.set_hdr("dir_offset", p.hdr("dir_offset") + 4), E_FORMAT,
        "directory out of bounds or misaligned")
    add("dir-n-tensors", lambda p: p.set_hdr("n_tensors", 0xFFFFFFFF), E_FORMAT,
        "directory out of bounds")
    add("data-offset-past-eof", lambda p: p.set_hdr("data_offset", p.size + 4096), E_FORMAT,
        "data_offset out of bounds")
    add("name-unterminated", lambda p: p.set_name("norm.weight", b"x" * 80), E_FORMAT,
        "name not terminated")
    add("ndim-5", lambda p: p.set("norm.weight", "ndim", 5), E_FORMAT, "bad ndim 5")
    add("offset-misaligned", lambda p: p.set("norm.weight", "offset",
                                             p.get("norm.weight", "offset") + 4), E_FORMAT,
        "norm.weight: data out of bounds or misaligned")
    add("offset-before-data", lambda p: p.set("norm.weight", "offset", 0), E_FORMAT,
        "norm.weight: data out of bounds or misaligned")
    # sizes, shapes and dtypes of F32 tensors
    add("f32-nbytes", lambda p: p.set("norm.weight", "nbytes", p.get("norm.weight", "nbytes") - 4),
        E_FORMAT, "norm.weight: nbytes")
    add("shape-wrap", lambda p: p.set("mtp.norm.weight", "ndim", 4)
        .set_shape("mtp.norm.weight", [256, 1 << 30, 1 << 30, 16]), E_FORMAT,
        "mtp.norm.weight: shape larger than the file")
    add("shape-huge", lambda p: p.set("norm.weight", "ndim", 4)
        .set_shape("norm.weight", [0xFFFFFFFF] * 4), E_FORMAT, "norm.weight: shape larger")
    add("shape-zero", lambda p: p.set_shape("norm.weight", [0]), E_FORMAT,
        "norm.weight: zero dimension")
    add("dtype-unknown", lambda p: p.set("norm.weight", "dtype", 99), E_FORMAT,
        "unknown dtype 99")
    add("vec-wrong-length", lambda p: p.set_shape("norm.weight", [128])
        .set("norm.weight", "nbytes", 512), E_FORMAT, "norm.weight: expected F32 [256]")
    add("tensor-missing", lambda p: p.set_name("norm.weight", b"norm.weigh"), E_FORMAT,
        "missing tensor norm.weight")
    add("both-A-and-A-log", lambda p: p.set_name("layers.0.linear_attn.dt_bias",
                                                 b"layers.0.linear_attn.A"), E_FORMAT,
        "both linear_attn.A and A_log")
    add("conv-shape", lambda p: p.set_shape("layers.0.linear_attn.conv1d.weight",
                                            [p.shape("layers.0.linear_attn.conv1d.weight")[0], 2])
        .set("layers.0.linear_attn.conv1d.weight", "nbytes",
             p.shape("layers.0.linear_attn.conv1d.weight")[0] * 8), E_FORMAT,
        "bad or missing conv1d.weight")
    # Q4K_G32 matrices
    add("q-nbytes", lambda p: p.set(GATE, "nbytes", p.get(GATE, "nbytes") - SB), E_FORMAT,
        f"{GATE}: nbytes")
    def at_eof(p):  # in bounds and ending (almost) at EOF: only the size check stops it
        short = p.get(GATE, "nbytes") - SB
        return p.set(GATE, "nbytes", short).set(GATE, "offset", (p.size - short) // 64 * 64)

    add("q-nbytes-at-eof", at_eof, E_FORMAT, f"{GATE}: nbytes")
    add("q-rows", lambda p: p.set_shape(GATE, [p.shape(GATE)[0] - 1, p.shape(GATE)[1]]), E_FORMAT,
        f"{GATE}: quantized dtype")
    add("q-cols", lambda p: p.set_shape(GATE, [p.shape(GATE)[0], 1000]), E_FORMAT,
        f"{GATE}: quantized dtype")
    add("q-ndim", lambda p: p.set(GATE, "ndim", 1), E_FORMAT, f"{GATE}: quantized dtype")
    add("q-as-f32", lambda p: p.set(GATE, "dtype", 0), E_FORMAT, f"{GATE}: nbytes")
    add("q-wrong-shape", lambda p: p.set_shape(GATE, [p.shape(GATE)[0] - 4, p.shape(GATE)[1]])
        .set(GATE, "nbytes", p.get(GATE, "nbytes") - SB * p.shape(GATE)[1] // 256), E_FORMAT,
        f"{GATE}: expected shape")
    add("q8-dtype", lambda p: p.set(GATE, "dtype", 2), E_FORMAT, f"{GATE}: nbytes")
    add("mtp-fc-nbytes", lambda p: p.set("mtp.fc.weight", "nbytes",
                                         p.get("mtp.fc.weight", "nbytes") - SB), E_FORMAT,
        "mtp.fc.weight: nbytes")
    return c


@pytest.mark.parametrize("patch,code,text,size", cases())
def test_malformed_file_refused(model, lib, tmp_path, patch, code, text, size):
    path = tmp_path / "bad.pq"
    if patch is not None:
        patch(model.copy()).write(path, size(model) if size else None)
    rc, msg = load(lib, path)
    assert rc == code, f"error {rc}, expected {code}; stderr: {msg!r}"
    assert text in msg, f"the refusal does not name its check ({text!r}): {msg!r}"


def test_unpatched_control_passes_every_check(model, lib, tmp_path):
    """The unpatched header + directory over zero weights passes the file checks; without a
    GPU it stops at device creation, with one it loads."""
    rc, msg = load(lib, model.write(tmp_path / "control.pq"))
    assert rc in (0, E_NOMEM), (rc, msg)
    for check in ("bad", "missing", "out of bounds", "nbytes", "expected"):
        assert check not in msg, msg
