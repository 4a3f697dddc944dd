"""The DeltaNet gates' libm: the correctly rounded expf / log1pf of this engine and its checker
against the host glibc's, on the reference engine itself (CPU, no GPU).

The reference computes beta = sigmoid(b) and the decay exp(A softplus(a + dt_bias)) with libm
(engine/src/forward_lin.c:18-19,59-66); the device cannot call glibc, so the kernels use one
binary64-evaluated, correctly rounded exp / log1p, and the end-to-end checker
(oracle/_ref/libpinfer_refq4k.so) has its gates bound to the same functions. Here that checker
runs beside the same engine sources built on glibc's gates (libpinfer_refq4k_glibc.so, the
reference's own build choice), so the only difference between the two is the gates' last ulp.

What it pins: tokens and speculative statistics identical; the logits of the next token within
1e-5 of the largest logit; every DeltaNet recurrent state within 1e-5 normwise. The attention
KV rows are only reported: a 1-ulp change of a hidden can flip one int8 code of the A8 input of
a projection (a jump of one quantum, 1/127 of the block's largest value), so those rows may
move by far more than the gates' ulp without any change of a token.
"""
from __future__ import annotations

import struct

import numpy as np
import pytest

from oracle import refengine

TOL = 1e-5
needs_both = pytest.mark.skipif(
    not (refengine.REFQ4K.exists() and refengine.REFQ4K_GLIBC.exists()),
    reason="oracle/_ref not built (reference absent when the tree was built)")

HDR = struct.Struct("<8s13IIQ")  # the 72-byte state header of engine/src/state.c


def sections(blob: bytes) -> dict[str, np.ndarray]:
    """Float arrays of a state blob (f32 KV), in the blob's order (engine/src/state.c): conv
    and recurrent state of every linear layer, then K and V rows of every full-attention
    layer, then the MTP head's K and V rows."""
    (magic, version, n_past, kv_dtype, mtp_rows, n_layers, hidden, n_kv, hd, lkh, lvh, lkd, lvd,
     conv_k, full_mask, _fp) = HDR.unpack_from(blob)
    assert magic.rstrip(b"\0") == b"PINFERS" and kv_dtype == 0
    conv_dim = 2 * lkh * lkd + lvh * lvd
    f = np.frombuffer(blob, np.float32, offset=HDR.size)
    out, o = {}, 0

    def take(name, size):
        nonlocal o
        out[name] = f[o:o + size].astype(np.float64)
        o += size

    for layer in range(n_layers):
        if not (full_mask >> layer) & 1:
            take(f"conv{layer}", (conv_k - 1) * conv_dim)
            take(f"rec{layer}", lvh * lkd * lvd)
    for layer in range(n_layers):
        if (full_mask >> layer) & 1:
            take(f"K{layer}", n_kv * n_past * hd)
            take(f"V{layer}", n_kv * n_past * hd)
    if mtp_rows:
        take("mtpK", n_kv * mtp_rows * hd)
        take("mtpV", n_kv * mtp_rows * hd)
    assert o == f.size, (o, f.size)
    return out


def compare(path, prompt, n_gen, k, draft_vocab):
    a = refengine.bench_generate(path, prompt, n_gen, k, draft_vocab, 8, max_ctx=512,
                                 want_state=True, lib=refengine.REFQ4K, next_logits=True)
    b = refengine.bench_generate(path, prompt, n_gen, k, draft_vocab, 8, max_ctx=512,
                                 want_state=True, lib=refengine.REFQ4K_GLIBC, next_logits=True)
    assert a.tokens == b.tokens
    assert (a.rounds, a.drafted, a.accepted) == (b.rounds, b.drafted, b.accepted)
    la, lb = a.next_logits.astype(np.float64), b.next_logits.astype(np.float64)
    dev = {"logits": np.abs(la - lb).max() / np.abs(lb).max()}
    sa, sb = sections(a.state), sections(b.state)
    for name in sb:
        nb = np.linalg.norm(sb[name])
        dev[name] = np.linalg.norm(sa[name] - sb[name]) / nb if nb else 0.0
    print({k: float(f"{v:.3g}") for k, v in dev.items()})
    assert dev["logits"] <= TOL
    for name, v in dev.items():
        if name.startswith("rec"):
            assert v <= TOL, f"{name}: {v}"
    return dev


@pytest.fixture(scope="module")
def small_models(tmp_path_factory):
    from nibblemac_amd import pqfile

    d = tmp_path_factory.mktemp("gate")
    w = pqfile.agreeing_norm(pqfile.SMALL.hidden)
    return {
        "small": pqfile.write_model(d / "small.pq", pqfile.SMALL, seed=3, random_norms=True),
        "agree": pqfile.write_model(d / "agree.pq", pqfile.SMALL, seed=3, random_norms=True,
                                    overrides={"norm.weight": w, "mtp.norm.weight": w}),
    }


@needs_both
@pytest.mark.parametrize("which,k", [("small", 0), ("small", 4), ("agree", 4)])
def test_gates_glibc_vs_correctly_rounded(small_models, which, k):
    prompt = np.random.default_rng(2).integers(0, 2047, 24).astype(np.int32)
    compare(small_models[which], prompt, 64, k, 1024)


def test_blob_sections_cover_the_blob():
    """The parser above against a synthetic header (a full-attention layer between linear
    ones): the sections come in the blob's order and their sizes add up to the blob."""
    n_past, mtp_rows = 7, 5
    hdr = HDR.pack(b"PINFERS", 2, n_past, 0, mtp_rows, 4, 256, 2, 64, 2, 4, 64, 64, 4, 0b0010, 1)
    conv_dim = 2 * 2 * 64 + 4 * 64
    rec0 = 3 * conv_dim
    floats = 3 * (3 * conv_dim + 4 * 64 * 64) + 2 * 2 * n_past * 64 + 2 * 2 * mtp_rows * 64
    s = sections(hdr + np.arange(floats, dtype=np.float32).tobytes())
    assert list(s) == ["conv0", "rec0", "conv2", "rec2", "conv3", "rec3", "K1", "V1", "mtpK",
                       "mtpV"]
    assert s["rec0"][0] == rec0 and s["mtpV"][-1] == floats - 1
