"""GPU parity of the reference-engine operator plug (nibblemac_amd/csrc/plug/matvec_nmx.c).

1. The contract functions (engine/src/ops.h:47-93) called directly through
   oracle/_ref/libpinfer_nmxplug.so against the oracle: pf_matmul at 3 and at 100 vectors (more
   than one device call), pf_lin_rule plain at 100 tokens after 70 deferred updates, logged at 5
   tokens after 3 (row 0 of the log left untouched), pf_lin_apply over 70 rows.
2. The reference's own C engine (forward pass, DeltaNet mixer and rollback log, MTP head,
   speculative loop; engine/src/*.c) on the plug against the same engine objects on the
   oracle's operators (oracle/_ref/libpinfer_refq4k.so): the two libraries differ only in the
   operator plug.

Bar: bit-exact outputs, state and log; identical tokens and speculative statistics.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest

import oracle
from nibblemac_amd import pqfile
from oracle import HERE as ORACLE_DIR
from tests.refmath import state_from_dev, state_to_dev

pytestmark = pytest.mark.gpu

PLUG = ORACLE_DIR / "_ref" / "libpinfer_nmxplug.so"
REF = ORACLE_DIR / "_ref" / "libpinfer_refq4k.so"
needs_plug = pytest.mark.skipif(not (PLUG.exists() and REF.exists()),
                                reason="oracle/_ref not built (reference absent when the tree "
                                "was built)")
PQ_Q4K_G32 = 4
_vp = ctypes.c_void_p


class PfMat(ctypes.Structure):
    """Mirror of pf_mat (engine/src/ops.h:16-20)."""

    _fields_ = [("dtype", ctypes.c_uint32), ("rows", ctypes.c_int), ("cols", ctypes.c_int),
                ("data", _vp)]


def bits_equal(a, b, what):
    a = np.ascontiguousarray(a, np.float32).view(np.uint32).ravel()
    b = np.ascontiguousarray(b, np.float32).view(np.uint32).ravel()
    bad = np.flatnonzero(a != b)
    assert bad.size == 0, f"{what}: {bad.size} mismatches, first at {bad[0]}"


@pytest.fixture
def plug():
    """A fresh pool per test: a pool keys its device weights by host address, valid while the
    matrices outlive it (as in the engine, engine/src/pinfer.c:185-186), and a test's arrays do
    not outlive the test."""
    L = ctypes.CDLL(str(PLUG))
    L.pf_pool_create.restype, L.pf_pool_create.argtypes = _vp, [ctypes.c_int]
    L.pf_pool_destroy.restype, L.pf_pool_destroy.argtypes = None, [_vp]
    L.pf_matmul.restype = None
    L.pf_matmul.argtypes = [_vp, ctypes.POINTER(PfMat), _vp, _vp, ctypes.c_int]
    L.pf_lin_rule.restype = None
    L.pf_lin_rule.argtypes = [_vp, ctypes.POINTER(oracle.RefLinArgs)]
    L.pf_lin_apply.restype = None
    L.pf_lin_apply.argtypes = [_vp, _vp, _vp] + [ctypes.c_int] * 4
    pool = L.pf_pool_create(1)
    assert pool, "pf_pool_create failed (no device?)"
    yield L, pool
    L.pf_pool_destroy(pool)


def dev_layout(S, heads, dk, dv):
    """[h][dk][dv] (oracle) -> the plug's private layout (the device kernels', nmx_state_index)."""
    return state_to_dev(S, heads, dk, dv)


def from_dev(S, heads, dk, dv):
    return state_from_dev(S, heads, dk, dv)


def lin_inputs(rng, n, heads, rep, dk, dv):
    kd = heads // rep * dk
    stride = 2 * kd + heads * dv
    qkv = np.zeros((n, stride), np.float32)
    qk = rng.standard_normal((n, 2, heads // rep, dk)).astype(np.float32)
    qk /= np.linalg.norm(qk, axis=-1, keepdims=True).astype(np.float32)
    qkv[:, :kd], qkv[:, kd:2 * kd] = qk[:, 0].reshape(n, kd), qk[:, 1].reshape(n, kd)
    qkv[:, 2 * kd:] = rng.standard_normal((n, heads * dv))
    sig = lambda x: (1.0 / (1.0 + np.exp(-x))).astype(np.float32)
    decay = (0.9 + 0.1 * sig(rng.standard_normal((n, heads)))).astype(np.float32)
    beta = sig(rng.standard_normal((n, heads)))
    return qkv, decay, beta, stride


def log_rows(rng, m, heads, dk, dv):
    """m rollback-log rows k | delta | decay per head (normalised k, small delta)."""
    lg = np.zeros((m, heads, dk + dv + 1), np.float32)
    k = rng.standard_normal((m, heads, dk)).astype(np.float32)
    lg[..., :dk] = k / np.linalg.norm(k, axis=-1, keepdims=True)
    lg[..., dk:dk + dv] = 0.1 * rng.standard_normal((m, heads, dv))
    lg[..., -1] = 0.9 + 0.1 * rng.random((m, heads))
    return lg


@needs_plug
@pytest.mark.parametrize("n", [3, 100])
def test_pf_matmul(plug, n):
    L, pool = plug
    rng = np.random.default_rng(30 + n)
    rows, cols = 256, 1024
    W = oracle.q4k_quantize(rng.standard_normal((rows, cols)).astype(np.float32) * 0.03)
    X = rng.standard_normal((n, cols)).astype(np.float32)
    Y = np.empty((n, rows), np.float32)
    m = PfMat(PQ_Q4K_G32, rows, cols, W.ctypes.data)
    L.pf_matmul(pool, ctypes.byref(m), X.ctypes.data, Y.ctypes.data, n)
    bits_equal(Y, oracle.q4k_matmul(W, rows, cols, *oracle.quant_a8(X), n), f"pf_matmul n={n}")


@needs_plug
@pytest.mark.parametrize("logged", [False, True])
def test_pf_lin_rule(plug, logged):
    L, pool = plug
    heads, rep, dk, dv = 4, 2, 128, 128
    n, keep = (5, 3) if logged else (100, 70)
    rng = np.random.default_rng(40 + logged)
    qkv, decay, beta, stride = lin_inputs(rng, n, heads, rep, dk, dv)
    S0 = (0.05 * rng.standard_normal((heads, dk, dv))).astype(np.float32)
    pend = log_rows(rng, keep, heads, dk, dv)
    S_ref, o_ref, lg_ref = oracle.lin_rule(qkv, decay, beta, S0, n=n, heads=heads, rep=rep, dk=dk,
                                           dv=dv, log=logged, pend=pend, keep=keep)
    S = dev_layout(S0, heads, dk, dv)
    o = np.zeros((n, heads * dv), np.float32)
    lg = np.full((n, heads, dk + dv + 1), 7.0, np.float32) if logged else None
    a = oracle.RefLinArgs(n, heads, rep, dk, dv, stride, heads * dv, qkv.ctypes.data,
                          decay.ctypes.data, beta.ctypes.data, S.ctypes.data, o.ctypes.data,
                          None if lg is None else lg.ctypes.data, pend.ctypes.data, keep, None)
    L.pf_lin_rule(pool, ctypes.byref(a))
    bits_equal(o, o_ref, "o")
    bits_equal(from_dev(S, heads, dk, dv), S_ref, "S")
    if logged:
        assert np.all(lg[0] == 7.0), "log row 0 written"
        bits_equal(lg[1:], lg_ref[1:], "log rows 1..n-1")


@needs_plug
def test_pf_lin_apply(plug):
    L, pool = plug
    heads, dk, dv, keep = 4, 64, 128, 70
    rng = np.random.default_rng(50)
    S0 = (0.05 * rng.standard_normal((heads, dk, dv))).astype(np.float32)
    lg = log_rows(rng, keep, heads, dk, dv)
    S = dev_layout(S0, heads, dk, dv)
    L.pf_lin_apply(pool, S.ctypes.data, lg.ctypes.data, keep, heads, dk, dv)
    bits_equal(from_dev(S, heads, dk, dv), oracle.lin_apply(S0, lg, keep, heads, dk, dv), "S")


@pytest.fixture(scope="module")
def small_pq(tmp_path_factory):
    return pqfile.write_model(tmp_path_factory.mktemp("pq") / "small.pq", pqfile.SMALL, seed=3,
                              random_norms=True)


def engines(path):
    from nibblemac_amd.pinfer import Model, load_library

    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    return (Model(str(path), max_ctx=512, lib=load_library(str(PLUG))),
            Model(str(path), max_ctx=512, lib=load_library(str(REF)), n_threads=threads))


@needs_plug
def test_engine_eval_on_plug(small_pq):
    dev, ref = engines(small_pq)
    rng = np.random.default_rng(60)
    prompt = rng.integers(0, pqfile.SMALL.vocab, 40)
    bits_equal(dev.eval(prompt), ref.eval(prompt), "logits after prefill")
    more = rng.integers(0, pqfile.SMALL.vocab, 7)
    bits_equal(dev.eval(more), ref.eval(more), "logits after continuation")
    dev.close(), ref.close()


@needs_plug
@pytest.mark.parametrize("k", [2, 4])
def test_engine_generate_on_plug(agree_model, k):
    """Speculative generation through the reference's own loop with drafts accepted in many
    rounds: multi-token commits and deferred replays through pf_lin_rule's pend / keep."""
    path, prompt = agree_model
    print(f"[case] plug generate agree k={k}", flush=True)
    dev, ref = engines(path)
    ta, sa = dev.generate(prompt, 64, k=k)
    tb, sb = ref.generate(prompt, 64, k=k)
    assert ta == tb
    assert (sa.rounds, sa.drafted, sa.accepted) == (sb.rounds, sb.drafted, sb.accepted)
    assert sa.accepted >= sa.drafted // 4
    probe = [1, 2, 3]
    bits_equal(dev.eval(probe), ref.eval(probe), "logits after the generation")
    dev.close(), ref.close()
