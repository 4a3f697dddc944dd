"""Pins of the oracle's scalar primitives (CPU only): the reference's Cephes-style pf_expf
bit for bit against oracle/_ref (the reference's own forward_ops.c), the gate exp / log1p
(binary64 evaluation) against x87 extended precision and against glibc expf / log1pf, and
argmax / acceptance against brute force and the reference's pf_argmax."""
from __future__ import annotations

import ctypes
import ctypes.util

import numpy as np
import pytest

import oracle

L = oracle.lib()
ref = oracle.ref_lib()
libm = ctypes.CDLL(ctypes.util.find_library("m"))
libm.expf.restype, libm.expf.argtypes = ctypes.c_float, [ctypes.c_float]
libm.log1pf.restype, libm.log1pf.argtypes = ctypes.c_float, [ctypes.c_float]


def sweep(lo, hi, n, seed=0):
    rng = np.random.default_rng(seed)
    x = np.concatenate([np.linspace(lo, hi, n // 2), rng.uniform(lo, hi, n // 2)])
    return x.astype(np.float32)


@pytest.mark.skipif(ref is None, reason="oracle/_ref not built (reference absent)")
def test_expf_cephes_bit_exact_vs_reference_build():
    xs = np.concatenate([sweep(-95, 95, 20000), np.float32([0.0, -0.0, 1e-30, -87, 88, 88.5])])
    for x in xs:
        a, b = L.orc_expf_cephes(float(x)), ref.pf_expf(float(x))
        assert np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32), x


def correctly_rounded(fn, x):
    return np.float32(fn(np.longdouble(x)))


def test_gate_functions_equal_host_libm_everywhere():
    """The DeltaNet gates' expf / log1pf (the reference calls libm, forward_lin.c:18-19,59-66)
    restated from this platform's C library equal it on every one of the 2^32 binary32 inputs
    (all threads of this host; a few seconds)."""
    import os

    thr = max(1, min(16, len(os.sched_getaffinity(0))))
    assert L.orc_libm_mismatches(0, thr) == 0, "expf"
    assert L.orc_libm_mismatches(1, thr) == 0, "log1pf"


def test_gate_exp2_table_is_correctly_rounded():
    """expf's table: entry i + (i << 47) is 2^(i/32) rounded to nearest binary64, computed
    exactly here from rationals (bisection of the integer 2^(i/32) 2^e bounds)."""
    from fractions import Fraction

    for i in range(32):
        bits = L.orc_exp2_tab(i) + (i << 47)
        d = np.uint64(bits).view(np.float64)
        m, e = Fraction(float(d)), 52  # d in [1, 2): ulp 2^-52
        ulp = Fraction(1, 1 << e)
        # |d - 2^(i/32)| <= ulp / 2  <=>  (d -+ ulp/2)^32 brackets 2^i
        assert (m - ulp / 2) ** 32 <= 2 ** i <= (m + ulp / 2) ** 32, i


@pytest.mark.parametrize("lo,hi", [(-20, 20), (-103, 88), (-1e-3, 1e-3)])
def test_gate_expf_within_an_ulp_of_exp(lo, hi):
    """A sanity bound that does not come from the C library: within 1 ulp of the correctly
    rounded exp (extended precision), and correctly rounded on almost every input."""
    xs = sweep(lo, hi, 20000, seed=1)
    got = np.array([L.orc_gate_expf(float(x)) for x in xs], np.float32)
    exact = np.array([correctly_rounded(np.exp, x) for x in xs], np.float32)
    ulps = np.abs(got.view(np.int32).astype(np.int64) - exact.view(np.int32).astype(np.int64))
    assert ulps.max() <= 1 and (ulps == 0).mean() > 0.999


@pytest.mark.parametrize("lo,hi", [(0, 5e8), (0, 20), (1e-9, 1e-3), (-0.9, 0.9)])
def test_gate_log1pf_within_an_ulp_of_log1p(lo, hi):
    xs = sweep(lo, hi, 20000, seed=2)
    got = np.array([L.orc_gate_log1pf(float(x)) for x in xs], np.float32)
    exact = np.array([correctly_rounded(np.log1p, x) for x in xs], np.float32)
    ulps = np.abs(got.view(np.int32).astype(np.int64) - exact.view(np.int32).astype(np.int64))
    assert ulps.max() <= 1 and (ulps == 0).mean() > 0.9


def test_argmax_first_maximum():
    v = np.array([1, 3, 2, 3, -1], np.float32)
    assert oracle.argmax(v) == 1
    assert oracle.argmax(np.array([-0.0, 0.0, -1.0], np.float32)) == 0
    assert oracle.argmax(np.array([-2.0, 0.0, -0.0], np.float32)) == 1
    rng = np.random.default_rng(3)
    for _ in range(200):
        v = rng.integers(-5, 5, rng.integers(1, 300)).astype(np.float32)
        assert oracle.argmax(v) == int(np.argmax(v))
        if ref is not None:
            assert ref.pf_argmax(v.ctypes.data, v.size) == int(np.argmax(v))


def test_accept_brute_force():
    rng = np.random.default_rng(4)
    for _ in range(300):
        k = int(rng.integers(0, 6))
        V = int(rng.integers(2, 40))
        logits = rng.integers(-3, 3, (k + 1, V)).astype(np.float32)
        am = [int(np.argmax(r)) for r in logits]
        drafts = np.array([am[t] if rng.random() < 0.7 else (am[t] + 1) % V for t in range(k)],
                          np.int32)
        a = 0
        while a < k and drafts[a] == am[a]:
            a += 1
        got_a, bonus, rows = oracle.accept(logits, drafts)
        assert (got_a, bonus, list(rows)) == (a, am[a], am)


def near_threshold_rows(rng, n, p):
    """Rows whose top-1 probability is about p: one logit 0, the others equal up to small noise,
    so that (n - 1) exp(x) = 1 / p - 1."""
    x = np.log((1.0 / p - 1.0) / (n - 1))
    return (np.concatenate([[0.0], x + rng.normal(0, 1e-3, n - 1)])).astype(np.float32)


@pytest.mark.skipif(ref is None, reason="oracle/_ref not built (reference absent)")
@pytest.mark.parametrize("n", [1, 3, 4, 7, 100, 4099, 32768])
def test_top1_prob_vs_reference_build(n):
    """orc_top1_prob against the reference's own pf_softmax_max / pf_softmax_exp (the top1_prob
    of engine/src/spec.c:93-97 composed from them), on random, peaked and near-0.6 rows."""
    rng = np.random.default_rng(n)
    rows = [rng.normal(0, 3, n).astype(np.float32), rng.normal(0, 0.1, n).astype(np.float32)]
    if n > 1:
        rows.append(near_threshold_rows(rng, n, 0.6))
    for l in rows:
        work = l.copy()
        s = ref.pf_softmax_exp(work.ctypes.data, n, ref.pf_softmax_max(l.ctypes.data, n))
        want = np.float32(1.0) / np.float32(s) if s > 0 else np.float32(0.0)
        got = oracle.top1_prob(l)
        assert got.view(np.uint32) == want.view(np.uint32), (n, got, want)


def test_top1_prob_closed_forms():
    assert oracle.top1_prob(np.float32([0.0, -1000, -1000, -1000])) == np.float32(1.0)
    assert oracle.top1_prob(np.zeros(8, np.float32)) == np.float32(0.125)
