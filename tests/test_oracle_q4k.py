"""Pins of the oracle's Q4K_G32 format, A8 quantization and Q4K x A8 matmul (CPU only).

Each check comes from something other than the oracle's own formula: the byte layout decoded
independently from engine/FORMAT.md (tests/refmath.py), the reference's analytical identity-
input test (engine/metal/check.c:147-201), int64 brute force of every sub-block dot, exact
single-rounding FMA chains evaluated with rationals, a float64 dequantised reference within
1e-5 (engine/bench/kbench_util.c:223-227), and planted mistakes that these checks must catch.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from nibblemac_amd import pqtool
from tests.refmath import fma32, pack_superblock, put6, unpack_q4k


def test_get6_all_values_both_halves():
    rng = np.random.default_rng(0)
    for trial in range(50):
        vals = rng.integers(0, 64, 32) if trial else np.arange(32) * 2 + 1
        p = np.frombuffer(put6(vals), np.uint8).copy()
        got = [oracle.lib().orc_get6(p.ctypes.data, j) for j in range(32)]
        assert got == [int(v) for v in vals]


def analytical_matrix(rows=8, cols=512):
    """engine/metal/check.c:147-201 restated: D = (r+1)/16, M = (r+1)/8 per row, sub-scales
    b*32 + i and sub-minima 63 - (b*32 + i) over two superblocks (all 64 values), codes
    (col + r%4 + k + tile) % 16 so both nibble halves of every byte vary."""
    out = bytearray()
    for tile in range(rows // 4):
        for b in range(cols // 256):
            D = [(tile * 4 + r + 1) / 16.0 for r in range(4)]
            M = [(tile * 4 + r + 1) / 8.0 for r in range(4)]
            s = [[b * 32 + 4 * k + i for i in range(4)] for k in range(8)]
            m = [[63 - (b * 32 + 4 * k + i) for i in range(4)] for k in range(8)]
            codes = [[((c % 32) + r + (c // 32) + tile) % 16 for c in range(256)] for r in range(4)]
            out += pack_superblock(D, M, s, m, codes)
    return np.frombuffer(bytes(out), np.uint8).copy()


def test_get_row_analytical_layout():
    rows, cols = 8, 512
    W = analytical_matrix(rows, cols)
    for r in range(rows):
        got = oracle.q4k_get_row(W, rows, cols, r)
        for c in range(cols):
            k = (c % 256) // 32
            sub = (c // 256) * 32 + k * 4 + r % 4
            code = (c % 32 + r % 4 + k + r // 4) % 16
            exp = np.float32((r + 1) / 16.0 * sub * code - (r + 1) / 8.0 * (63 - sub))
            assert got[c] == exp, (r, c)


def test_matmul_analytical_identity_inputs():
    """One-hot activations recover every weight through the A8 path; the expected value is the
    reference's two-FMA chain evaluated exactly: fma(-(M m), fsum, fma(127 u, (D s) d, 0))."""
    rows, cols = 8, 512
    W = analytical_matrix(rows, cols)
    cs = list(range(0, cols, 7)) + [cols - 1]
    X = np.zeros((len(cs), cols), np.float32)
    for v, c in enumerate(cs):
        X[v, c] = 1.0
    q, d, fs = oracle.quant_a8(X)
    Y = oracle.q4k_matmul(W, rows, cols, q, d, fs, len(cs))
    for v, c in enumerate(cs):
        b = c // 32
        dv, fv = d[b, v], fs[b, v]
        assert q[b, v, c % 32] == 127 and dv == np.float32(1.0) / np.float32(127.0)
        for r in range(rows):
            k = (c % 256) // 32
            sub = (c // 256) * 32 + k * 4 + r % 4
            code = (c % 32 + r % 4 + k + r // 4) % 16
            sc = np.float32((r + 1) / 16.0) * np.float32(sub)
            of = np.float32((r + 1) / 8.0) * np.float32(63 - sub)
            acc = np.float32(0.0)
            for bb in range(cols // 32):  # blocks before / after c hold zero activations
                if bb == b:
                    acc = fma32(np.float32(127 * code), sc * dv, acc)
                    acc = fma32(-of, fv, acc)
            assert Y[v, r] == acc, (v, r)


def test_quant_a8_closed_forms():
    x = np.zeros((3, 64), np.float32)
    x[0, :32] = np.arange(-16, 16, dtype=np.float32) * 4          # amax 64
    x[0, 0] = -127.0                                              # amax 127 -> id 1
    x[0, 1:5] = [2.5, 3.5, -2.5, -0.5]                            # ties to even
    x[1, 32:] = 1e-30                                             # tiny but nonzero
    q, d, fs = oracle.quant_a8(x)
    assert q[0, 0, 0] == -127 and list(q[0, 0, 1:5]) == [2, 4, -2, 0]
    assert d[0, 0] == np.float32(1.0) and fs[0, 0] == np.float32(q[0, 0].astype(np.int64).sum())
    assert not q[:, 2].any() and d[0, 2] == 0 and fs[0, 2] == 0  # zero blocks of vector 2
    assert (q[1, 1] == 127).all() and d[1, 1] == np.float32(1e-30) / np.float32(127.0)


def test_quant_a8_matches_numpy_restatement():
    rng = np.random.default_rng(1)
    X = (rng.standard_normal((7, 1024)) * rng.uniform(0.1, 10, (7, 1))).astype(np.float32)
    q, d, fs = oracle.quant_a8(X)
    xb = X.reshape(7, 32, 32)
    amax = np.abs(xb).max(-1)
    inv = np.where(amax > 0, np.float32(127.0) / np.where(amax > 0, amax, 1), 0).astype(np.float32)
    codes = np.rint(xb * inv[..., None]).astype(np.int32)
    dd = (amax / np.float32(127.0)).astype(np.float32)
    fsum = (dd * codes.sum(-1).astype(np.float32)).astype(np.float32)
    assert np.array_equal(q.transpose(1, 0, 2), codes.astype(np.int8))
    assert np.array_equal(d.T, dd) and np.array_equal(fs.T, fsum)


def brute_dots(W, rows, cols, q, n):
    u = unpack_q4k(W, rows, cols)[0]                          # [rows][cols] int64
    x = q.transpose(1, 0, 2).reshape(n, cols).astype(np.int64)  # [n][cols]
    return (u.reshape(rows, cols // 32, 32)[None] * x.reshape(n, 1, cols // 32, 32)).sum(-1)


@pytest.mark.parametrize("rows,cols,n", [(4, 256, 1), (16, 512, 3), (64, 1024, 5), (20, 768, 8)])
def test_matmul_dots_brute_force_and_fp64(rows, cols, n):
    rng = np.random.default_rng(rows + cols + n)
    W = pqtool.gauss_q4k(3, rows, rows, cols)
    X = rng.standard_normal((n, cols)).astype(np.float32)
    q, d, fs = oracle.quant_a8(X)
    Y, dots = oracle.q4k_matmul(W, rows, cols, q, d, fs, n, want_dots=True)
    assert np.array_equal(dots, brute_dots(W, rows, cols, q, n))
    # float64 reference with the dequantised weights and int8-dequantised activations
    deq = np.stack([oracle.q4k_get_row(W, rows, cols, r) for r in range(rows)]).astype(np.float64)
    xq = (q.astype(np.float64) * d[..., None]).transpose(1, 0, 2).reshape(n, cols)
    ref = xq @ deq.T
    err = np.abs(Y - ref).max() / max(np.abs(ref).max(), 1e-30)
    assert err < 1e-5, err
    # batch == single
    for v in range(n):
        qv, dv, fv = oracle.quant_a8(X[v:v + 1])
        assert np.array_equal(oracle.q4k_matmul(W, rows, cols, qv, dv, fv, 1)[0].view(np.uint32),
                              Y[v].view(np.uint32))


def test_matmul_exact_fma_chain_small():
    """Every output of a 4x256 x 3 case equals the chain evaluated with exact single-rounding
    FMAs in block order (a separately rounded multiply-add, a reordered chain or a dropped min
    term would differ on these inputs)."""
    rows, cols, n = 4, 256, 3
    rng = np.random.default_rng(5)
    W = pqtool.gauss_q4k(4, 0, rows, cols)
    X = rng.standard_normal((n, cols)).astype(np.float32)
    q, d, fs = oracle.quant_a8(X)
    Y, dots = oracle.q4k_matmul(W, rows, cols, q, d, fs, n, want_dots=True)
    u, s, m, D, M = unpack_q4k(W, rows, cols)
    for v in range(n):
        for r in range(rows):
            acc = np.float32(0.0)
            for b in range(cols // 32):
                sc = np.float32(D[r, b // 8] * np.float32(s[r, b]))
                of = np.float32(M[r, b // 8] * np.float32(m[r, b]))
                acc = fma32(np.float32(dots[v, r, b]), np.float32(sc * d[b, v]), acc)
                acc = fma32(-of, fs[b, v], acc)
            assert Y[v, r] == acc, (v, r)


def test_planted_mistakes_are_caught():
    """The fp64 tolerance and brute-force pins reject plausible mistakes (applied to the inputs
    the oracle sees, never to the product): swapped nibble halves, a dropped min term."""
    rows, cols, n = 64, 1024, 2
    rng = np.random.default_rng(6)
    W = pqtool.gauss_q4k(5, 1, rows, cols)
    X = rng.standard_normal((n, cols)).astype(np.float32)
    q, d, fs = oracle.quant_a8(X)
    deq = np.stack([oracle.q4k_get_row(W, rows, cols, r) for r in range(rows)]).astype(np.float64)
    xq = (q.astype(np.float64) * d[..., None]).transpose(1, 0, 2).reshape(n, cols)
    ref = xq @ deq.T
    rel = lambda Y: np.abs(Y - ref).max() / np.abs(ref).max()
    Wswap = W.reshape(-1, 576).copy()
    body = Wswap[:, 64:]
    Wswap[:, 64:] = ((body & 15) << 4) | (body >> 4)
    assert rel(oracle.q4k_matmul(Wswap.reshape(-1), rows, cols, q, d, fs, n)) > 1e-3
    assert rel(oracle.q4k_matmul(W, rows, cols, q, d, np.zeros_like(fs), n)) > 1e-3
    Y, dots = oracle.q4k_matmul(Wswap.reshape(-1), rows, cols, q, d, fs, n, want_dots=True)
    assert not np.array_equal(dots, brute_dots(W, rows, cols, q, n))


def test_quantizer_matches_numpy_restatement_and_bounds():
    """The oracle's quantizer and the product's (libpinfer pqt_quantize_q4k) give the same
    bytes; a numpy restatement of engine/bench/kbench_util.c:100-132 gives them too; every
    weight dequantizes within half a quantum of its group."""
    rng = np.random.default_rng(7)
    w = (rng.standard_normal((8, 512)) * 0.02).astype(np.float32)
    a, b = oracle.q4k_quantize(w), pqtool.quantize_q4k(w)
    assert np.array_equal(a, b)
    g = w.reshape(8, 2, 8, 32)
    lo = np.minimum(g.min(-1), 0).astype(np.float32)
    hi = g.max(-1)
    scale = ((hi - lo) / np.float32(15)).astype(np.float32)
    off = (-lo).astype(np.float32)
    D = (scale.max(-1) / np.float32(63)).astype(np.float16).astype(np.float32)
    Mx = (off.max(-1) / np.float32(63)).astype(np.float16).astype(np.float32)
    s6 = np.minimum(np.ceil(scale / D[..., None]), 63).astype(np.int32)
    m6 = np.rint(np.minimum(off / Mx[..., None], 63)).astype(np.int32)
    u, s, m, DD, MM = unpack_q4k(a, 8, 512)
    assert np.array_equal(s, s6.reshape(8, 16)) and np.array_equal(m, m6.reshape(8, 16))
    assert np.array_equal(DD, D) and np.array_equal(MM, Mx)
    deq = np.stack([oracle.q4k_get_row(a, 8, 512, r) for r in range(8)])
    step = (D[..., None] * s6).reshape(8, 16)
    assert (np.abs(deq - w).reshape(8, 16, 32) <= step[..., None] * 0.5 + 1e-4).all()
