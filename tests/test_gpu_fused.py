"""GPU parity of the fused entry points against the separate kernels they replace.

nmx_q4k_matmul_norm = nmx_rmsnorm_xo (residual add + RMSNorm + A8) followed by the Q4K matmul;
nmx_q4k_swiglu = [RMSNorm + A8 +] gate / up matmuls + nmx_silu_mul (+ A8). Bar: bit-exact
(outputs, the residual sum, and the A8 codes / scales of the SwiGLU output). Shapes cover the
fused kernel (every 0.8B projection at 1..8 rows), several vector passes (13, 64 rows) and the
fallback to the separate kernels (widths whose workgroup tile does not fit in LDS). The
separate kernels are themselves checked against the oracle (test_gpu_q4k.py) and, through the
reference engine, against the reference's RMSNorm and SwiGLU (test_gpu_e2e.py); the RMSNorm is
also checked here against a float32 restatement of its summation order.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from tests.test_gpu_q4k import assert_bits_equal, gaussian_q4k

pytestmark = pytest.mark.gpu

EPS = 1e-6


def rmsnorm_restated(x, w, eps):
    """engine/src/forward_ops.c:168-200 in float32: 4 interleaved partial sums of squares over
    the first cols/4*4 columns, (c0 + c1) + (c2 + c3) + tail, r = 1 / sqrtf(ss / cols + eps),
    y = (x * r) * w."""
    x = x.astype(np.float32)
    n, cols = x.shape
    sq = x * x
    c = np.zeros((n, 4), np.float32)
    m4 = cols // 4
    for m in range(m4):
        c = c + sq[:, 4 * m:4 * m + 4]
    t = np.zeros(n, np.float32)
    for i in range(4 * m4, cols):
        t = t + sq[:, i]
    s = ((c[:, 0] + c[:, 1]) + (c[:, 2] + c[:, 3])) + t
    r = np.float32(1.0) / np.sqrt(s / np.float32(cols) + np.float32(eps))
    return (x * r[:, None]) * w[None, :]


def a8_bufs(dev, n, cols):
    return (dev.zeros((cols // 32, n, 32), np.int8), dev.zeros((cols // 32, n), np.float32),
            dev.zeros((cols // 32, n), np.float32))


@pytest.mark.parametrize("cols,shapes", [(1024, [6144, 2048, 16, 16]), (1024, [4096, 512, 512]),
                                         (2048, [1024]), (3584, [1024]), (8192, [64])])
@pytest.mark.parametrize("n", [1, 5, 8, 13, 64])
def test_matmul_norm_equals_separate(dev, cols, shapes, n):
    print(f"[case] matmul_norm cols={cols} rows={shapes} n={n}", flush=True)
    rng = np.random.default_rng(cols + n)
    Ws = [gaussian_q4k(rng, r, cols) for r in shapes]
    x = rng.standard_normal((n, cols)).astype(np.float32)
    add = rng.standard_normal((n, cols)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    dWs = [dev.to_device(t) for t in Ws]
    dx, dadd, dw = dev.to_device(x), dev.to_device(add), dev.to_device(w)
    # separate kernels
    xo_ref = dev.zeros((n, cols), np.float32)
    a8 = a8_bufs(dev, n, cols)
    dev.rmsnorm(dx, n, cols, dw, EPS, add=dadd, xo=xo_ref, a8=a8)
    Yref = [dev.zeros((n, r), np.float32) for r in shapes]
    dev.q4k_matmul_multi(dWs, shapes, Yref, shapes, cols, n, *a8)
    # fused
    xo = dev.zeros((n, cols), np.float32)
    tmp = a8_bufs(dev, n, cols)
    Y = [dev.zeros((n, r), np.float32) for r in shapes]
    dev.q4k_matmul_norm(dWs, shapes, Y, cols, n, dx, dw, EPS, add=dadd, xo=xo, a8_tmp=tmp)
    dev.sync()
    assert_bits_equal(xo.numpy(), x + add, "residual sum")
    assert_bits_equal(xo.numpy(), xo_ref.numpy(), "residual sum (separate)")
    for r, a, b in zip(shapes, Y, Yref):
        assert_bits_equal(a.numpy(), b.numpy(), f"rows={r}")
    # the separate RMSNorm against the restated order (its A8 through the oracle)
    q, d, fs = oracle.quant_a8(rmsnorm_restated(x + add, w, EPS))
    assert_bits_equal(a8[0].numpy(), q, "A8 codes of the norm")
    assert_bits_equal(a8[1].numpy(), d, "A8 scales of the norm")
    assert_bits_equal(a8[2].numpy(), fs, "A8 fsum of the norm")


@pytest.mark.parametrize("cols", [64, 1024, 2048, 3584, 4096, 4100, 8192])
@pytest.mark.parametrize("n", [1, 5])
def test_rmsnorm_outputs(dev, cols, n):
    """The RMSNorm alone (float4 rows up to 4096 columns, the per-column kernel otherwise or
    for widths that are not a multiple of 32): residual sum, y and A8 against the restated
    summation order and the oracle's A8."""
    print(f"[case] rmsnorm cols={cols} n={n}", flush=True)
    rng = np.random.default_rng(7 * cols + n)
    x = rng.standard_normal((n, cols)).astype(np.float32)
    add = rng.standard_normal((n, cols)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    dx, dadd, dw = dev.to_device(x), dev.to_device(add), dev.to_device(w)
    xo, y = dev.zeros((n, cols), np.float32), dev.zeros((n, cols), np.float32)
    a8 = a8_bufs(dev, n, cols) if cols % 32 == 0 else (None, None, None)
    dev.rmsnorm(dx, n, cols, dw, EPS, add=dadd, xo=xo, y=y, a8=a8)
    dev.sync()
    want = rmsnorm_restated(x + add, w, EPS)
    assert_bits_equal(xo.numpy(), x + add, "residual sum")
    assert_bits_equal(y.numpy(), want, "y")
    if cols % 32 == 0:
        for got, ref, what in zip(a8, oracle.quant_a8(want), ("codes", "scales", "fsum")):
            assert_bits_equal(got.numpy(), ref, f"A8 {what}")


@pytest.mark.parametrize("n", [1, 2, 5, 6, 8, 13])
@pytest.mark.parametrize("fused_norm", [True, False])
def test_swiglu_equals_separate(dev, n, fused_norm):
    print(f"[case] swiglu n={n} norm={fused_norm}", flush=True)
    ffn, cols = 3584, 1024
    rng = np.random.default_rng(100 + n)
    Wg, Wu = gaussian_q4k(rng, ffn, cols), gaussian_q4k(rng, ffn, cols)
    dWg, dWu = dev.to_device(Wg), dev.to_device(Wu)
    x = rng.standard_normal((n, cols)).astype(np.float32)
    add = rng.standard_normal((n, cols)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    dx, dadd, dw = dev.to_device(x), dev.to_device(add), dev.to_device(w)
    a8_in = a8_bufs(dev, n, cols)
    dev.rmsnorm(dx, n, cols, dw, EPS, add=dadd, a8=a8_in)
    # separate: matmuls + silu_mul
    g, u = dev.zeros((n, ffn), np.float32), dev.zeros((n, ffn), np.float32)
    dev.q4k_matmul_multi([dWg, dWu], [ffn, ffn], [g, u], [ffn, ffn], cols, n, *a8_in)
    yref = dev.zeros((n, ffn), np.float32)
    outref = a8_bufs(dev, n, ffn)
    dev.silu_mul(g, u, n, ffn, y=yref, a8=outref)
    # fused
    y = dev.zeros((n, ffn), np.float32)
    out = a8_bufs(dev, n, ffn)
    tmp = a8_bufs(dev, n, cols)
    gt, ut = dev.zeros((n, ffn), np.float32), dev.zeros((n, ffn), np.float32)
    xo = dev.zeros((n, cols), np.float32)
    if fused_norm:
        dev.q4k_swiglu(dWg, dWu, ffn, cols, n, out, norm=(dx, dw, EPS, dadd, xo), y=y,
                       a8_tmp=tmp, gate_tmp=gt, up_tmp=ut)
    else:
        dev.q4k_swiglu(dWg, dWu, ffn, cols, n, out, a8=a8_in, y=y, gate_tmp=gt, up_tmp=ut)
    dev.sync()
    assert_bits_equal(y.numpy(), yref.numpy(), "silu(gate) * up")
    for a, b, what in zip(out, outref, ("codes", "scales", "fsum")):
        assert_bits_equal(a.numpy(), b.numpy(), f"A8 {what}")
    if fused_norm:
        assert_bits_equal(xo.numpy(), x + add, "residual sum")


def test_fused_invalid_calls_rejected(dev):
    from nibblemac_amd.nmx import NmxError
    W = dev.zeros(576 * 4, np.uint8)
    x = dev.zeros((2, 256), np.float32)
    w = dev.zeros(256, np.float32)
    Y = dev.zeros((2, 16), np.float32)
    with pytest.raises(NmxError):   # x_out aliases x
        dev.q4k_matmul_norm([W], [16], [Y], 256, 2, x, w, EPS, add=x, xo=x)
    with pytest.raises(NmxError):   # output aliases the norm input
        dev.q4k_matmul_norm([W], [16], [x], 256, 2, x, w, EPS)
    with pytest.raises(NmxError):   # cols not a multiple of 256
        dev.q4k_matmul_norm([W], [16], [Y], 255, 2, x, w, EPS)
    out = a8_bufs(dev, 2, 32)
    with pytest.raises(NmxError):   # no input
        dev.q4k_swiglu(W, W, 32, 256, 2, out)


@pytest.mark.parametrize("cols", [1024, 2048])
@pytest.mark.parametrize("n", [1, 5])
def test_embed_norm(dev, cols, n):
    """nmx_embed_norm (the embedding decoded inside the first norm, with a second independent
    norm in the same launch at cols <= 1024; embedding + two norms at 2048): the rows equal the
    oracle's Q4K row dequantisation, both norms and their A8 the restated order and the oracle."""
    print(f"[case] embed_norm cols={cols} n={n}", flush=True)
    rng = np.random.default_rng(31 * cols + n)
    vocab = 256
    E = oracle.q4k_quantize((rng.standard_normal((vocab, cols)) * 0.02).astype(np.float32))
    tok = rng.integers(0, vocab, n).astype(np.int32)
    emb = np.stack([oracle.q4k_get_row(E, vocab, cols, int(t)) for t in tok])
    x1 = rng.standard_normal((n, cols)).astype(np.float32)
    w0, w1 = (rng.uniform(0.5, 1.5, cols).astype(np.float32) for _ in range(2))
    dE, dtok, dx1 = dev.to_device(E), dev.to_device(tok), dev.to_device(x1)
    dw0, dw1 = dev.to_device(w0), dev.to_device(w1)
    xo0, y0, y1 = (dev.zeros((n, cols), np.float32) for _ in range(3))
    a0, a1 = a8_bufs(dev, n, cols), a8_bufs(dev, n, cols)
    dev.embed_norm(dE, vocab, dtok, n, cols, EPS, dw0, xo0=xo0, y0=y0, a0=a0, x1=dx1, w1=dw1,
                   y1=y1, a1=a1)
    dev.sync()
    assert_bits_equal(xo0.numpy(), emb, "embedding rows")
    for got_y, got_a, x, w, what in ((y0, a0, emb, w0, "set 0"), (y1, a1, x1, w1, "set 1")):
        want = rmsnorm_restated(x, w, EPS)
        assert_bits_equal(got_y.numpy(), want, f"{what} y")
        for got, ref, part in zip(got_a, oracle.quant_a8(want), ("codes", "scales", "fsum")):
            assert_bits_equal(got.numpy(), ref, f"{what} A8 {part}")


@pytest.mark.parametrize("H,n", [(1024, 1), (1024, 5), (1024, 6), (1024, 7), (1024, 8), (256, 3),
                                 (256, 5), (256, 6), (256, 7), (256, 8), (512, 6), (512, 13)])
def test_matmul_embed_norm(dev, H, n):
    """nmx_q4k_matmul_embed_norm (the MTP head's fc projection with its embedding and both input
    norms inside the matmul's workgroups; 13 rows take the two-call path) against
    nmx_embed_norm + nmx_q4k_matmul bit for bit, and against the oracle: the Q4K product of the
    A8 of [restated norm of the oracle's embedding rows | restated norm of h]."""
    print(f"[case] matmul_embed_norm H={H} n={n}", flush=True)
    rng = np.random.default_rng(7 * H + n)
    vocab, rows = 512, H
    E = oracle.q4k_quantize((rng.standard_normal((vocab, H)) * 0.02).astype(np.float32))
    W = gaussian_q4k(rng, rows, 2 * H)
    tok = rng.integers(0, vocab, n).astype(np.int32)
    h = rng.standard_normal((n, H)).astype(np.float32)
    w_emb, w_hid = (rng.uniform(0.5, 1.5, H).astype(np.float32) for _ in range(2))
    dE, dW, dtok, dh = dev.to_device(E), dev.to_device(W), dev.to_device(tok), dev.to_device(h)
    dwe, dwh = dev.to_device(w_emb), dev.to_device(w_hid)
    # separate: both halves' A8 into one 2H-column buffer, then the matmul
    a8 = a8_bufs(dev, n, 2 * H)
    hb = H // 32   # the h half's blocks start at block hb of [block][n][32]
    a1 = (a8[0].offset(hb * n * 32), a8[1].offset(hb * n * 4), a8[2].offset(hb * n * 4))
    dev.embed_norm(dE, vocab, dtok, n, H, EPS, dwe, a0=a8, x1=dh, w1=dwh, a1=a1)
    Yref = dev.zeros((n, rows), np.float32)
    dev.q4k_matmul(dW, rows, 2 * H, n, *a8, Yref)
    Y = dev.zeros((n, rows), np.float32)
    dev.q4k_matmul_embed_norm(dW, rows, Y, n, H, dE, vocab, dtok, dwe, dh, dwh, EPS,
                              a8_tmp=a8_bufs(dev, n, 2 * H))
    dev.sync()
    assert_bits_equal(Y.numpy(), Yref.numpy(), "fused against separate")
    emb = np.stack([oracle.q4k_get_row(E, vocab, H, int(t)) for t in tok])
    act = np.concatenate([rmsnorm_restated(emb, w_emb, EPS), rmsnorm_restated(h, w_hid, EPS)],
                         axis=1)
    q, d, fs = oracle.quant_a8(act)
    assert_bits_equal(Y.numpy(), oracle.q4k_matmul(W, rows, 2 * H, q, d, fs, n), "oracle")


@pytest.mark.gpu
@pytest.mark.parametrize("sel,want_y", [((0, 0), True), ((4, -1), True), ((2, 2), True),
                                         ((9, -1), True), ((3, -1), False)])
def test_rmsnorm_row(dev, sel, want_y):
    """nmx_rmsnorm_row (the MTP head's final norm of one device-selected row): y and the
    one-vector A8 equal the restated norm of row idx + off of x + add and the oracle's A8 of it;
    an index past the rows takes the last row; without y (the draft-only call) the A8 alone."""
    idx0, off = sel
    n, cols = 5, 1024
    print(f"[case] rmsnorm_row idx={idx0} off={off}", flush=True)
    rng = np.random.default_rng(77 + idx0)
    x = rng.standard_normal((n, cols)).astype(np.float32)
    add = rng.standard_normal((n, cols)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    r = min(max(idx0 + off, 0), n - 1)
    want = rmsnorm_restated((x[r] + add[r])[None, :], w, EPS)
    dx, dadd, dw = dev.to_device(x), dev.to_device(add), dev.to_device(w)
    didx = dev.to_device(np.array([idx0], np.int32))
    y = dev.zeros((1, cols), np.float32)
    a = a8_bufs(dev, 1, cols)
    dev.rmsnorm_row(dx, n, cols, dw, EPS, didx, off, add=dadd, y=y if want_y else None, a8=a)
    dev.sync()
    if want_y:
        assert_bits_equal(y.numpy(), want, "y")
    else:
        assert not y.numpy().any(), "y written without being asked for"
    for got, ref, part in zip(a, oracle.quant_a8(want), ("codes", "scales", "fsum")):
        assert_bits_equal(got.numpy(), ref, f"A8 {part}")
