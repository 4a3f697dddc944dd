"""GPU parity: A8 quantization and the Q4K x A8 matmul (libnmx.so) against the oracle.

Bar: bit-exact. The fp32 outputs are compared with memcmp semantics (array_equal on the raw
bits) and so are the int32 sub-block sums. Shapes follow the reference's own exactness gate
(engine/metal/check_a8.c:107-113: 4x256, 20x768, 128x3584 at batches 1,2,3,7,8,31,64) plus the
speculative-verify shapes of one Qwen3.5-0.8B layer at k+1 = 5 rows.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from nibblemac_amd.nmx import NmxError

pytestmark = pytest.mark.gpu

DELTANET_LAYER = [("qkv", 6144, 1024), ("z", 2048, 1024), ("b", 16, 1024), ("a", 16, 1024),
                  ("out", 1024, 2048), ("gate", 3584, 1024), ("up", 3584, 1024),
                  ("down", 1024, 3584)]
FULLATTN_LAYER = [("q", 4096, 1024), ("k", 512, 1024), ("v", 512, 1024), ("o", 1024, 2048)]


def gaussian_q4k(rng, rows, cols, std=0.02):
    return oracle.q4k_quantize((rng.standard_normal((rows, cols)) * std).astype(np.float32))


def random_bytes_q4k(rng, rows, cols):
    """Random packed bytes with fixed fp16 D / M per row (engine/metal/check_a8.c:20-27)."""
    W = rng.integers(0, 256, oracle.q4k_nbytes(rows, cols), dtype=np.uint8)
    sb = W.reshape(-1, 576)
    for r in range(8):
        sb[:, 2 * r:2 * r + 2] = np.frombuffer(np.float16((r + 1) * 0.0007).tobytes(), np.uint8)
    return W


def run_gpu(dev, W, rows, cols, X, want_dots=True, y_stride=None):
    n = X.shape[0]
    dX = dev.to_device(X)
    dq = dev.empty((cols // 32, n, 32), np.int8)
    dd = dev.empty((cols // 32, n), np.float32)
    dfs = dev.empty((cols // 32, n), np.float32)
    dev.quant_a8(dX, n, cols, dq, dd, dfs)
    dW = dev.to_device(W)
    ys = y_stride or rows
    dY = dev.zeros((n, ys), np.float32)
    ddots = dev.zeros((n, rows, cols // 32), np.int32) if want_dots else None
    dev.q4k_matmul(dW, rows, cols, n, dq, dd, dfs, dY, ys, ddots)
    dev.sync()
    out = dict(q=dq.numpy(), d=dd.numpy(), fs=dfs.numpy(), Y=dY.numpy()[:, :rows])
    if want_dots:
        out["dots"] = ddots.numpy()
    for b in (dX, dq, dd, dfs, dW, dY, ddots):
        if b is not None:
            b.free()
    return out


def assert_bits_equal(a, b, what):
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    assert a.shape == b.shape, what
    if a.dtype == np.float32:
        a, b = a.view(np.uint32), b.view(np.uint32)
    bad = np.flatnonzero(a.ravel() != b.ravel())
    assert bad.size == 0, f"{what}: {bad.size} mismatches, first at {bad[0]}: {a.ravel()[bad[0]]} vs {b.ravel()[bad[0]]}"


def check_case(dev, W, rows, cols, X, dots=True):
    """Both device paths: the one that also returns the int32 sub-block sums (row-per-lane /
    K-split kernels) and the production one (small-row shapes: every vector of a pass in one
    workgroup, chains from LDS)."""
    q, d, fs = oracle.quant_a8(X)
    ref = oracle.q4k_matmul(W, rows, cols, q, d, fs, X.shape[0], want_dots=dots)
    Yr, Dr = ref if dots else (ref, None)
    got = run_gpu(dev, W, rows, cols, X, want_dots=dots)
    assert_bits_equal(got["q"], q, "A8 codes")
    assert_bits_equal(got["d"], d, "A8 scales")
    assert_bits_equal(got["fs"], fs, "A8 fsum")
    if dots:
        assert_bits_equal(got["dots"], Dr, "int32 sub-block sums")
        assert_bits_equal(got["Y"], Yr, "fp32 outputs (dots path)")
        got = run_gpu(dev, W, rows, cols, X, want_dots=False)
    assert_bits_equal(got["Y"], Yr, "fp32 outputs")


@pytest.mark.parametrize("n", [1, 2, 3, 7, 8, 31, 64])
@pytest.mark.parametrize("rows,cols", [(4, 256), (20, 768), (128, 3584)])
def test_q4k_check_a8_shapes(dev, rows, cols, n):
    print(f"[case] check_a8 shape rows={rows} cols={cols} n={n}", flush=True)
    rng = np.random.default_rng(1000 + rows + n)
    W = random_bytes_q4k(rng, rows, cols)
    X = (rng.integers(0, 2001, (n, cols)) - 1000).astype(np.float32) / np.float32(997.0)
    check_case(dev, W, rows, cols, X)


def test_q4k_3584x1024_matvec(dev):
    """3584x1024 Q4K (N(0, 0.02) quantized), one activation row N(0, 1)."""
    print("[case] matvec 3584x1024 n=1", flush=True)
    rng = np.random.default_rng(1)
    W = gaussian_q4k(rng, 3584, 1024)
    X = rng.standard_normal((1, 1024)).astype(np.float32)
    check_case(dev, W, 3584, 1024, X)


@pytest.mark.parametrize("layer", ["deltanet", "fullattn"])
def test_q4k_verify_layer_5_rows(dev, layer):
    """Every matrix of one decoder layer against k+1 = 5 activation rows."""
    mats = DELTANET_LAYER if layer == "deltanet" else FULLATTN_LAYER
    rng = np.random.default_rng(2)
    for name, rows, cols in mats:
        print(f"[case] verify layer {layer}.{name} {rows}x{cols} n=5", flush=True)
        W = gaussian_q4k(rng, rows, cols)
        X = rng.standard_normal((5, cols)).astype(np.float32)
        check_case(dev, W, rows, cols, X)


def test_q4k_batch_equals_single(dev):
    """Row v of an n-vector call equals the single-vector call bit for bit (kbench.c:216-223)."""
    rng = np.random.default_rng(3)
    rows, cols = 1024, 2048
    W = gaussian_q4k(rng, rows, cols)
    X = rng.standard_normal((5, cols)).astype(np.float32)
    full = run_gpu(dev, W, rows, cols, X, want_dots=False)["Y"]
    for v in range(5):
        one = run_gpu(dev, W, rows, cols, X[v:v + 1], want_dots=False)["Y"]
        assert_bits_equal(one[0], full[v], f"vector {v}")


@pytest.mark.parametrize("n", [5, 64])
def test_q4k_multi_segment(dev, n):
    """The fused launch of several matrices gives each matrix's own result (n = 64: the prefill
    kernel, whose 16-row groups straddle no segment)."""
    print(f"[case] multi-segment n={n}", flush=True)
    rng = np.random.default_rng(4)
    cols = 1024
    shapes = [6144, 2048, 16, 16]
    Ws = [gaussian_q4k(rng, r, cols) for r in shapes]
    X = rng.standard_normal((n, cols)).astype(np.float32)
    q, d, fs = oracle.quant_a8(X)
    dq, dd, dfs = dev.to_device(q), dev.to_device(d), dev.to_device(fs)
    dWs = [dev.to_device(w) for w in Ws]
    strides = [r + 12 for r in shapes]
    dYs = [dev.zeros((n, s), np.float32) for s in strides]
    dev.q4k_matmul_multi(dWs, shapes, dYs, strides, cols, n, dq, dd, dfs)
    dev.sync()
    for W, r, dY in zip(Ws, shapes, dYs):
        ref = oracle.q4k_matmul(W, r, cols, q, d, fs, n)
        assert_bits_equal(dY.numpy()[:, :r], ref, f"segment rows={r}")
        assert not dY.numpy()[:, r:].any(), "padding columns written"


@pytest.mark.parametrize("n,cols", [(3, 1024), (4, 2048), (5, 1024), (6, 3584), (7, 1024),
                                    (8, 4096), (11, 1024)])
def test_q4k_matrix_core_matvec(dev, n, cols):
    """Matrices past 32767 rows at 3..8 vectors per pass take the matrix-core kernel
    (q4k_mvx_k, block-diagonal activation operand); n = 11 runs as passes of 6 and 5. Two
    segments, the second ending inside a wave, outputs with padded strides; bit-exact against
    the oracle, padding untouched. cols = 4096 at 8 vectors fills the activation table's 64 KB."""
    print(f"[case] matrix-core matvec n={n} cols={cols}", flush=True)
    rng = np.random.default_rng(70 + n)
    shapes = [32768, 1000]
    Ws = [gaussian_q4k(rng, r, cols) for r in shapes]
    X = rng.standard_normal((n, cols)).astype(np.float32)
    q, d, fs = oracle.quant_a8(X)
    dq, dd, dfs = dev.to_device(q), dev.to_device(d), dev.to_device(fs)
    dWs = [dev.to_device(w) for w in Ws]
    strides = [r + 4 for r in shapes]
    dYs = [dev.zeros((n, s), np.float32) for s in strides]
    dev.q4k_matmul_multi(dWs, shapes, dYs, strides, cols, n, dq, dd, dfs)
    dev.sync()
    for W, r, dY in zip(Ws, shapes, dYs):
        ref = oracle.q4k_matmul(W, r, cols, q, d, fs, n)
        assert_bits_equal(dY.numpy()[:, :r], ref, f"segment rows={r}")
        assert not dY.numpy()[:, r:].any(), "padding columns written"
    for b in (dq, dd, dfs, *dWs, *dYs):
        b.free()


@pytest.mark.parametrize("n", [9, 16, 17, 40, 64])
def test_q4k_prefill_chunk(dev, n):
    """More than 8 vectors (prefill chunks, the MFMA kernel): ragged vector tiles, a matrix whose
    rows are not a multiple of 16, one wave per vector tile (1024 rows) and every tile in one
    wave (8224 rows)."""
    rng = np.random.default_rng(5000 + n)
    for rows, cols in [(20, 256), (1024, 3584), (8224, 1024)]:
        print(f"[case] prefill chunk rows={rows} cols={cols} n={n}", flush=True)
        W = gaussian_q4k(rng, rows, cols)
        X = rng.standard_normal((n, cols)).astype(np.float32)
        check_case(dev, W, rows, cols, X, dots=False)


def test_q4k_invalid_calls_rejected(dev):
    """Invalid shapes and aliasing are refused on the host before any launch
    (engine/metal/check_a8.c:71-100)."""
    W = dev.zeros(576, np.uint8)
    q = dev.zeros(256, np.int8)
    d = dev.zeros(8, np.float32)
    fs = dev.zeros(8, np.float32)
    Y = dev.zeros(4, np.float32)
    bad = [
        dict(rows=3, cols=256, n=1), dict(rows=4, cols=255, n=1), dict(rows=4, cols=256, n=0),
        dict(rows=4, cols=256, n=65), dict(rows=4, cols=256, n=1, y_stride=3),
    ]
    for b in bad:
        with pytest.raises(NmxError):
            dev.q4k_matmul(W, b["rows"], b["cols"], b["n"], q, d, fs, Y, b.get("y_stride"))
    with pytest.raises(NmxError):
        dev.q4k_matmul(W, 4, 256, 1, q, d, fs, W)  # output aliases the weights
    with pytest.raises(NmxError):
        dev.q4k_matmul(W, 4, 256, 1, q, d, fs, d)  # output aliases the scales
    with pytest.raises(NmxError):
        dev.q4k_matmul(None, 4, 256, 1, q, d, fs, Y)
    with pytest.raises(NmxError):
        dev.quant_a8(Y, 1, 255, q, d, fs)
