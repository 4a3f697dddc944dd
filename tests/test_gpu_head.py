"""GPU parity: LM head (Q4K matvec over k + 1 rows) fused with greedy argmax and draft
acceptance (libnmx.so nmx_head_accept) against the oracle.

Bar: logits bit-exact, every argmax and the accepted count / bonus token identical
(engine/src/spec.c:340-345, engine/src/forward_ops.c:387-409).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from tests.test_gpu_q4k import assert_bits_equal

pytestmark = pytest.mark.gpu


def quantized_head(rng, rows, cols, chunk=16384):
    out = np.empty(oracle.q4k_nbytes(rows, cols), np.uint8)
    per = oracle.q4k_nbytes(4, cols) // 4
    for r0 in range(0, rows, chunk):
        r1 = min(rows, r0 + chunk)
        w = (rng.standard_normal((r1 - r0, cols), dtype=np.float32) * np.float32(0.02))
        out[r0 * per:r1 * per] = oracle.q4k_quantize(w)
    return out


def planted_drafts(argmax_rows, a, k):
    """Drafts d_1..d_k with exactly a accepted: d_t = argmax(row t-1) for t <= a, then a draft
    that differs from argmax(row a) (acceptance planted at 0 / 50 / 100 %)."""
    d = np.zeros(k, np.int32)
    for t in range(k):
        d[t] = argmax_rows[t] if t < a else (argmax_rows[t] + 1 + t) % 1000003
    return d


def run_head(dev, W, rows, cols, X, drafts, logits=True):
    n = X.shape[0]
    q, d, fs = oracle.quant_a8(X)
    dW, dq, dd, dfs = dev.to_device(W), dev.to_device(q), dev.to_device(d), dev.to_device(fs)
    dl = dev.zeros((n, rows), np.float32) if logits else None
    ddr = dev.to_device(np.asarray(drafts, np.int32)) if n > 1 else None
    work = dev.zeros(dev.head_work_bytes(rows, n), np.uint8)
    out = dev.zeros(2 + n, np.int32)
    dev.head_accept(dW, rows, cols, n, dq, dd, dfs, dl, ddr, work, out)
    dev.sync()
    res = out.numpy(), (dl.numpy() if logits else None)
    for b in (dW, dq, dd, dfs, dl, ddr, work, out):
        if b is not None:
            b.free()
    return res


_HEAD_CASE: dict = {}


def head_248320x1024_case():
    """248320 x 1024 Q4K head (N(0, 0.02) quantized) and 5 rows N(0, 1), built once."""
    if not _HEAD_CASE:
        rng = np.random.default_rng(40)
        rows, cols = 248320, 1024
        W = quantized_head(rng, rows, cols)
        X = rng.standard_normal((5, cols)).astype(np.float32)
        q, d, fs = oracle.quant_a8(X)
        _HEAD_CASE.update(W=W, X=X, ref=oracle.q4k_matmul(W, rows, cols, q, d, fs, 5, threads=8))
    return _HEAD_CASE["W"], _HEAD_CASE["X"], _HEAD_CASE["ref"]


@pytest.mark.parametrize("accept", [0, 2, 4])
def test_head_248320x1024_accept(dev, accept):
    """The config-4 head with 4 planted drafts at 0 / 50 / 100 % acceptance."""
    print(f"[case] head 248320x1024 accept={accept}", flush=True)
    rows, cols = 248320, 1024
    W, X, ref = head_248320x1024_case()
    am = np.array([oracle.argmax(ref[t]) for t in range(5)], np.int32)
    drafts = planted_drafts(am, accept, 4)
    a_ref, bonus_ref, rows_ref = oracle.accept(ref, drafts)
    assert a_ref == accept
    out, logits = run_head(dev, W, rows, cols, X, drafts)
    assert np.array_equal(logits.view(np.uint32), ref.view(np.uint32)), "logits differ"
    assert out[0] == a_ref and out[1] == bonus_ref, (out[:2], a_ref, bonus_ref)
    assert np.array_equal(out[2:], rows_ref)


def test_head_ties_pick_first_index(dev):
    """Duplicate tiles give equal logits: the first index of the maximum wins, across waves."""
    rng = np.random.default_rng(41)
    rows, cols = 8192, 512
    W = quantized_head(rng, rows, cols)
    per = oracle.q4k_nbytes(4, cols)
    Y0 = oracle.q4k_matmul(W, rows, cols, *oracle.quant_a8(np.ones((1, cols), np.float32)), 1)
    best = int(np.argmax(Y0[0])) // 4
    for dst in (best + 1, best + 700, rows // 4 - 1):  # same wave, another wave, the last tile
        if dst < rows // 4:
            W[dst * per:(dst + 1) * per] = W[best * per:(best + 1) * per]
    X = np.ones((3, cols), np.float32)
    X[1] *= -1
    q, d, fs = oracle.quant_a8(X)
    ref = oracle.q4k_matmul(W, rows, cols, q, d, fs, 3)
    am = [oracle.argmax(ref[t]) for t in range(3)]
    out, logits = run_head(dev, W, rows, cols, X, np.array([am[0], am[1]], np.int32))
    assert np.array_equal(logits.view(np.uint32), ref.view(np.uint32))
    assert list(out[2:]) == am
    assert out[0] == 2 and out[1] == am[2]


@pytest.mark.parametrize("n", [1, 2, 3, 5, 8, 9])
def test_head_widths_and_no_logits(dev, n):
    """Any verify width (k = n - 1, plain step at n = 1; 3..8 on the matrix cores, 9 as passes
    of 5 and 4), logits optional."""
    rng = np.random.default_rng(42 + n)
    rows, cols = 32768, 1024
    W = quantized_head(rng, rows, cols)
    X = rng.standard_normal((n, cols)).astype(np.float32)
    q, d, fs = oracle.quant_a8(X)
    ref = oracle.q4k_matmul(W, rows, cols, q, d, fs, n)
    am = np.array([oracle.argmax(ref[t]) for t in range(n)], np.int32)
    drafts = planted_drafts(am, n // 2, n - 1) if n > 1 else np.zeros(0, np.int32)
    a_ref, bonus_ref, _ = oracle.accept(ref, drafts)
    out, _ = run_head(dev, W, rows, cols, X, drafts, logits=False)
    assert out[0] == a_ref and out[1] == bonus_ref
    assert np.array_equal(out[2:], am)


@pytest.mark.parametrize("n", [3, 5, 8])
def test_head_2048_cols_widths(dev, n):
    """A 2048-column head (8 superblocks per row): the one-launch head at 3-7 rows, and at 8 rows
    the row-per-lane matrix-core kernel it falls back to in 16-wave workgroups; logits
    bit-exact, argmax and acceptance equal."""
    print(f"[case] head 2048 cols n={n}", flush=True)
    rng = np.random.default_rng(70 + n)
    rows, cols = 16384, 2048
    W = quantized_head(rng, rows, cols)
    X = rng.standard_normal((n, cols)).astype(np.float32)
    q, d, fs = oracle.quant_a8(X)
    ref = oracle.q4k_matmul(W, rows, cols, q, d, fs, n, threads=8)
    am = np.array([oracle.argmax(ref[t]) for t in range(n)], np.int32)
    drafts = planted_drafts(am, n // 2, n - 1)
    a_ref, bonus_ref, _ = oracle.accept(ref, drafts)
    out, logits = run_head(dev, W, rows, cols, X, drafts)
    assert_bits_equal(logits, ref, f"logits 2048 cols n={n}")
    assert out[0] == a_ref and out[1] == bonus_ref
    assert np.array_equal(out[2:], am)


def test_head_accept_graph_replays_reuse_work(dev):
    """The fused argmax keeps its device-wide state in the caller's work buffer and leaves it
    reset: consecutive calls and several replays of one captured graph (with eager uploads of new
    drafts between them) all give the oracle's answer."""
    rng = np.random.default_rng(44)
    rows, cols, n = 65536, 1024, 5
    W = quantized_head(rng, rows, cols)
    X = rng.standard_normal((n, cols)).astype(np.float32)
    q, d, fs = oracle.quant_a8(X)
    ref = oracle.q4k_matmul(W, rows, cols, q, d, fs, n)
    am = np.array([oracle.argmax(ref[t]) for t in range(n)], np.int32)
    dW, dq, dd, dfs = dev.to_device(W), dev.to_device(q), dev.to_device(d), dev.to_device(fs)
    ddr = dev.zeros(n - 1, np.int32)
    work = dev.zeros(dev.head_work_bytes(rows, n), np.uint8)
    out = dev.zeros(2 + n, np.int32)
    dev.graph_begin()
    dev.head_accept(dW, rows, cols, n, dq, dd, dfs, None, ddr, work, out)
    g = dev.graph_end()
    for rep, a in enumerate([4, 0, 2, 4, 1]):
        drafts = planted_drafts(am, a, n - 1)
        dev.upload(ddr, drafts)
        if rep % 2:
            dev.head_accept(dW, rows, cols, n, dq, dd, dfs, None, ddr, work, out)
        else:
            dev.graph_launch(g)
        dev.sync()
        got = out.numpy()
        a_ref, bonus_ref, _ = oracle.accept(ref, drafts)
        assert got[0] == a_ref and got[1] == bonus_ref, (rep, got, a_ref, bonus_ref)
        assert np.array_equal(got[2:], am)



@pytest.mark.parametrize("a", [0, 2, 4])
def test_accept_commit_mailbox(dev, a):
    """nmx_accept_commit_mb: vt[a + 1] = bonus and ctl[1] = a + 1 as nmx_accept_commit, and
    the host mailbox holds [a, bonus, vt after the update] with its flag word set last (the
    engine clears the flag before the launch and polls it)."""
    import ctypes

    k = 4
    vt0 = np.arange(100, 100 + k + 2, dtype=np.int32)
    out = dev.to_device(np.array([a, 777] + [0] * (k + 1), np.int32))
    vt, ctl = dev.to_device(vt0), dev.zeros(16, np.int32)
    nvt = k + 2
    mb = dev.host_alloc((3 + nvt) * 4)
    try:
        view = (ctypes.c_int32 * (3 + nvt)).from_address(mb)
        for i in range(3 + nvt):
            view[i] = -1
        view[2 + nvt] = 0
        dev.accept_commit(out, vt, ctl, mailbox=mb, nvt=nvt)
        dev.sync()
        want_vt = vt0.copy()
        want_vt[a + 1] = 777
        assert list(view) == [a, 777] + list(want_vt) + [1]
        assert np.array_equal(vt.numpy(), want_vt) and ctl.numpy()[1] == a + 1
    finally:
        dev.host_free(mb)
        for b in (out, vt, ctl):
            b.free()


@pytest.mark.parametrize("accept,mailbox", [(0, True), (2, True), (4, True), (3, False)])
def test_head_accept_commit_equals_two_launches(dev, accept, mailbox):
    """nmx_head_accept_commit (the accept commit inside the head's last kernel) against
    nmx_head_accept + nmx_accept_commit(_mb) on the same inputs: out, vt, ctl and the mailbox
    identical, the drafts being vt[1..k] as in the verify round."""
    import ctypes

    print(f"[case] head_accept_commit accept={accept} mailbox={mailbox}", flush=True)
    rng = np.random.default_rng(70 + accept)
    rows, cols, k = 32768, 1024, 4
    n = k + 1
    W = quantized_head(rng, rows, cols)
    X = rng.standard_normal((n, cols)).astype(np.float32)
    q, d, fs = oracle.quant_a8(X)
    ref = oracle.q4k_matmul(W, rows, cols, q, d, fs, n, threads=8)
    am = np.array([oracle.argmax(ref[t]) for t in range(n)], np.int32)
    vt0 = np.concatenate([[12345], planted_drafts(am, accept, k)]).astype(np.int32)
    dW, dq, dd, dfs = dev.to_device(W), dev.to_device(q), dev.to_device(d), dev.to_device(fs)
    nvt = k + 2
    got = []
    for fused in (False, True):
        vt = dev.to_device(np.concatenate([vt0, [-1]]).astype(np.int32))
        ctl = dev.to_device(np.full(16, 9, np.int32))
        work = dev.zeros(dev.head_work_bytes(rows, n), np.uint8)
        out = dev.zeros(2 + n, np.int32)
        mb = dev.host_alloc((3 + nvt) * 4) if mailbox else None
        try:
            if mb:
                view = (ctypes.c_int32 * (3 + nvt)).from_address(mb)
                for i in range(3 + nvt):
                    view[i] = -7
                view[2 + nvt] = 0
            if fused:
                dev.head_accept_commit(dW, rows, cols, n, dq, dd, dfs, vt.ptr + 4, work, out, vt,
                                       ctl, mailbox=mb, nvt=nvt if mb else 0)
            else:
                dev.head_accept(dW, rows, cols, n, dq, dd, dfs, None, vt.ptr + 4, work, out)
                dev.accept_commit(out, vt, ctl, mailbox=mb, nvt=nvt)
            dev.sync()
            got.append((out.numpy(), vt.numpy(), ctl.numpy(), list(view) if mb else None))
        finally:
            if mb:
                dev.host_free(mb)
            for b in (vt, ctl, work, out):
                b.free()
    for b in (dW, dq, dd, dfs):
        b.free()
    (o0, v0, c0, m0), (o1, v1, c1, m1) = got
    a_ref, bonus_ref, _ = oracle.accept(ref, vt0[1:])
    assert o0[0] == a_ref == accept and o0[1] == bonus_ref
    assert np.array_equal(o0, o1) and np.array_equal(v0, v1) and np.array_equal(c0, c1)
    assert v1[accept + 1] == bonus_ref and c1[1] == accept + 1
    if mailbox:
        assert m0 == m1 and m1[-1] == 1 and m1[:2] == [accept, bonus_ref]


@pytest.mark.parametrize("rows,k,accept", [(248320, 4, 0), (248320, 4, 2), (248320, 4, 4),
                                            (32768, 4, 3), (32768, 8, 5), (32768, 1, 1)])
def test_head_keys_commit_equals_head_accept_commit(dev, rows, k, accept):
    """The round's verify tail with the reduction inside the commit (nmx_head_keys, then
    nmx_lin_commit_keys: every commit workgroup resolves the argmax keys and the acceptance)
    against nmx_head_accept_commit + nmx_lin_commit on the same inputs: out, vt, ctl, the
    mailbox, the conv state, its backup and the pending rows identical; a and the bonus equal
    the oracle's. The drafts are vt[1..k], as in the verify round."""
    import ctypes

    from nibblemac_amd.nmx import AcceptKeys, CommitArgs

    print(f"[case] head_keys commit rows={rows} k={k} accept={accept}", flush=True)
    rng = np.random.default_rng(90 + rows % 7 + k + accept)
    cols, n = 1024, k + 1
    W = quantized_head(rng, rows, cols)
    X = rng.standard_normal((n, cols)).astype(np.float32)
    q, d, fs = oracle.quant_a8(X)
    ref = oracle.q4k_matmul(W, rows, cols, q, d, fs, n, threads=8)
    am = np.array([oracle.argmax(ref[t]) for t in range(n)], np.int32)
    vt0 = np.concatenate([[12345], planted_drafts(am, accept, k)]).astype(np.int32)
    layers, C, conv_k, cap, row = 3, 640, 4, 9, 2 * (16 + 16 + 1)
    st0 = rng.standard_normal((layers, conv_k - 1, C)).astype(np.float32)
    xin0 = rng.standard_normal((layers, cap, C)).astype(np.float32)
    log0 = rng.standard_normal((layers, cap, row)).astype(np.float32)
    dW, dq, dd, dfs = dev.to_device(W), dev.to_device(q), dev.to_device(d), dev.to_device(fs)
    dxin, dlog = dev.to_device(xin0), dev.to_device(log0)
    nvt = k + 2
    got = []
    for fused in (False, True):
        vt = dev.to_device(np.concatenate([vt0, [-1]]).astype(np.int32))
        ctl = dev.to_device(np.full(16, 9, np.int32))
        work = dev.zeros(dev.head_work_bytes(rows, n), np.uint8)
        dcopy = dev.zeros(16, np.int32)
        out = dev.zeros(2 + n, np.int32)
        state, bak = dev.to_device(st0), dev.zeros(st0.shape, np.float32)
        pend = dev.zeros((layers, cap, row), np.float32)
        mb = dev.host_alloc((3 + nvt) * 4)
        try:
            view = (ctypes.c_int32 * (3 + nvt)).from_address(mb)
            for i in range(3 + nvt):
                view[i] = -7
            view[2 + nvt] = 0
            args = CommitArgs(layers, C, conv_k, state.ptr, dxin.ptr, dlog.ptr, pend.ptr, cap, row,
                              ctl.ptr, vt.ptr, bak.ptr, 0)
            if fused:
                dev.head_keys(dW, rows, cols, n, dq, dd, dfs, vt.ptr + 4, work, dcopy)
                keys = AcceptKeys(work.ptr, dev.head_nkeys(rows, cols, n), n, dcopy.ptr, out.ptr,
                                  mb, nvt)
                dev.lin_commit(args, keys)
            else:
                dev.head_accept_commit(dW, rows, cols, n, dq, dd, dfs, vt.ptr + 4, work, out, vt,
                                       ctl, mailbox=mb, nvt=nvt)
                dev.lin_commit(args)
            dev.sync()
            got.append((out.numpy(), vt.numpy(), ctl.numpy(), list(view), state.numpy(),
                        bak.numpy(), pend.numpy()))
        finally:
            dev.host_free(mb)
            for b in (vt, ctl, work, dcopy, out, state, bak, pend):
                b.free()
    for b in (dW, dq, dd, dfs, dxin, dlog):
        b.free()
    a_ref, bonus_ref, _ = oracle.accept(ref, vt0[1:])
    assert a_ref == accept
    two, one = got
    for name, x, y in zip(("out", "vt", "ctl", "mailbox", "state", "bak", "pend"), two, one):
        assert np.array_equal(np.asarray(x), np.asarray(y)), name
    o, v, c, m = one[:4]
    assert o[0] == accept and o[1] == bonus_ref and list(o[2:]) == list(am)
    assert v[accept + 1] == bonus_ref and v[0] == bonus_ref and c[1] == accept + 1
    assert c[2] == accept and m[:2] == [accept, bonus_ref] and m[-1] == 1


def test_head_accept_to_writes_token(dev):
    """nmx_head_accept_to stores out[1] (the greedy token) at tok_dst as well."""
    rng = np.random.default_rng(5)
    rows, cols = 4096, 1024
    W = quantized_head(rng, rows, cols)
    X = rng.standard_normal((1, cols)).astype(np.float32)
    q, d, fs = oracle.quant_a8(X)
    ref = oracle.q4k_matmul(W, rows, cols, q, d, fs, 1)
    dW, dq, dd, dfs = dev.to_device(W), dev.to_device(q), dev.to_device(d), dev.to_device(fs)
    work = dev.zeros(dev.head_work_bytes(rows, 1), np.uint8)
    out, tok = dev.zeros(3, np.int32), dev.to_device(np.array([-5, -6], np.int32))
    dev.head_accept(dW, rows, cols, 1, dq, dd, dfs, None, None, work, out, tok_dst=tok.ptr + 4)
    dev.sync()
    g = oracle.argmax(ref[0])
    assert list(out.numpy()) == [0, g, g] and list(tok.numpy()) == [-5, g]
    for b in (dW, dq, dd, dfs, work, out, tok):
        b.free()


@pytest.mark.parametrize("case", [(0, 0, 1, 32768, True, True), (3, -1, 5, 32768, True, True),
                                  (9, -1, 5, 10004, True, False), (0, -1, 5, 32768, False, True)],
                         ids=["row0_of1", "row2_of5", "clamped_no_y", "below0_no_add"])
def test_head_row_accept_equals_norm_then_head(dev, case):
    """nmx_head_row_accept_to (the MTP draft head with its final RMSNorm inside the head's
    workgroups) against nmx_rmsnorm_row + nmx_head_accept_to: the argmax, the draft written to
    tok_dst and the normed row y bit for bit, for a device-selected row (clamped at both ends),
    with and without the residual add and the y output; with a control block to advance
    (n_past += e by the head's last kernel) on the cases that keep y."""
    idx0, off, nrows, rows, with_add, want_y = case
    cols, eps = 1024, 1e-6
    print(f"[case] head_row_accept {case}", flush=True)
    rng = np.random.default_rng(500 + idx0 + rows)
    W = quantized_head(rng, rows, cols)
    x = rng.standard_normal((nrows, cols)).astype(np.float32)
    add = rng.standard_normal((nrows, cols)).astype(np.float32) if with_add else None
    w = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    dW, dx, dw = dev.to_device(W), dev.to_device(x), dev.to_device(w)
    dadd = dev.to_device(add) if with_add else None
    didx = dev.to_device(np.array([idx0], np.int32))
    nb = cols // 32
    a8 = (dev.zeros((nb, 1, 32), np.int8), dev.zeros((nb, 1), np.float32),
          dev.zeros((nb, 1), np.float32))
    y_ref = dev.zeros((1, cols), np.float32)
    dev.rmsnorm_row(dx, nrows, cols, dw, eps, didx, off, add=dadd, y=y_ref, a8=a8)
    work_ref = dev.zeros(dev.head_work_bytes(rows, 1), np.uint8)
    out_ref, tok_ref = dev.zeros(3, np.int32), dev.zeros(1, np.int32)
    dev.head_accept(dW, rows, cols, 1, *a8, None, None, work_ref, out_ref, tok_dst=tok_ref)
    y = dev.zeros((1, cols), np.float32)
    work = dev.zeros(dev.head_work_bytes(rows, 1), np.uint8)
    out, tok = dev.zeros(3, np.int32), dev.zeros(1, np.int32)
    ctl0 = np.array([1000 + idx0, 3 + idx0, 77], np.int32)
    dctl = dev.to_device(ctl0) if want_y else None
    dev.head_row_accept_to(dW, rows, cols, dx, nrows, dw, eps, didx, off, work, out, tok,
                           add=dadd, y=y if want_y else None, advance=dctl)
    dev.sync()
    if want_y:
        assert dctl.numpy().tolist() == [ctl0[0] + ctl0[1], ctl0[1], 77], "control block"
    assert_bits_equal(out.numpy(), out_ref.numpy(), "out")
    assert_bits_equal(tok.numpy(), tok_ref.numpy(), "draft token")
    if want_y:
        assert_bits_equal(y.numpy(), y_ref.numpy(), "y")
    else:
        assert not y.numpy().any(), "y written without being asked for"


@pytest.mark.parametrize("rows,n", [(32768, 5), (10004, 1), (2048, 3)])
def test_head_row_keys_resolved_by_consumers(dev, rows, n):
    """nmx_head_row_keys (the draft head without its reduction) resolved by its two consumers:
    nmx_embed_norm_keys (the verify's first norm, last row) and nmx_q4k_matmul_embed_norm with
    tok_keys (the next MTP pass's fc input). The token each writes equals the one
    nmx_head_row_accept_to returns, and their outputs equal those of the same calls given that
    token, bit for bit."""
    cols, eps, vocab = 1024, 1e-6, rows
    print(f"[case] head_row_keys rows={rows} n={n}", flush=True)
    rng = np.random.default_rng(900 + rows + n)
    W = quantized_head(rng, rows, cols)
    x = rng.standard_normal((3, cols)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    dW, dx, dw = dev.to_device(W), dev.to_device(x), dev.to_device(w)
    didx = dev.to_device(np.array([1], np.int32))
    # the token by the head with its own reduction
    work = dev.zeros(dev.head_work_bytes(rows, 1), np.uint8)
    out, tok_ref = dev.zeros(3, np.int32), dev.zeros(1, np.int32)
    dev.head_row_accept_to(dW, rows, cols, dx, 3, dw, eps, didx, 0, work, out, tok_ref)
    nk = dev.head_row_nkeys(rows)
    keys = dev.zeros(nk, np.uint64)
    y = dev.zeros((1, cols), np.float32)
    dev.head_row_keys(dW, rows, cols, dx, 3, dw, eps, didx, 0, keys, y=y)
    dev.sync()
    t = int(tok_ref.numpy()[0])
    # the verify's first norm: rows 0..n-2 from tok, row n-1 from the keys
    toks = rng.integers(0, vocab, n).astype(np.int32)
    toks_ref = toks.copy()
    toks_ref[n - 1] = t
    toks[n - 1] = -7  # never read
    dtok, dtok_ref = dev.to_device(toks), dev.to_device(toks_ref)
    xo, xo_ref = dev.zeros((n, cols), np.float32), dev.zeros((n, cols), np.float32)
    a8 = tuple(dev.zeros(s, t_) for s, t_ in (((cols // 32, n, 32), np.int8),
                                              ((cols // 32, n), np.float32),
                                              ((cols // 32, n), np.float32)))
    a8_ref = tuple(dev.zeros(s, t_) for s, t_ in (((cols // 32, n, 32), np.int8),
                                                  ((cols // 32, n), np.float32),
                                                  ((cols // 32, n), np.float32)))
    dev.embed_norm_keys(dW, vocab, dtok, n, cols, eps, dw, keys, nk, xo=xo, a8=a8)
    dev.embed_norm(dW, vocab, dtok_ref, n, cols, eps, dw, xo0=xo_ref, a0=a8_ref)
    # the fc input of the next pass: one row, its token from the keys
    H = cols
    Wfc = quantized_head(rng, H, 2 * H)
    h = rng.standard_normal((1, H)).astype(np.float32)
    dWfc, dh = dev.to_device(Wfc), dev.to_device(h)
    tk1, tk1_ref = dev.to_device(np.array([-5], np.int32)), dev.to_device(np.array([t], np.int32))
    Y, Y_ref = dev.zeros((1, H), np.float32), dev.zeros((1, H), np.float32)
    dev.q4k_matmul_embed_norm(dWfc, H, Y, 1, H, dW, vocab, tk1, dw, dh, dw, eps, tok_keys=keys,
                              nkeys=nk)
    dev.q4k_matmul_embed_norm(dWfc, H, Y_ref, 1, H, dW, vocab, tk1_ref, dw, dh, dw, eps)
    dev.sync()
    assert int(dtok.numpy()[n - 1]) == t, "embed_norm_keys token"
    assert_bits_equal(dtok.numpy(), toks_ref, "token row")
    assert_bits_equal(xo.numpy(), xo_ref.numpy(), "embedding rows")
    for a, b, what in zip(a8, a8_ref, ("codes", "scales", "fsum")):
        assert_bits_equal(a.numpy(), b.numpy(), f"A8 {what}")
    assert int(tk1.numpy()[0]) == t, "fc token"
    assert_bits_equal(Y.numpy(), Y_ref.numpy(), "fc output")
