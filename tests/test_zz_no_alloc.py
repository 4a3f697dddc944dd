"""GPU: the allocation-free head entry point (libnmx.so nmx_head_accept_noalloc, its partial
argmax keys in the library's static device array) against nmx_head_accept with a workspace
the caller allocated, through the C ABI. Bar: out (a, bonus, every row's argmax) and the logits
bit-identical, on two calls in a row, the second with a smaller input (the array keeps the
first call's keys); a shape whose keys exceed the array is refused before any launch."""
from __future__ import annotations

import numpy as np
import pytest

from nibblemac_amd import pqtool
from nibblemac_amd.nmx import NmxError

pytestmark = pytest.mark.gpu


def a8(dev, X):
    n, cols = X.shape
    q = dev.empty((cols // 32, n, 32), np.int8)
    d, fs = dev.empty((cols // 32, n), np.float32), dev.empty((cols // 32, n), np.float32)
    dev.quant_a8(dev.to_device(X), n, cols, q, d, fs)
    return q, d, fs


def both(dev, rows, cols, n, accept, seed):
    rng = np.random.default_rng(seed)
    W = dev.to_device(pqtool.gauss_q4k(seed, 0, rows, cols, 0.02))
    q, d, fs = a8(dev, rng.standard_normal((n, cols)).astype(np.float32))
    lw, ln = dev.zeros((n, rows), np.float32), dev.zeros((n, rows), np.float32)
    ow, on = dev.zeros(2 + n, np.int32), dev.zeros(2 + n, np.int32)
    work = dev.zeros(dev.head_work_bytes(rows, n), np.uint8)
    drafts = dev.zeros(max(1, n - 1), np.int32)
    dev.head_accept(W, rows, cols, n, q, d, fs, lw, drafts, work, ow)  # plant `accept` drafts
    dev.sync()
    am = ow.numpy()[2:]
    dr = np.array([am[t] if t < accept else (am[t] + 1) % rows for t in range(n - 1)], np.int32)
    dev.upload(drafts, dr if n > 1 else np.zeros(1, np.int32))
    dev.head_accept(W, rows, cols, n, q, d, fs, lw, drafts, work, ow)
    dev.head_accept_noalloc(W, rows, cols, n, q, d, fs, ln, drafts, on)
    dev.sync()
    return ow.numpy(), on.numpy(), lw.numpy(), ln.numpy()


@pytest.mark.parametrize("rows,cols,n,accept", [(248320, 1024, 5, 2), (65536, 1024, 3, 1)])
def test_noalloc_head_equals_workspace_head(dev, rows, cols, n, accept):
    """Run in this order: the second call is smaller than the first."""
    print(f"[case] head noalloc rows={rows} n={n} accept={accept}", flush=True)
    ow, on, lw, ln = both(dev, rows, cols, n, accept, seed=rows % 97 + n)
    assert ow[0] == accept
    assert np.array_equal(on, ow), (on, ow)
    assert np.array_equal(ln.view(np.uint32), lw.view(np.uint32))


def test_noalloc_head_refuses_shapes_beyond_the_array(dev):
    """Every buffer is NULL: the size check refuses the call first, and were it to let the call
    through, the head's own argument check would refuse it before any launch (with a message
    that this test does not accept)."""
    print("[case] head noalloc over the limit", flush=True)
    rows, n = 1 << 21, 16  # keys of 16 x 8192 workgroups: 1 MiB, above the 512 KiB array
    with pytest.raises(NmxError, match="scratch"):
        dev.head_accept_noalloc(None, rows, 1024, n, None, None, None, None, None, None)
