"""GPU parity of the fused attention entry (nmx_attn_fused: the scores kernel normalises and
rotates its own queries and the pass's new keys and stores the new K / V rows) against the two
calls it replaces (nmx_attn_prep + nmx_attn), which the end-to-end tests pin against the
reference engine (engine/src/forward_attn.c:231-266, forward_kv.c:83-127).

Bar: bit-exact for the attention output and its A8, the scores workspace and both caches
(every byte, the rows written by the pass and the rows left alone). Cases: the three cache
formats, 1 / 5 / 8 tokens (a draft step, a verify pass, the fused kernel's limit), positions
at 0, inside a 32-position chunk, straddling chunks and at the end of the cache, and the
two-call path behind the same entry (64-token prefill chunks, a head size of 128)."""
from __future__ import annotations

import numpy as np
import pytest

from nibblemac_amd.nmx import A8, AttnArgs
from tests.test_gpu_q4k import assert_bits_equal

pytestmark = pytest.mark.gpu


def cache_bytes(rng, kv_dtype, nkv, max_ctx, hd):
    rows = nkv * max_ctx
    if kv_dtype == 0:
        return (rng.standard_normal(rows * hd).astype(np.float32)).view(np.uint8)
    if kv_dtype == 1:
        return rng.standard_normal(rows * hd).astype(np.float16).view(np.uint8)
    codes = rng.integers(-127, 128, rows * hd).astype(np.int8).view(np.uint8)
    scales = rng.uniform(0.001, 0.05, rows).astype(np.float32).view(np.uint8)
    return np.concatenate([codes, scales])


def run(dev, case, fused):
    n, nh, nkv, hd, rot, max_ctx, kvt, pos0 = (case[k] for k in
                                                ("n", "nh", "nkv", "hd", "rot", "max_ctx", "kvt", "pos0"))
    hst = case["host"]
    d = {k: dev.to_device(v) for k, v in hst.items()}
    pos = dev.to_device(np.array([pos0], np.int32))
    o = dev.zeros((n, nh * hd), np.float32)
    nb = nh * hd // 32
    aq, ad, afs = (dev.zeros((nb, n, 32), np.int8), dev.zeros((nb, n), np.float32),
                   dev.zeros((nb, n), np.float32))
    sc = dev.zeros((n, nh, max_ctx), np.float32)
    a = AttnArgs(n, nh, nkv, hd, rot, max_ctx, d["q"].ptr, d["k_in"].ptr, d["v_in"].ptr,
                 d["q_norm"].ptr, d["k_norm"].ptr, 1e-6, np.float32(1.0 / np.sqrt(hd)),
                 d["cos"].ptr, d["sin"].ptr, d["kc"].ptr, d["vc"].ptr, pos.ptr, 0, o.ptr,
                 A8(aq.ptr, ad.ptr, afs.ptr), sc.ptr, kvt)
    if fused:
        dev.attn_fused(a)
    else:
        dev.attn_prep(a)
        dev.attn(a)
    dev.sync()
    return dict(o=o.numpy(), aq=aq.numpy(), ad=ad.numpy(), afs=afs.numpy(), sc=sc.numpy(),
                kc=d["kc"].numpy(), vc=d["vc"].numpy())


CASES = [
    # n, kv dtype, position of token 0, max_ctx, hd
    (5, 0, 0, 1024, 256),
    (5, 0, 30, 1024, 256),    # the pass straddles the chunk at 32
    (5, 0, 517, 1024, 256),
    (1, 0, 600, 1024, 256),
    (5, 1, 517, 1024, 256),
    (1, 1, 31, 1024, 256),
    (5, 2, 517, 1024, 256),
    (1, 2, 1023, 1024, 256),  # the last position of the cache
    (8, 0, 27, 1024, 256),    # the most tokens the fused kernel takes, across a chunk
    (64, 0, 448, 1024, 256),  # a prefill chunk: the two calls behind the same entry
    (64, 2, 40, 1024, 256),
    (5, 0, 517, 600, 256),    # max_ctx not a multiple of the chunk
    (5, 0, 100, 1024, 128),   # outside the fused kernel's limits: the two calls
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "n%d_kv%d_pos%d_ctx%d_hd%d" % c)
def test_attn_fused_equals_prep_and_attn(dev, case):
    n, kvt, pos0, max_ctx, hd = case
    print(f"[case] attn_fused {case}", flush=True)
    nh, nkv, rot = 8, 2, hd // 4
    rng = np.random.default_rng(n * 7 + kvt * 131 + pos0 + hd)
    ang = rng.uniform(0, 2 * np.pi, (max_ctx, rot // 2))
    host = dict(
        q=rng.standard_normal((n, nh, 2 * hd)).astype(np.float32),
        k_in=rng.standard_normal((n, nkv * hd)).astype(np.float32),
        v_in=rng.standard_normal((n, nkv * hd)).astype(np.float32),
        q_norm=rng.uniform(0.5, 1.5, hd).astype(np.float32),
        k_norm=rng.uniform(0.5, 1.5, hd).astype(np.float32),
        cos=np.cos(ang).astype(np.float32), sin=np.sin(ang).astype(np.float32),
        kc=cache_bytes(rng, kvt, nkv, max_ctx, hd), vc=cache_bytes(rng, kvt, nkv, max_ctx, hd),
    )
    c = dict(n=n, nh=nh, nkv=nkv, hd=hd, rot=rot, max_ctx=max_ctx, kvt=kvt, pos0=pos0, host=host)
    want = run(dev, c, fused=False)
    got = run(dev, c, fused=True)
    for k in want:
        assert_bits_equal(got[k], want[k], k)
