"""Pins of the oracle's Gated DeltaNet recurrence, rollback log and replay (CPU only).

  - bit for bit against the reference's own scalar code (engine/src/matvec_ref.c, compiled
    from its sources into oracle/_ref/ where the reference is present);
  - against the closed form S' = a S (I - b k k^T) + b v k^T (per head, state as [v][k]),
    o = S' q, evaluated in float64 (tolerance 1e-5 relative);
  - replay of logged rows == running those tokens directly;
  - a planted mistake (k and q swapped) fails the closed-form check.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle


def inputs(rng, n, heads, rep, dk, dv, pad=3):
    kd = heads // rep * dk
    stride = 2 * kd + heads * dv + pad
    qkv = rng.standard_normal((n, stride)).astype(np.float32)
    for t in range(n):   # L2-normalised q and k per head
        for u in range(2 * (heads // rep)):
            seg = qkv[t, u * dk:(u + 1) * dk]
            seg /= np.float32(np.linalg.norm(seg))
    decay = (0.9 + 0.1 * rng.random((n, heads))).astype(np.float32)
    beta = rng.random((n, heads)).astype(np.float32)
    S = (rng.standard_normal((heads, dk, dv)) * 0.05).astype(np.float32)
    return qkv, decay, beta, S


def closed_form(S, qkv, decay, beta, n, heads, rep, dk, dv):
    kd = heads // rep * dk
    S = S.astype(np.float64).copy()
    o = np.zeros((n, heads * dv))
    for t in range(n):
        for h in range(heads):
            kh = h // rep
            q = qkv[t, kh * dk:(kh + 1) * dk].astype(np.float64)
            k = qkv[t, kd + kh * dk:kd + (kh + 1) * dk].astype(np.float64)
            v = qkv[t, 2 * kd + h * dv:2 * kd + (h + 1) * dv].astype(np.float64)
            a, b = float(decay[t, h]), float(beta[t, h])
            St = S[h].T                                    # [dv][dk]
            St = a * St @ (np.eye(dk) - b * np.outer(k, k)) + b * np.outer(v, k)
            S[h] = St.T
            o[t, h * dv:(h + 1) * dv] = St @ q
    return S, o


@pytest.mark.parametrize("heads,rep,dk,dv,n", [(4, 2, 32, 64, 3), (16, 1, 128, 128, 5)])
def test_lin_closed_form(heads, rep, dk, dv, n):
    rng = np.random.default_rng(heads + n)
    qkv, decay, beta, S = inputs(rng, n, heads, rep, dk, dv)
    S1, o, _ = oracle.lin_rule(qkv, decay, beta, S, n=n, heads=heads, rep=rep, dk=dk, dv=dv)
    Sx, ox = closed_form(S, qkv, decay, beta, n, heads, rep, dk, dv)
    assert np.abs(S1 - Sx).max() <= 1e-5 * np.abs(Sx).max()
    assert np.abs(o - ox).max() <= 1e-5 * np.abs(ox).max()
    # planted mistake: q and k swapped in the input layout
    kd = heads // rep * dk
    bad = qkv.copy()
    bad[:, :kd], bad[:, kd:2 * kd] = qkv[:, kd:2 * kd], qkv[:, :kd]
    _, ob, _ = oracle.lin_rule(bad, decay, beta, S, n=n, heads=heads, rep=rep, dk=dk, dv=dv)
    assert np.abs(ob - ox).max() > 1e-3 * np.abs(ox).max()


@pytest.mark.parametrize("n", [1, 3, 5])
def test_lin_replay_equals_direct(n):
    heads, rep, dk, dv = 4, 1, 64, 64
    rng = np.random.default_rng(10 + n)
    qkv, decay, beta, S = inputs(rng, n, heads, rep, dk, dv)
    S0, o0, lg = oracle.lin_rule(qkv, decay, beta, S, n=n, heads=heads, rep=rep, dk=dk, dv=dv,
                                 log=True, log0=True)
    assert np.array_equal(S0, S)
    for L in range(n + 1):
        direct = S if L == 0 else oracle.lin_rule(qkv[:L], decay[:L], beta[:L], S, n=L,
                                                  heads=heads, rep=rep, dk=dk, dv=dv)[0]
        replay = oracle.lin_apply(S, lg, L, heads, dk, dv)
        assert np.array_equal(replay.view(np.uint32), direct.view(np.uint32)), L
    # reference mode: token 0 in place, rows >= 1 logged, same outputs
    S1, o1, lg1 = oracle.lin_rule(qkv, decay, beta, S, n=n, heads=heads, rep=rep, dk=dk, dv=dv,
                                  log=True)
    assert np.array_equal(o1, o0) and np.array_equal(lg1[1:], lg[1:])
    assert np.array_equal(S1, oracle.lin_apply(S, lg, 1, heads, dk, dv))


ref = oracle.ref_lib()
needs_ref = pytest.mark.skipif(ref is None, reason="oracle/_ref not built (reference absent)")


def ref_rule(S, qkv, decay, beta, n, heads, rep, dk, dv, log=False, pend=None, keep=0):
    S = S.copy()
    o = np.zeros((n, heads * dv), np.float32)
    lg = np.zeros((n, heads, dk + dv + 1), np.float32) if log else None
    work = np.zeros(dk * dv, np.float32)
    p = lambda a: None if a is None else a.ctypes.data
    args = oracle.RefLinArgs(n, heads, rep, dk, dv, qkv.shape[1], heads * dv, p(qkv), p(decay),
                             p(beta), p(S), p(o), p(lg), p(pend), keep, p(work))
    ref.pf_lin_rule(None, ctypes.byref(args))
    return S, o, lg


@needs_ref
@pytest.mark.parametrize("heads,rep,dk,dv,n", [(4, 2, 32, 64, 1), (4, 2, 32, 64, 7),
                                               (16, 1, 128, 128, 5), (2, 1, 256, 512, 3)])
def test_lin_bit_exact_vs_reference_build(heads, rep, dk, dv, n):
    """The oracle == engine/src/matvec_ref.c (built from the reference's own sources) for a
    plain pass, a logged pass, and a logged pass with 3 pending updates."""
    rng = np.random.default_rng(20 + n + dk)
    qkv, decay, beta, S = inputs(rng, n, heads, rep, dk, dv)
    keep = 3
    pend = (rng.standard_normal((keep, heads, dk + dv + 1)) * 0.1).astype(np.float32)
    pend[:, :, dk + dv] = 0.9375
    for logged, kp in ((False, 0), (True, 0), (True, keep), (False, keep)):
        pp = pend if kp else None
        a = oracle.lin_rule(qkv, decay, beta, S, n=n, heads=heads, rep=rep, dk=dk, dv=dv,
                            log=logged, pend=pp, keep=kp)
        b = ref_rule(S, qkv, decay, beta, n, heads, rep, dk, dv, log=logged, pend=pp, keep=kp)
        assert np.array_equal(a[0].view(np.uint32), b[0].view(np.uint32)), "state"
        assert np.array_equal(a[1].view(np.uint32), b[1].view(np.uint32)), "outputs"
        if logged and n > 1:
            assert np.array_equal(a[2][1:], b[2][1:]), "log"
    Sr = S.copy()
    ref.pf_lin_apply(None, Sr.ctypes.data, pend.ctypes.data, keep, heads, dk, dv)
    assert np.array_equal(oracle.lin_apply(S, pend, keep, heads, dk, dv), Sr)
