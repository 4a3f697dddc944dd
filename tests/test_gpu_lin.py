"""GPU parity: the Gated DeltaNet recurrence with rollback log and replay (libnmx.so) against
the oracle (a restatement of engine/src/matvec_ref.c:114-188).

Bar: bit-exact state, outputs and log (memcmp), which implies any tolerance (1e-5 after rollback).
Protocols follow the reference's own gates: engine/metal/check_graphs.c:92-148 (sequential
passes on one persistent state: plain, logged, logged with pending updates, restored, explicit
replay) and lbench --check's modes (engine/bench/lbench.c:131-210).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from nibblemac_amd.nmx import NmxError
from tests.refmath import state_from_dev, state_to_dev

pytestmark = pytest.mark.gpu


def to_dev_layout(S, heads, dk, dv):
    """oracle [h][dk][dv] -> the device layout (include/nmx.h, nmx_state_index)."""
    return state_to_dev(S, heads, dk, dv)


def from_dev_layout(S, heads, dk, dv):
    return state_from_dev(S, heads, dk, dv)


def bits_equal(a, b, what):
    a = np.ascontiguousarray(a, np.float32).view(np.uint32).ravel()
    b = np.ascontiguousarray(b, np.float32).view(np.uint32).ravel()
    bad = np.flatnonzero(a != b)
    assert bad.size == 0, f"{what}: {bad.size} mismatches, first at {bad[0]}"


def deltanet_16x128_inputs(rng, n=5, heads=16, dk=128, dv=128, rep=1, pad=0):
    """The 5-token recurrence workload: q, k ~ N(0,1) then L2-normalised per head; v ~ N(0,1);
    a_t = 0.9 + 0.1 sigmoid(N(0,1)) in (0.9, 1); b_t = sigmoid(N(0,1)) in (0, 1)."""
    kh = heads // rep
    kd = kh * dk
    stride = 2 * kd + heads * dv + pad
    qkv = np.zeros((n, stride), np.float32)
    qk = rng.standard_normal((n, 2, kh, dk)).astype(np.float32)
    qk /= np.linalg.norm(qk, axis=-1, keepdims=True).astype(np.float32)
    qkv[:, :kd] = qk[:, 0].reshape(n, kd)
    qkv[:, kd:2 * kd] = qk[:, 1].reshape(n, kd)
    qkv[:, 2 * kd:2 * kd + heads * dv] = rng.standard_normal((n, heads * dv))
    sig = lambda x: (1.0 / (1.0 + np.exp(-x))).astype(np.float32)
    decay = (0.9 + 0.1 * sig(rng.standard_normal((n, heads)))).astype(np.float32)
    beta = sig(rng.standard_normal((n, heads)))
    return qkv, decay, beta, stride


class Lin:
    """One persistent device state plus scratch, driven pass by pass."""

    def __init__(self, dev, heads, rep, dk, dv, nmax, S0):
        self.dev, self.heads, self.rep, self.dk, self.dv = dev, heads, rep, dk, dv
        self.S = dev.to_device(to_dev_layout(S0, heads, dk, dv))
        self.logw = dk + dv + 1
        self.log = dev.zeros((nmax, heads, self.logw), np.float32)
        self.o_stride = heads * dv + 4
        self.o = dev.zeros((nmax, self.o_stride), np.float32)

    def state(self):
        return from_dev_layout(self.S.numpy(), self.heads, self.dk, self.dv)

    def set_state(self, S):
        self.dev.upload(self.S, to_dev_layout(S, self.heads, self.dk, self.dv))

    def rule(self, qkv, decay, beta, *, logged=False, pend=None, keep=0, log0=False):
        n, stride = qkv.shape
        dq, dd, db = self.dev.to_device(qkv), self.dev.to_device(decay), self.dev.to_device(beta)
        dp = self.dev.to_device(pend) if pend is not None else None
        self.dev.lin_rule(n=n, heads=self.heads, rep=self.rep, dk=self.dk, dv=self.dv,
                          qkv_stride=stride, o_stride=self.o_stride, qkv=dq, decay=dd, beta=db,
                          S=self.S, o=self.o, log=self.log if logged else None, pend=dp,
                          keep=keep, log0=log0)
        self.dev.sync()
        o = self.o.numpy()[:n, :self.heads * self.dv]
        lg = self.log.numpy()[:n]
        for b in (dq, dd, db, dp):
            if b is not None:
                b.free()
        return o, lg


def oracle_rule(S, qkv, decay, beta, lin, **kw):
    n = qkv.shape[0]
    return oracle.lin_rule(qkv, decay, beta, S, n=n, heads=lin.heads, rep=lin.rep, dk=lin.dk,
                           dv=lin.dv, **kw)


def test_deltanet_16x128_plain_and_logged(dev):
    """16 heads x 128 x 128, 5 draft tokens: plain pass, then the reference-mode logged pass."""
    rng = np.random.default_rng(30)
    heads, dk, dv = 16, 128, 128
    S0 = (rng.standard_normal((heads, dk, dv)) * 0.02).astype(np.float32)
    lin = Lin(dev, heads, 1, dk, dv, 8, S0)
    qkv, decay, beta, _ = deltanet_16x128_inputs(rng)
    print("[case] deltanet 16x128 plain n=5", flush=True)
    o, _ = lin.rule(qkv, decay, beta)
    S1, o_ref, _ = oracle_rule(S0, qkv, decay, beta, lin)
    bits_equal(lin.state(), S1, "state after plain pass")
    bits_equal(o, o_ref, "outputs of plain pass")

    print("[case] deltanet 16x128 logged n=5", flush=True)
    qkv2, decay2, beta2, _ = deltanet_16x128_inputs(rng)
    o, lg = lin.rule(qkv2, decay2, beta2, logged=True)
    S2, o_ref, lg_ref = oracle_rule(S1, qkv2, decay2, beta2, lin, log=True)
    bits_equal(lin.state(), S2, "state after token 0 of the logged pass")
    bits_equal(o, o_ref, "outputs of logged pass")
    bits_equal(lg[1:], lg_ref[1:], "log rows 1..4")


@pytest.mark.parametrize("L", [0, 1, 2, 3, 4, 5])
def test_deltanet_16x128_rollback_replay(dev, L):
    """Log every draft step (log0 mode), roll back to an accepted prefix of length L (0..5) and
    replay: the state equals a direct run of exactly those L tokens, bit for bit."""
    rng = np.random.default_rng(300 + L)
    heads, dk, dv = 16, 128, 128
    S0 = (rng.standard_normal((heads, dk, dv)) * 0.02).astype(np.float32)
    lin = Lin(dev, heads, 1, dk, dv, 8, S0)
    qkv, decay, beta, _ = deltanet_16x128_inputs(rng)
    print(f"[case] deltanet 16x128 rollback L={L}", flush=True)
    o, lg = lin.rule(qkv, decay, beta, logged=True, log0=True)
    bits_equal(lin.state(), S0, "log0 pass leaves the state untouched")
    _, o_ref, lg_ref = oracle_rule(S0, qkv, decay, beta, lin, log=True, log0=True)
    bits_equal(o, o_ref, "outputs")
    bits_equal(lg, lg_ref, "log rows 0..4")
    dlog = dev.to_device(lg)
    dev.lin_apply(lin.S, dlog, L, heads, dk, dv)
    dev.sync()
    direct = S0 if L == 0 else oracle_rule(S0, qkv[:L], decay[:L], beta[:L], lin)[0]
    bits_equal(lin.state(), direct, f"state after replaying {L} of 5")
    dlog.free()


@pytest.mark.parametrize("heads,rep,dk,dv,n", [
    (4, 2, 32, 64, 1), (4, 2, 32, 64, 3), (4, 2, 32, 64, 7), (4, 2, 32, 64, 64),
    (16, 1, 128, 128, 1), (2, 1, 256, 512, 3), (16, 1, 64, 128, 5)])
def test_check_graphs_protocol(dev, heads, rep, dk, dv, n):
    """engine/metal/check_graphs.c:113-131: four sequential passes on one persistent state
    (plain; logged; logged with 3 pending updates; restored from a snapshot), then an explicit
    replay of the 3 pending rows. Every state, output and log is bit-identical to the oracle."""
    print(f"[case] check_graphs heads={heads} rep={rep} dk={dk} dv={dv} n={n}", flush=True)
    rng = np.random.default_rng(heads * 1000 + dk + dv + n)
    rf = lambda shape: ((rng.integers(0, 2001, shape) - 1000) / 16384.0).astype(np.float32)
    S = rf((heads, dk, dv))
    snapshot = S.copy()
    lin = Lin(dev, heads, rep, dk, dv, n, S)
    kd = heads // rep * dk
    stride = 2 * kd + heads * dv + 4
    qkv = rf((n, stride))
    decay = (0.875 + np.abs(rf((n, heads)))).astype(np.float32)
    beta = (0.5 + rf((n, heads))).astype(np.float32)
    keep = 3
    pend = rf((keep, heads, dk + dv + 1))
    pend[:, :, dk + dv] = 0.9375
    for p in range(4):
        logged, pending = p in (1, 2), keep if p == 2 else 0
        if p == 3:
            S = snapshot.copy()
            lin.set_state(S)
        o, lg = lin.rule(qkv, decay, beta, logged=logged, pend=pend if pending else None,
                         keep=pending)
        S, o_ref, lg_ref = oracle_rule(S, qkv, decay, beta, lin, log=logged,
                                       pend=pend if pending else None, keep=pending)
        bits_equal(lin.state(), S, f"pass {p} state")
        bits_equal(o, o_ref, f"pass {p} output")
        if logged and n > 1:
            bits_equal(lg[1:], lg_ref[1:], f"pass {p} log")
    dp = dev.to_device(pend)
    dev.lin_apply(lin.S, dp, keep, heads, dk, dv)
    dev.sync()
    bits_equal(lin.state(), oracle.lin_apply(S, pend, keep, heads, dk, dv), "explicit replay")


def test_lin_reference_mode_commit_matches_direct(dev):
    """The reference's commit: token 0 in place + e - 1 deferred rows replayed at the start of
    the next pass == running the e tokens directly, for e = 1..5."""
    rng = np.random.default_rng(31)
    heads, dk, dv = 16, 128, 128
    S0 = (rng.standard_normal((heads, dk, dv)) * 0.02).astype(np.float32)
    qkv, decay, beta, _ = deltanet_16x128_inputs(rng)
    for e in range(1, 6):
        lin = Lin(dev, heads, 1, dk, dv, 8, S0)
        _, lg = lin.rule(qkv, decay, beta, logged=True)
        if e > 1:
            dp = dev.to_device(lg[1:e])
            dev.lin_apply(lin.S, dp, e - 1, heads, dk, dv)
            dev.sync()
            dp.free()
        direct = oracle_rule(S0, qkv[:e], decay[:e], beta[:e], lin)[0]
        bits_equal(lin.state(), direct, f"commit e={e}")


def test_lin_invalid_calls_rejected(dev):
    S = dev.zeros((4, 64, 32), np.float32)
    with pytest.raises(NmxError):
        dev.lin_rule(n=1, heads=4, rep=3, dk=32, dv=64, qkv_stride=1000, o_stride=256, qkv=S,
                     decay=S, beta=S, S=S, o=S)
    with pytest.raises(NmxError):
        dev.lin_rule(n=65, heads=4, rep=2, dk=32, dv=64, qkv_stride=1000, o_stride=256, qkv=S,
                     decay=S, beta=S, S=S, o=S)
    with pytest.raises(NmxError):
        dev.lin_rule(n=1, heads=4, rep=2, dk=48, dv=64, qkv_stride=1000, o_stride=256, qkv=S,
                     decay=S, beta=S, S=S, o=S)
    with pytest.raises(NmxError):  # output aliases the state
        dev.lin_rule(n=1, heads=4, rep=2, dk=32, dv=64, qkv_stride=1000, o_stride=256, qkv=S,
                     decay=S, beta=S, S=S, o=S)
    with pytest.raises(NmxError):
        dev.lin_apply(S, None, 3, 4, 32, 64)
