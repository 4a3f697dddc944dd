"""GPU parity of the fused Gated DeltaNet mixer (nmx_lin_mix) against the three kernels it
replaces (nmx_lin_pre + nmx_lin_rule + nmx_lin_post), which are themselves checked against the
oracle (test_gpu_lin.py) and, through the reference engine, end to end (test_gpu_e2e.py).

Bar: bit-exact for every output and every piece of state the mixer leaves behind: the A8 of
the gated-normed output and its float rows, the recurrent state, the conv state, the logged
raw inputs (xin) and the rollback log rows. Cases: verify passes (logged) of 1..8 tokens with
and without pending replays, the reference-mode and extension logs, plain passes up to a
64-token prefill chunk, dk = dv = 64 and 128, and shared key heads (rep = 2, which runs the
three kernels inside nmx_lin_mix).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from nibblemac_amd.nmx import A8, LinArgs, LinMixArgs, LinPreArgs
from tests.refmath import state_from_dev
from tests.test_gpu_q4k import assert_bits_equal

pytestmark = pytest.mark.gpu


def p(b):
    return None if b is None else b.ptr


def make_case(dev, rng, n, heads, rep, dk, dv, K=4, logged=True, keep=0, log0=False):
    kh = heads // rep
    kd = kh * dk
    C = 2 * kd + heads * dv
    cap = max(9, keep + 1)
    host = dict(
        raw=rng.standard_normal((n, C)).astype(np.float32),
        z=rng.standard_normal((n, heads * dv)).astype(np.float32),
        b=rng.standard_normal((n, heads)).astype(np.float32),
        a=rng.standard_normal((n, heads)).astype(np.float32) * 2,
        A_log=rng.uniform(np.log(0.2), np.log(0.4), heads).astype(np.float32),
        dt_bias=rng.uniform(-4.5, -3.5, heads).astype(np.float32),
        conv_w=rng.uniform(-0.5, 0.5, (C, K)).astype(np.float32),
        state=rng.standard_normal((K - 1, C)).astype(np.float32),
        S=(rng.standard_normal((heads, dv, dk)) * 0.05).astype(np.float32),
        pend=(rng.standard_normal((cap, heads, dk + dv + 1)) * 0.1).astype(np.float32),
        norm_w=rng.uniform(0.5, 1.5, dv).astype(np.float32),
    )
    host["pend"][:, :, dk + dv] = rng.uniform(0.9, 1.0, (cap, heads))
    return dict(n=n, heads=heads, rep=rep, dk=dk, dv=dv, K=K, kd=kd, C=C, cap=cap, logged=logged,
                keep=keep, log0=log0, host=host)


def run(dev, case, fused):
    h = case["host"]
    n, heads, dk, dv, C, cap = case["n"], case["heads"], case["dk"], case["dv"], case["C"], case["cap"]
    d = {k: dev.to_device(v) for k, v in h.items()}
    conv = dev.zeros((n, C), np.float32)
    beta = dev.zeros((n, heads), np.float32)
    decay = dev.zeros((n, heads), np.float32)
    o = dev.zeros((n, heads * dv), np.float32)
    xin = dev.zeros((cap, C), np.float32) if case["logged"] else None
    log = dev.zeros((cap, heads, dk + dv + 1), np.float32) if case["logged"] else None
    y = dev.zeros((n, heads * dv), np.float32)
    nb = heads * dv // 32
    aq, ad, afs = (dev.zeros((nb, n, 32), np.int8), dev.zeros((nb, n), np.float32),
                   dev.zeros((nb, n), np.float32))
    pre = LinPreArgs(n, C, case["K"], dk, case["kd"], p(d["raw"]), C, p(conv), p(d["state"]),
                     p(d["conv_w"]), p(xin), np.float32(1.0 / np.sqrt(dk)), 1e-6, p(d["b"]),
                     p(d["a"]), heads, heads, p(d["A_log"]), None, p(d["dt_bias"]), p(beta),
                     p(decay))
    rule = LinArgs(n, heads, case["rep"], dk, dv, C, heads * dv, p(conv), p(decay), p(beta),
                   p(d["S"]), p(o), p(log), p(d["pend"]), case["keep"], int(case["log0"]), None)
    if fused:
        dev.lin_mix(LinMixArgs(pre, rule, p(d["z"]), heads * dv, p(d["norm_w"]), 1e-6, p(y),
                               heads * dv, A8(p(aq), p(ad), p(afs))))
    else:
        dev.lin_pre(pre)
        dev.lin_rule(n=n, heads=heads, rep=case["rep"], dk=dk, dv=dv, qkv_stride=C,
                     o_stride=heads * dv, qkv=conv, decay=decay, beta=beta, S=d["S"], o=o,
                     log=log, pend=d["pend"], keep=case["keep"], log0=case["log0"])
        dev.lin_post(o, heads * dv, d["z"], heads * dv, d["norm_w"], n, heads, dv, 1e-6, y,
                     heads * dv, (aq, ad, afs))
    dev.sync()
    out = dict(aq=aq.numpy(), ad=ad.numpy(), afs=afs.numpy(), y=y.numpy(), S=d["S"].numpy(),
               state=d["state"].numpy())
    if case["logged"]:
        out["xin"] = xin.numpy()[1:n]
        out["log"] = log.numpy()[(0 if case["log0"] else 1):n]
    return out


CASES = [
    # n, heads, rep, dk, dv, logged, keep, log0
    (5, 16, 1, 128, 128, True, 0, False),
    (5, 16, 1, 128, 128, True, 3, False),
    (1, 16, 1, 128, 128, True, 0, False),
    (8, 4, 1, 128, 128, True, 7, False),
    (5, 4, 1, 128, 128, True, 12, False),  # two batches of pending rows
    (5, 4, 1, 128, 128, True, 2, True),
    (1, 4, 1, 128, 128, False, 0, False),
    (13, 4, 1, 128, 128, False, 4, False),
    (64, 4, 1, 128, 128, False, 0, False),
    (5, 4, 1, 64, 64, True, 1, False),
    (33, 4, 1, 64, 64, False, 0, False),
    (5, 4, 2, 64, 64, True, 2, False),   # shared key heads: the three-kernel path
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "n%d_h%d_rep%d_dk%d_%s_keep%d%s" % (
    c[0], c[1], c[2], c[3], "logged" if c[5] else "plain", c[6], "_log0" if c[7] else ""))
def test_lin_mix_equals_three_kernels(dev, case):
    n, heads, rep, dk, dv, logged, keep, log0 = case
    print(f"[case] lin_mix {case}", flush=True)
    rng = np.random.default_rng(n * 131 + heads + dk + keep)
    c = make_case(dev, rng, n, heads, rep, dk, dv, logged=logged, keep=keep, log0=log0)
    want = run(dev, c, fused=False)
    got = run(dev, c, fused=True)
    for k in want:
        assert_bits_equal(got[k], want[k], k)


def from_dev(S, heads, dk, dv):
    """the device layout (include/nmx.h, nmx_state_index) -> oracle [h][dk][dv]"""
    return state_from_dev(S, heads, dk, dv)


@pytest.mark.parametrize("e", [1, 2, 3, 4, 5])
def test_lin_mix_commit_replay_against_oracle(dev, e):
    """Config 3 through the round's own kernels (lin_mix_k, commit_k, lin_mix_k again), each
    result against the oracle (engine/src/matvec_ref.c:114-188 restated) on the same inputs:
    16 heads, dk = dv = 128, a logged verify pass of 5 tokens; the commit of e = 1..5 tokens
    (an accepted prefix of e - 1 drafts: the conv state from the kept rows, e - 1 pending rows,
    keep = e - 1 in the control block); then the next logged pass, which replays the pending
    rows (keep read on the device) before its own tokens. Checked bit for bit: the state after
    token 0 and the log rows of each pass against oracle.lin_rule over the mixer's own q / k /
    v / gates (nmx_lin_pre on the same inputs), the committed conv state against the last
    rows of [state, raw inputs of the e tokens], and the state after the second pass against
    the oracle's direct run of the e tokens followed by the second pass's token 0."""
    from nibblemac_amd.nmx import CommitArgs

    print(f"[case] lin_mix commit replay e={e}", flush=True)
    heads, rep, dk, dv, n, K = 16, 1, 128, 128, 5, 4
    rng = np.random.default_rng(700 + e)
    A = make_case(dev, rng, n, heads, rep, dk, dv, K=K, logged=True, keep=0)
    B = make_case(dev, rng, n, heads, rep, dk, dv, K=K, logged=True, keep=0)
    hA, hB = A["host"], B["host"]
    C, cap, row = A["C"], A["cap"], heads * (dk + dv + 1)
    kw = dict(heads=heads, rep=rep, dk=dk, dv=dv)

    def pre_outputs(h, state):
        """the mixer's rule inputs: nmx_lin_pre on raw inputs and the conv state `state`"""
        d = {k: dev.to_device(v) for k, v in h.items()}
        dev.upload(d["state"], state)
        conv, beta, decay = (dev.zeros((n, C), np.float32), dev.zeros((n, heads), np.float32),
                             dev.zeros((n, heads), np.float32))
        pre = LinPreArgs(n, C, K, dk, A["kd"], p(d["raw"]), C, p(conv), p(d["state"]),
                         p(d["conv_w"]), None, np.float32(1.0 / np.sqrt(dk)), 1e-6, p(d["b"]),
                         p(d["a"]), heads, heads, p(d["A_log"]), None, p(d["dt_bias"]), p(beta),
                         p(decay))
        dev.lin_pre(pre)
        dev.sync()
        out = conv.numpy(), decay.numpy(), beta.numpy()
        for b in list(d.values()) + [conv, beta, decay]:
            b.free()
        return out

    # device state shared by the two passes and the commit
    S = dev.to_device(hA["S"])
    conv_state = dev.to_device(hA["state"])
    xin = dev.zeros((cap, C), np.float32)
    log = dev.zeros((cap, heads, dk + dv + 1), np.float32)
    pend = dev.zeros((cap, heads, dk + dv + 1), np.float32)
    ctl = dev.to_device(np.zeros(16, np.int32))
    y = dev.zeros((n, heads * dv), np.float32)
    nb = heads * dv // 32
    aq, ad, afs = (dev.zeros((nb, n, 32), np.int8), dev.zeros((nb, n), np.float32),
                   dev.zeros((nb, n), np.float32))
    o = dev.zeros((n, heads * dv), np.float32)

    def mix(h, keep_dev):
        d = {k: dev.to_device(h[k]) for k in ("raw", "z", "b", "a", "A_log", "dt_bias", "conv_w",
                                              "norm_w")}
        pre = LinPreArgs(n, C, K, dk, A["kd"], p(d["raw"]), C, None, p(conv_state),
                         p(d["conv_w"]), p(xin), np.float32(1.0 / np.sqrt(dk)), 1e-6, p(d["b"]),
                         p(d["a"]), heads, heads, p(d["A_log"]), None, p(d["dt_bias"]), None,
                         None)
        rule = LinArgs(n, heads, rep, dk, dv, C, heads * dv, None, None, None, p(S), p(o),
                       p(log), p(pend), cap if keep_dev else 0, 0, keep_dev)
        dev.lin_mix(LinMixArgs(pre, rule, p(d["z"]), heads * dv, p(d["norm_w"]), 1e-6, p(y),
                               heads * dv, A8(p(aq), p(ad), p(afs))))
        dev.sync()
        for b in d.values():
            b.free()

    try:
        # pass A: logged, nothing pending
        qkvA, decA, betA = pre_outputs(hA, hA["state"])
        mix(hA, None)
        S0 = from_dev(hA["S"], heads, dk, dv)
        S1, _, lgA = oracle.lin_rule(qkvA, decA, betA, S0, n=n, log=True, **kw)
        assert_bits_equal(from_dev(S.numpy(), heads, dk, dv), S1,
                          "state after token 0 of pass A")
        assert_bits_equal(log.numpy()[1:n], lgA[1:n], "log rows 1..4 of pass A")
        # the commit of e tokens
        dev.upload(ctl, np.array([0, e] + [0] * 14, np.int32))
        dev.lin_commit(CommitArgs(1, C, K, conv_state.ptr, xin.ptr, log.ptr, pend.ptr, cap, row,
                                  ctl.ptr, None, None, 0))
        dev.sync()
        want_conv = np.concatenate([hA["state"], hA["raw"][:e]])[-(K - 1):]
        assert_bits_equal(conv_state.numpy(), want_conv, "conv state after the commit")
        assert int(ctl.numpy()[2]) == e - 1
        assert_bits_equal(pend.numpy()[:e - 1], lgA[1:e], "pending rows")
        # pass B: replays the e - 1 pending rows (keep from the control block), then logs
        qkvB, decB, betB = pre_outputs(hB, want_conv)
        mix(hB, ctl.ptr + 8)
        Se = oracle.lin_rule(qkvA[:e], decA[:e], betA[:e], S0, n=e, **kw)[0]
        S2, _, lgB = oracle.lin_rule(qkvB, decB, betB, Se, n=n, log=True, **kw)
        assert_bits_equal(from_dev(S.numpy(), heads, dk, dv), S2, "state after pass B token 0")
        assert_bits_equal(log.numpy()[1:n], lgB[1:n], "log rows 1..4 of pass B")
    finally:
        for b in (S, conv_state, xin, log, pend, ctl, y, aq, ad, afs, o):
            b.free()
