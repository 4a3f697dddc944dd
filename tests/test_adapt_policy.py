"""The engine's adaptive speculation policy (nibblemac_amd/csrc/host/adapt.c, e_adapt_*, built
alone into oracle/_ref/libnmx_adapt.so) against the reference's own (engine/src/spec_adapt.c,
pf_adapt_* in oracle/_ref/libpinfer_ref.so): driven with the same random sequences of plain-step
times and speculative rounds (widths, emitted tokens, round and verify seconds), every decision
and the whole policy state agree after every call. CPU only."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle

W = 10  # PINFER_SPEC_MAX_K + 2 verify widths


class Adapt(ctypes.Structure):
    """pf_spec_adapt (engine/src/spec.h:49-57) = e_adapt (engine.h)."""

    _fields_ = [("tv", ctypes.c_double * W), ("t_plain", ctypes.c_double),
                ("r_tok", ctypes.c_double), ("r_sec", ctypes.c_double), ("n_spec", ctypes.c_int),
                ("plain_mode", ctypes.c_int), ("plain_run", ctypes.c_int),
                ("probe_after", ctypes.c_int), ("probing", ctypes.c_int)]


MINE = oracle.HERE / "_ref" / "libnmx_adapt.so"
pytestmark = pytest.mark.skipif(oracle.ref_lib() is None or not MINE.exists(),
                                reason="oracle/_ref not built (reference absent)")


def bind(lib, prefix):
    P = ctypes.POINTER(Adapt)
    f = {}
    for name, res, args in [("init", None, [P]), ("plain_now", ctypes.c_int, [P]),
                            ("plain", None, [P, ctypes.c_double]),
                            ("round", None, [P, ctypes.c_int, ctypes.c_int, ctypes.c_double,
                                             ctypes.c_double])]:
        fn = getattr(lib, prefix + name)
        fn.restype, fn.argtypes = res, args
        f[name] = fn
    return f


@pytest.mark.parametrize("seed,regime", [(1, "slow"), (2, "fast"), (3, "mixed"), (4, "cheap")])
def test_policy_matches_reference(seed, regime):
    ref = bind(oracle.ref_lib(), "pf_adapt_")
    mine = bind(ctypes.CDLL(str(MINE)), "e_adapt_")
    a, b = Adapt(), Adapt()
    ref["init"](ctypes.byref(a))
    mine["init"](ctypes.byref(b))
    rng = np.random.default_rng(seed)
    plain_t = {"slow": 0.01, "fast": 0.05, "mixed": 0.02, "cheap": 0.004}[regime]
    decisions = []
    for step in range(600):
        pa, pb = ref["plain_now"](ctypes.byref(a)), mine["plain_now"](ctypes.byref(b))
        assert pa == pb, step
        decisions.append(pa)
        if pa:
            sec = plain_t * rng.uniform(0.8, 1.2)
            ref["plain"](ctypes.byref(a), sec)
            mine["plain"](ctypes.byref(b), sec)
        else:
            n = int(rng.integers(1, W + 1))  # includes widths the policy ignores
            emitted = int(rng.integers(1, n + 1)) if regime != "slow" else 1
            tv = 0.01 * (1 + 0.1 * n) * rng.uniform(0.9, 1.1)
            sec = tv + (0.02 if regime == "slow" else 0.002) * rng.uniform(0.5, 1.5)
            if regime == "mixed" and step % 97 < 40:
                emitted = 1
            ref["round"](ctypes.byref(a), n, emitted, sec, tv)
            mine["round"](ctypes.byref(b), n, emitted, sec, tv)
        assert bytes(a) == bytes(b), f"state differs after call {step}"
    if regime == "slow":
        assert any(decisions), "the slow regime never took plain steps"
    if regime == "fast":
        assert not all(decisions)
