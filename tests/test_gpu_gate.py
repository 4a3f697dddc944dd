"""GPU parity: the device form of the reference's chain gate (libnmx.so nmx_top1_gate: the
top-1 softmax probability of a draft row, the reference's top1_prob, engine/src/spec.c:89-92,
compared with CONF_TAU as in engine/src/spec_adapt.c:56) against the oracle's. The engine's own
adaptive policy does not gate chains; the device ABI keeps the gate for callers of the
reference's policy.

Bar: the flag equals (oracle top1_prob(row) >= tau) for every row. The rows include ones whose
probability lies within the kernel's double-precision error band around tau, where the decision
is taken from the exact ordered float32 sum, and ones past a segment (4096 exponentials) of it.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

TAU = np.float32(0.6)


def rows_for(n, rng):
    rows = [rng.normal(0, 3, n), rng.normal(0, 0.05, n)]
    peaked = rng.normal(0, 1, n)
    peaked[rng.integers(n)] += 40.0
    rows.append(peaked)
    if n > 1:  # one logit 0, the others near x0 with (n - 1) exp(x0) = 1 / tau - 1
        x0 = np.float32(np.log((1.0 / float(TAU) - 1.0) / (n - 1)))
        ulp = np.spacing(x0)
        for j in range(-24, 25):
            r = np.full(n, x0 + j * ulp, np.float32)
            r += (rng.integers(-2, 3, n) * ulp).astype(np.float32)
            r[rng.integers(n)] = 0.0
            rows.append(r)
    return [np.asarray(r, np.float32) for r in rows]


def in_band(r):
    """Rows whose double-precision probability lies well inside the kernel's error band
    2 (n + 16) 2^-24 around tau, so the kernel decides them with the exact float32 sum."""
    s = np.exp(r.astype(np.float64) - r.max()).sum()
    return abs(1.0 / s - float(TAU)) < (r.size + 16) * 2.0 ** -24 * float(TAU)


@pytest.mark.parametrize("n", [1, 4, 7, 1000, 4100, 32768, 248320])
def test_gate_matches_oracle(dev, n):
    rng = np.random.default_rng(n)
    rows = rows_for(n, rng)
    print(f"[case] top1 gate n={n} rows={len(rows)}", flush=True)
    dl, flag = dev.empty((n,), np.float32), dev.zeros((1,), np.int32)
    want, got, band = [], [], 0
    for r in rows:
        dev.upload(dl, r)
        dev.top1_gate(dl, n, float(TAU), flag)
        got.append(int(dev.download(flag)[0]))
        want.append(int(oracle.top1_prob(r) >= TAU))
        band += in_band(r)
    dev.free(dl), dev.free(flag)
    assert got == want, [i for i, (a, b) in enumerate(zip(got, want)) if a != b]
    if n > 4:
        assert band > 0 and 0 < sum(want) < len(want), "no row near the threshold"


def test_gate_rejects_bad_arguments(dev):
    flag = dev.zeros((1,), np.int32)
    with pytest.raises(RuntimeError):
        dev.top1_gate(flag, 0, 0.6, flag)
    dev.free(flag)
