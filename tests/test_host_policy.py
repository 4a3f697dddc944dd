"""The engine's host-side drafting policies, built from their sources alone (no GPU, no
reference): the prompt-lookup drafter (nibblemac_amd/csrc/host/ngram.c) and the adaptive
width policy (adapt.c). Neither can change an emitted token (the GPU end-to-end tests check
speculative output == plain greedy with both on); what is pinned here is that each does what
its specification says.

Drafter: against a brute-force restatement of its rule over every earlier occurrence of the
history's last 2-gram (the continuation of the occurrence that agrees backwards with the tail
over the most tokens, capped at 32, the newest among equals), on random histories with planted
repeats, through pushes and pops (the lazily built index must answer like a fresh one).

Policy: in a simulated environment (round seconds T(w) = a + b w, each draft accepted with
probability p once reached) it settles on the width with the highest closed-form rate
E(w) / T(w), E(w) = sum_{s < w} p^s, and it re-measures the stalest width every 32 rounds.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
HOST = ROOT / "nibblemac_amd" / "csrc" / "host"
MAX_K = 8


@pytest.fixture(scope="module")
def lib(tmp_path_factory):
    out = tmp_path_factory.mktemp("hostpol") / "libhostpol.so"
    subprocess.run(["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-Wall", "-Werror",
                    f"-I{ROOT / 'include'}", f"-I{HOST}", str(HOST / "ngram.c"),
                    str(HOST / "adapt.c"), "-o", str(out)], check=True)
    L = ctypes.CDLL(str(out))
    vp, i, d = ctypes.c_void_p, ctypes.c_int, ctypes.c_double
    for name, res, args in [("e_ngram_init", i, [vp, i]), ("e_ngram_free", None, [vp]),
                            ("e_ngram_reset", None, [vp]), ("e_ngram_push", None, [vp, vp, i]),
                            ("e_ngram_pop", None, [vp]), ("e_ngram_draft", i, [vp, vp, i, vp]),
                            ("e_adapt_init", None, [vp, i]), ("e_adapt_width", i, [vp]),
                            ("e_adapt_observe", None, [vp, i, i, d])]:
        f = getattr(L, name)
        f.restype, f.argtypes = res, args
    return L


class Drafter:
    def __init__(self, L, cap):
        self.L, self.g = L, ctypes.create_string_buffer(256)
        assert L.e_ngram_init(self.g, cap) == 0

    def push(self, toks):
        a = np.ascontiguousarray(toks, np.int32)
        self.L.e_ngram_push(self.g, a.ctypes.data, a.size)

    def pop(self):
        self.L.e_ngram_pop(self.g)

    def draft(self, mx):
        out, m = np.zeros(64, np.int32), ctypes.c_int(-1)
        n = self.L.e_ngram_draft(self.g, out.ctypes.data, mx, ctypes.byref(m))
        return list(out[:n]), m.value

    def close(self):
        self.L.e_ngram_free(self.g)


def brute_draft(h, mx, ext=32):
    """The drafter's rule over every earlier occurrence (histories here hold fewer than the
    64 candidates one lookup examines)."""
    n = len(h)
    if n < 3 or mx <= 0:
        return [], 0
    best_q, best = -1, 0
    for q in range(n - 2, 0, -1):  # newest first; an occurrence is followed by a token
        ln = 0
        while ln < ext and q - ln >= 0 and h[q - ln] == h[n - 1 - ln]:
            ln += 1
        if ln > best:
            best, best_q = ln, q
            if ln == ext:
                break
    if best < 2:
        return [], 0
    return list(h[best_q + 1: best_q + 1 + min(mx, n - 1 - best_q)]), best


def history(rng, n, vocab):
    h = list(rng.integers(0, vocab, n))
    for _ in range(rng.integers(1, 4)):  # planted repeats of earlier spans
        ln = int(rng.integers(2, 40))
        s = int(rng.integers(0, max(1, len(h) - ln)))
        at = int(rng.integers(0, len(h)))
        h[at:at] = h[s:s + ln]
    return h


@pytest.mark.parametrize("seed", range(12))
def test_drafter_matches_brute_force(lib, seed):
    rng = np.random.default_rng(seed)
    vocab = [3, 7, 50, 5000][seed % 4]  # small vocabularies: many candidates, long agreements
    h = history(rng, int(rng.integers(10, 60)), vocab)
    if vocab <= 7:
        h = h[:40]  # keep the occurrence count under the 64 candidates of one lookup
    d = Drafter(lib, 512)
    d.push(h[:5])
    for t in range(5, len(h) + 1):
        for mx in (1, 4, 8):
            assert d.draft(mx) == brute_draft(h[:t], mx), (t, mx)
        if t < len(h):
            d.push(h[t:t + 1])
    d.close()


def test_drafter_pop_equals_fresh_index(lib):
    rng = np.random.default_rng(40)
    h = history(rng, 50, 20)
    d = Drafter(lib, 512)
    d.push(h)
    d.draft(8)  # index everything
    for _ in range(6):  # drop tokens the index holds, then lookups must not see them
        h.pop()
        d.pop()
        assert d.draft(8) == brute_draft(h, 8)
    d.push([h[3], h[4], 9999])
    h += [h[3], h[4], 9999]
    assert d.draft(8) == brute_draft(h, 8)
    d.close()


def test_drafter_edges(lib):
    d = Drafter(lib, 8)
    assert d.draft(4) == ([], 0)                      # empty
    d.push([1, 2])
    assert d.draft(4) == ([], 0)                      # too short
    d.push([1, 2])
    assert d.draft(4) == ([1, 2], 2)                  # "1 2" before, followed by "1 2"
    assert d.draft(0) == ([], 0)
    d.push([5, 6, 7, 8, 9])                           # past the capacity: the history stops
    assert d.draft(4) == brute_draft([1, 2, 1, 2, 5, 6, 7, 8], 4)
    d.L.e_ngram_reset(d.g)
    assert d.draft(4) == ([], 0)
    d.close()


class Policy:
    def __init__(self, L, k):
        self.L, self.a = L, ctypes.create_string_buffer(1024)
        L.e_adapt_init(self.a, k)

    def width(self):
        return self.L.e_adapt_width(self.a)

    def observe(self, w, acc, sec):
        self.L.e_adapt_observe(self.a, w, acc, sec)


def simulate(lib, k, p, a, b, rounds, seed=0):
    rng = np.random.default_rng(seed)
    pol, widths = Policy(lib, k), []
    for _ in range(rounds):
        w = pol.width()
        assert 1 <= w <= k + 1
        acc = 0
        while acc < w - 1 and rng.random() < p:
            acc += 1
        pol.observe(w, acc, (a + b * w) * (1 + 0.02 * rng.standard_normal()))
        widths.append(w)
    return widths


def best_width(k, p, a, b):
    rate = [sum(p ** s for s in range(w)) / (a + b * w) for w in range(1, k + 2)]
    return int(np.argmax(rate)) + 1


@pytest.mark.parametrize("k,p,a,b", [(4, 0.0, 1.0, 0.05), (4, 0.95, 1.0, 0.05), (4, 0.7, 1.0, 0.3),
                                     (8, 0.8, 1.0, 0.02), (2, 0.5, 1.0, 0.6), (4, 0.3, 0.2, 1.0)])
def test_policy_settles_on_the_best_width(lib, k, p, a, b):
    widths = simulate(lib, k, p, a, b, 600, seed=int(100 * p) + k)
    tail = widths[300:]
    want = best_width(k, p, a, b)
    top = max(set(tail), key=tail.count)
    assert top == want, (want, {w: tail.count(w) for w in set(tail)})
    assert tail.count(want) >= 0.8 * len(tail)


def test_policy_first_rounds_and_probes(lib):
    pol = Policy(lib, 4)
    assert pol.width() == 5  # nothing measured: the full width first
    pol.observe(5, 0, 1.0)
    assert pol.width() == 1  # an unmeasured plain step is costed below everything: tried once
    pol.observe(1, 0, 0.5)
    seen = []
    for _ in range(200):
        w = pol.width()
        seen.append(w)
        pol.observe(w, 0, {1: 0.5}.get(w, 1.0))
    # drafts never accepted and plain steps cheaper: plain steps, with every width re-measured
    # by the probes every 32 rounds
    assert seen.count(1) > 150 and set(seen) == {1, 2, 3, 4, 5}


def test_policy_width_bounds(lib):
    pol = Policy(lib, 0)
    assert pol.width() == 1
    pol.observe(3, 0, 1.0)  # out of range: ignored
    assert pol.width() == 1
