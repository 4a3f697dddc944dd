"""GPU end-to-end parity of the MI355X engine (libpinfer.so) against the reference engine's
own sources running Q4K models on the CPU (oracle/_ref/libpinfer_refq4k.so: the reference's
forward pass, attention, DeltaNet mixer + rollback log, MTP head and speculative loop, with the
oracle's restated Q4K / A8 / DeltaNet operators).

Bar: last-token logits bit-exact after prefill and after continuation; generated tokens and
speculative statistics (rounds, drafted, accepted) identical; speculative output equal to plain
greedy output for every k; the state after a generation equal (checked through the logits of a
further eval). Models are synthetic (random-init, seeded): a small model with the 0.8B layer
pattern, a tiny-vocabulary one so that drafts get accepted (multi-token commits and deferred
replays), and the 0.8B shape itself.
"""
from __future__ import annotations

import os
from dataclasses import replace

import numpy as np
import pytest

from nibblemac_amd import pqfile
from nibblemac_amd.pinfer import Model
from nibblemac_amd.synth import QWEN35_08B
from oracle import HERE as ORACLE_DIR

pytestmark = pytest.mark.gpu

REF = ORACLE_DIR / "_ref" / "libpinfer_refq4k.so"
needs_ref = pytest.mark.skipif(not REF.exists(), reason="oracle/_ref not built (reference absent "
                               "when the tree was built)")

TINY = replace(pqfile.SMALL, vocab=8, eos_id=7)


@pytest.fixture(scope="module")
def models(tmp_path_factory):
    d = tmp_path_factory.mktemp("pq")
    return {"small": pqfile.write_model(d / "small.pq", pqfile.SMALL, seed=3, random_norms=True),
            "tiny": pqfile.write_model(d / "tiny.pq", TINY, seed=4, random_norms=True)}


def pair(path, max_ctx=512):
    from nibblemac_amd.pinfer import load_library

    ref_lib = load_library(str(REF))
    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    return (Model(str(path), max_ctx=max_ctx),
            Model(str(path), max_ctx=max_ctx, lib=ref_lib, n_threads=threads))


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@needs_ref
def test_eval_logits_bit_exact(models):
    gpu, ref = pair(models["small"])
    rng = np.random.default_rng(0)
    prompt = rng.integers(0, pqfile.SMALL.vocab, 70)   # two prefill chunks (64 + 6)
    print("[case] small eval 70 tokens", flush=True)
    a, b = gpu.eval(prompt), ref.eval(prompt)
    assert np.array_equal(bits(a), bits(b)), f"max diff {np.abs(a - b).max()}"
    more = rng.integers(0, pqfile.SMALL.vocab, 5)
    a, b = gpu.eval(more), ref.eval(more)
    assert np.array_equal(bits(a), bits(b)), "continuation"
    for tok in more[:3]:                                 # single-token steps
        a, b = gpu.eval([tok]), ref.eval([tok])
        assert np.array_equal(bits(a), bits(b)), "single-token step"
    assert gpu.n_past == ref.n_past == 78
    gpu.close(), ref.close()


@needs_ref
@pytest.mark.parametrize("k", [0, 1, 2, 4, 8])
def test_generate_matches_reference(models, k):
    gpu, ref = pair(models["small"])
    prompt = np.random.default_rng(1).integers(0, pqfile.SMALL.vocab, 40)
    print(f"[case] small generate k={k}", flush=True)
    tg, sg = gpu.generate(prompt, 32, k=k, draft_vocab=1024)
    tr, sr = ref.generate(prompt, 32, k=k, draft_vocab=1024)
    assert tg == tr
    assert (sg.rounds, sg.drafted, sg.accepted) == (sr.rounds, sr.drafted, sr.accepted)
    plain, _ = gpu.generate(prompt, 32, k=0)
    assert tg == plain, "speculative output differs from plain greedy"
    probe = [5, 6]
    assert np.array_equal(bits(gpu.eval(probe)), bits(ref.eval(probe))), "state after generation"
    gpu.close(), ref.close()


@needs_ref
@pytest.mark.parametrize("k", [2, 4])
def test_accepting_drafts_tiny_vocab(models, k):
    """vocab 8: drafts are accepted often, so multi-token commits, deferred replays and the MTP
    pass over several committed rows all run; EOS (id 7) may stop a round early."""
    gpu, ref = pair(models["tiny"])
    prompt = np.random.default_rng(2).integers(0, 7, 24)
    print(f"[case] tiny generate k={k}", flush=True)
    tg, sg = gpu.generate(prompt, 96, k=k)
    tr, sr = ref.generate(prompt, 96, k=k)
    assert tg == tr
    assert (sg.rounds, sg.drafted, sg.accepted) == (sr.rounds, sr.drafted, sr.accepted)
    assert gpu.generate(prompt, 96, k=0)[0] == tg
    probe = [1, 2, 3]
    assert np.array_equal(bits(gpu.eval(probe)), bits(ref.eval(probe)))
    gpu.close(), ref.close()


@needs_ref
def test_generate_continuation_and_stop_ids(models):
    gpu, ref = pair(models["small"])
    prompt = np.random.default_rng(3).integers(0, pqfile.SMALL.vocab, 20)
    tg, _ = gpu.generate(prompt, 12, k=4, draft_vocab=1024)
    tr, _ = ref.generate(prompt, 12, k=4, draft_vocab=1024)
    assert tg == tr
    cg, _ = gpu.generate([tg[-1]] + [7, 8], 10, k=4, draft_vocab=1024, cont=True)
    cr, _ = ref.generate([tr[-1]] + [7, 8], 10, k=4, draft_vocab=1024, cont=True)
    assert cg == cr and gpu.n_past == ref.n_past
    stop = [tg[5]]
    sg_, _ = gpu.generate(prompt, 30, k=4, draft_vocab=1024, stop_ids=stop)
    sr_, _ = ref.generate(prompt, 30, k=4, draft_vocab=1024, stop_ids=stop)
    assert sg_ == sr_ and sg_[-1] == stop[0]
    gpu.close(), ref.close()


@needs_ref
def test_qwen35_08b_shape(tmp_path):
    """The 0.8B shape itself (24 layers, vocab 248320, tied Q4K head, MTP): prefill logits
    bit-exact, then the benchmark sequence (prefill, k = 4 decode with EOS ignored) generating
    the same tokens and statistics as the reference engine."""
    path = pqfile.write_model(tmp_path / "q08.pq", QWEN35_08B, seed=1)
    gpu, ref = pair(path, max_ctx=256)
    prompt = np.random.default_rng(8).integers(0, QWEN35_08B.vocab, 12)
    print("[case] 0.8B shape eval 12 tokens", flush=True)
    a, b = gpu.eval(prompt), ref.eval(prompt)
    assert np.array_equal(bits(a), bits(b)), f"max diff {np.abs(a - b).max()}"
    print("[case] 0.8B shape generate 9 tokens k=4", flush=True)
    tg, sg = gpu.generate(prompt, 9, k=4, draft_vocab=32768)
    tr, sr = ref.generate(prompt, 9, k=4, draft_vocab=32768)
    assert tg == tr
    assert (sg.rounds, sg.drafted, sg.accepted) == (sr.rounds, sr.drafted, sr.accepted)
    toks, st, tp, td = gpu.bench_generate(prompt, 9, k=4, draft_vocab=32768)
    assert toks[:len(tg)] == tg and tp > 0 and td > 0
    gpu.close(), ref.close()


def test_invalid_arguments(models):
    gpu = Model(str(models["small"]), max_ctx=64)
    from nibblemac_amd.pinfer import PinferError
    with pytest.raises(PinferError):
        gpu.eval([pqfile.SMALL.vocab])            # token id out of range
    with pytest.raises(PinferError):
        gpu.eval(np.zeros(65, np.int32))           # more than max_ctx
    assert gpu.n_past == 0
    gpu.close()
