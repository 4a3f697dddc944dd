"""GPU end-to-end parity of the MI355X engine (libpinfer.so) against the reference engine's
own sources running Q4K models on the CPU (oracle/_ref/libpinfer_refq4k.so: the reference's
forward pass, attention, DeltaNet mixer + rollback log, MTP head and speculative loop, with the
oracle's restated Q4K / A8 / DeltaNet operators).

Bar: last-token logits bit-exact after prefill and after continuation; generated tokens and
speculative statistics (rounds, drafted, accepted) identical; speculative output equal to plain
greedy output for every k; the state after a generation equal (checked through the logits of a
further eval). Models are synthetic (random-init, seeded): a small model with the 0.8B layer
pattern (its random MTP head's drafts are almost never accepted: single-token commits), the same
model with final norms that make drafts agree (the `agree_model` fixture: multi-token commits,
deferred DeltaNet replays of 1..k rows, stops inside a commit), and the 0.8B shape itself.
"""
from __future__ import annotations

import os

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

@pytest.fixture(scope="module")
def models(tmp_path_factory):
    d = tmp_path_factory.mktemp("pq")
    return {"small": pqfile.write_model(d / "small.pq", pqfile.SMALL, seed=3, random_norms=True)}


def pair(path, max_ctx=512, kv_dtype=0):
    from nibblemac_amd.pinfer import load_library

    ref_lib = load_library(str(REF))
    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    return (Model(str(path), max_ctx=max_ctx, kv_dtype=kv_dtype),
            Model(str(path), max_ctx=max_ctx, lib=ref_lib, n_threads=threads, kv_dtype=kv_dtype))


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
@pytest.mark.parametrize("k", [1, 2, 4, 8])
def test_accepting_drafts(agree_model, k):
    """Drafts accepted in many rounds: multi-token commits of the KV rows, deferred DeltaNet
    replays of up to k rows (pend / keep of the next pass) and the MTP pass over several
    committed rows all run; the state after the generation is compared byte for byte."""
    path, prompt = agree_model
    gpu, ref = pair(path)
    print(f"[case] agree generate k={k}", flush=True)
    tg, sg = gpu.generate(prompt, 64, k=k)
    tr, sr = ref.generate(prompt, 64, k=k)
    assert tg == tr
    assert (sg.rounds, sg.drafted, sg.accepted) == (sr.rounds, sr.drafted, sr.accepted)
    assert sg.accepted >= sg.drafted // 4, f"only {sg.accepted} of {sg.drafted} drafts accepted"
    if k > 1:
        assert sg.rounds < 64 - sg.accepted, "no round committed more than one token"
    assert gpu.state_save() == ref.state_save(), "state after an accepting generation"
    assert gpu.generate(prompt, 64, k=0)[0] == tg
    probe = [1, 2, 3]
    assert np.array_equal(bits(gpu.eval(probe)), bits(ref.eval(probe)))
    gpu.close(), ref.close()


def counters(s):
    return (s.rounds, s.drafted, s.accepted, s.ngram_rounds, s.ngram_drafted, s.ngram_accepted)


@needs_ref
@pytest.mark.parametrize("which,k,ngram", [("agree", 0, 4), ("agree", 4, 7), ("agree", 2, 8),
                                           ("small", 4, 7)])
def test_ngram_drafts_match_reference(models, agree_model, which, k, ngram):
    """Prompt-lookup drafts (pinfer_spec_params.ngram, engine/src/spec.c:133-151): a prompt
    that repeats a span, so the history holds matches of every class (trusted, checked against
    the MTP draft, short; with k = 0 the no-MTP rule). The drafter is this engine's own
    (ngram.c), so its rounds may differ from the reference engine's; the tokens equal the
    reference's and plain greedy, the states agree, and n-gram rounds were drafted and
    accepted."""
    path, base = agree_model if which == "agree" else (models["small"], np.random.default_rng(
        9).integers(0, pqfile.SMALL.vocab, 24))
    prompt = np.concatenate([base, base[:20], base])
    gpu, ref = pair(path)
    print(f"[case] ngram {which} k={k} ngram={ngram}", flush=True)
    tg, sg = gpu.generate(prompt, 64, k=k, ngram=ngram)
    tr, sr = ref.generate(prompt, 64, k=k, ngram=ngram)
    print(f"[stats] rounds drafted accepted (+ n-gram): {counters(sg)}, reference {counters(sr)}",
          flush=True)
    assert tg == tr
    assert sg.ngram_accepted <= sg.ngram_drafted and sg.ngram_rounds <= sg.rounds
    assert sg.accepted <= sg.drafted
    if which == "agree":  # its output repeats itself; the random model's rarely does
        assert sg.ngram_rounds > 0 and sg.ngram_accepted > 0, "no accepted n-gram round"
    assert gpu.state_save() == ref.state_save(), "state after an n-gram generation"
    assert gpu.generate(prompt, 64, k=0)[0] == tg  # plain greedy: the same tokens and state
    # a continuation leading with the last emitted token keeps the history (both engines)
    tg2, sg2 = gpu.generate([tg[-1]] + list(base[:6]), 24, k=k, ngram=ngram, cont=True)
    tr2, sr2 = ref.generate([tr[-1]] + list(base[:6]), 24, k=k, ngram=ngram, cont=True)
    assert tg2 == tr2
    probe = [1, 2, 3]
    assert np.array_equal(bits(gpu.eval(probe)), bits(ref.eval(probe)))
    gpu.close(), ref.close()


@needs_ref
@pytest.mark.parametrize("k", [2, 4])
def test_ngram_rounds_state_matches_reference(models, k):
    """Prompt-lookup rounds late in the generation (the repeated prompt is matched after about
    90 tokens): their committed rows wait for one MTP pass over up to k + 3 rows after the
    loop, which runs the MTP fc projection with its embedding and norms inside at 7 rows of a
    256-wide hidden. The state blob after the generation, MTP cache included, equals the
    reference engine's (it once held 6 wrong MTP rows: that launch's norm had fewer threads
    than chains)."""
    base = np.random.default_rng(9).integers(0, pqfile.SMALL.vocab, 24)
    prompt = np.concatenate([base, base[:20], base])
    gpu, ref = pair(models["small"])
    print(f"[case] n-gram rounds state k={k}", flush=True)
    tg, sg = gpu.generate(prompt, 96, k=k, ngram=4)
    tr, sr = ref.generate(prompt, 96, k=k, ngram=4)
    assert tg == tr
    # the drafters differ (this engine's match finder, the reference's hash tables), so the
    # rounds may too: only the reachability of an n-gram round and the state are checked
    assert sg.ngram_rounds > 0, "the workload no longer reaches an n-gram round"
    assert gpu.state_save() == ref.state_save(), "state after n-gram rounds"
    gpu.close(), ref.close()


@needs_ref
@pytest.mark.parametrize("which,k,ngram", [("agree", 4, 0), ("agree", 8, 7), ("small", 4, 0),
                                           ("small", 2, 4)])
def test_adaptive_matches_reference(models, agree_model, which, k, ngram):
    """The adaptive policy (pinfer_spec_params.adaptive; this engine's own, adapt.c: the
    verify width with the best expected tokens per second from acceptance counts and measured
    round times, plain steps included). The reference's policy differs and both follow
    measured times, so the engines take different rounds (the counters are not compared); the
    tokens and the state may not differ: both equal plain greedy, and the state blobs after
    the generation are identical. The random model's drafts are almost never accepted, so its
    runs move to plain steps."""
    path, base = agree_model if which == "agree" else (models["small"], np.random.default_rng(
        9).integers(0, pqfile.SMALL.vocab, 24))
    prompt = np.concatenate([base, base[:20], base]) if ngram else base
    gpu, ref = pair(path)
    print(f"[case] adaptive {which} k={k} ngram={ngram}", flush=True)
    plain, _ = gpu.generate(prompt, 96, k=0)
    tg, sg = gpu.generate(prompt, 96, k=k, ngram=ngram, adaptive=1)
    tr, sr = ref.generate(prompt, 96, k=k, ngram=ngram, adaptive=1)
    print(f"[stats] rounds drafted accepted (+ n-gram): {counters(sg)}, reference {counters(sr)}",
          flush=True)
    assert tg == tr == plain
    assert sg.accepted <= sg.drafted <= k * sg.rounds + ngram * sg.ngram_rounds
    assert gpu.state_save() == ref.state_save(), "state after an adaptive generation"
    tg2, _ = gpu.generate([tg[-1]] + list(base[:6]), 24, k=k, ngram=ngram, adaptive=1, cont=True)
    tr2, _ = ref.generate([tr[-1]] + list(base[:6]), 24, k=k, ngram=ngram, adaptive=1, cont=True)
    assert tg2 == tr2
    probe = [1, 2, 3]
    assert np.array_equal(bits(gpu.eval(probe)), bits(ref.eval(probe)))
    gpu.close(), ref.close()


@needs_ref
@pytest.mark.parametrize("kv_dtype", [1, 2])
def test_kv_dtypes_match_reference(models, agree_model, kv_dtype):
    """KV caches stored as binary16 (1) or int8 with row scales (2) (pinfer_params.kv_dtype,
    engine/src/forward_kv.c): prefill logits over two chunks, single-token steps, a speculative
    generation with accepted drafts (MTP cache included) and the state blob (rows in the cache
    format, int8 scales after each group's rows) equal the reference engine's bit for bit; the
    blob loads into the other engine."""
    gpu, ref = pair(models["small"], kv_dtype=kv_dtype)
    rng = np.random.default_rng(20 + kv_dtype)
    prompt = rng.integers(0, pqfile.SMALL.vocab, 70)
    print(f"[case] kv_dtype={kv_dtype} eval", flush=True)
    assert np.array_equal(bits(gpu.eval(prompt)), bits(ref.eval(prompt)))
    for tok in prompt[:3]:
        assert np.array_equal(bits(gpu.eval([tok])), bits(ref.eval([tok])))
    assert gpu.state_save() == ref.state_save(), "state blob after eval"
    gpu.close(), ref.close()
    path, p2 = agree_model
    gpu, ref = pair(path, kv_dtype=kv_dtype)
    print(f"[case] kv_dtype={kv_dtype} generate", flush=True)
    tg, sg = gpu.generate(p2, 48, k=4)
    tr, sr = ref.generate(p2, 48, k=4)
    assert tg == tr and (sg.rounds, sg.drafted, sg.accepted) == (sr.rounds, sr.drafted, sr.accepted)
    assert sg.accepted > 0
    blob = ref.state_save()
    assert gpu.state_save() == blob, "state blob after generation"
    gpu.state_load(blob)
    probe = [7, 8]
    assert np.array_equal(bits(gpu.eval(probe)), bits(ref.eval(probe)))
    gpu.close(), ref.close()


@needs_ref
def test_stop_inside_commit(agree_model):
    """A stop id that is reached among accepted drafts ends the generation inside the round's
    commit; the engines agree on tokens, n_past and the state (through the next logits)."""
    path, prompt = agree_model
    gpu, ref = pair(path)
    full, _ = ref.generate(prompt, 64, k=4)
    for stop in sorted(set(full[1:]))[:3]:
        tg, sg = gpu.generate(prompt, 64, k=4, stop_ids=[stop])
        tr, sr = ref.generate(prompt, 64, k=4, stop_ids=[stop])
        assert tg == tr and tg[-1] == stop and gpu.n_past == ref.n_past
        assert (sg.rounds, sg.drafted, sg.accepted) == (sr.rounds, sr.drafted, sr.accepted)
        assert np.array_equal(bits(gpu.eval([4])), bits(ref.eval([4])))
    gpu.close(), ref.close()


@needs_ref
def test_long_context(models):
    """A 1000-token context: the attention's value rows then span several LDS tiles (448
    positions, then 192 each) in the prefill chunks and in the single-token steps after them."""
    gpu, ref = pair(models["small"], max_ctx=1200)
    rng = np.random.default_rng(13)
    prompt = rng.integers(0, pqfile.SMALL.vocab, 1000)
    print("[case] long context prefill 1000", flush=True)
    assert np.array_equal(bits(gpu.eval(prompt)), bits(ref.eval(prompt))), "after 1000-token prefill"
    for tok in rng.integers(0, pqfile.SMALL.vocab, 3):
        assert np.array_equal(bits(gpu.eval([tok])), bits(ref.eval([tok]))), "single steps"
    tg, sg = gpu.generate([int(tok)], 12, k=4, draft_vocab=1024, cont=True)
    tr, sr = ref.generate([int(tok)], 12, k=4, draft_vocab=1024, cont=True)
    assert tg == tr and (sg.rounds, sg.accepted) == (sr.rounds, sr.accepted)
    gpu.close(), ref.close()


@needs_ref
@pytest.mark.parametrize("kv_dtype", [0, 2])
def test_context_past_lds_scores(models, kv_dtype):
    """max_ctx 9216, above the 8192 scores that the in-LDS softmax holds: the attention runs the
    segmented kernel (exponentials 4096 at a time, the ordered partial sums carried across
    segments, weights recomputed per value tile). An 8400-token prefill, single steps and a
    speculative continuation equal the reference engine's."""
    gpu, ref = pair(models["small"], max_ctx=9216, kv_dtype=kv_dtype)
    rng = np.random.default_rng(14)
    prompt = rng.integers(0, pqfile.SMALL.vocab, 8400)
    print(f"[case] context 8400 of 9216 kv_dtype={kv_dtype}", flush=True)
    assert np.array_equal(bits(gpu.eval(prompt)), bits(ref.eval(prompt))), "after the prefill"
    for tok in rng.integers(0, pqfile.SMALL.vocab, 2):
        assert np.array_equal(bits(gpu.eval([tok])), bits(ref.eval([tok]))), "single steps"
    tg, sg = gpu.generate([int(tok)], 10, k=4, draft_vocab=1024, cont=True)
    tr, sr = ref.generate([int(tok)], 10, k=4, draft_vocab=1024, cont=True)
    assert tg == tr and (sg.rounds, sg.accepted) == (sr.rounds, sr.accepted)
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


@needs_ref
def test_qwen35_08b_config5_workload(tmp_path):
    """The end-to-end workload at its stated size: the 0.8B shape (seed 1), a 512-token random
    prompt (eight 64-row prefill chunks), then exactly 128 tokens at k = 4 with draft vocabulary
    32768 and EOS ignored (engine/tools/pinfer_run.c:384-430), on the GPU engine and on the
    reference engine's sources (16 host threads). Tokens, (rounds, drafted, accepted) and the
    state blob after the decode (every DeltaNet state after 127 rounds of deferred replays, the
    KV caches of all 640 positions, the MTP rows) must be identical."""
    from oracle import refengine

    path = pqfile.write_model(tmp_path / "q08.pq", QWEN35_08B, seed=1)
    prompt = np.random.default_rng(512).integers(0, QWEN35_08B.vocab, 512).astype(np.int32)
    print("[case] 0.8B shape, prompt 512, 128 tokens, k=4: GPU", flush=True)
    gpu = Model(str(path), max_ctx=1024)
    toks, st, tp, td = gpu.bench_generate(prompt, 128, k=4, draft_vocab=32768)
    blob = gpu.state_save()
    gpu.close()
    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    print(f"[case] 0.8B shape, prompt 512, 128 tokens, k=4: reference on {threads} threads",
          flush=True)
    ref = refengine.bench_generate(path, prompt, 128, 4, 32768, threads, max_ctx=1024,
                                   want_state=True)
    print(f"[case] reference prefill {ref.prefill_s:.1f} s, decode {ref.decode_s:.1f} s", flush=True)
    assert toks == ref.tokens
    assert (st.rounds, st.drafted, st.accepted) == (ref.rounds, ref.drafted, ref.accepted)
    assert blob == ref.state, "state blobs differ after the config-5 decode"


def test_invalid_arguments(models):
    gpu = Model(str(models["small"]), max_ctx=64)
    from nibblemac_amd.pinfer import PinferError
    with pytest.raises(PinferError):
        gpu.eval([pqfile.SMALL.vocab])            # token id out of range
    with pytest.raises(PinferError):
        gpu.eval(np.zeros(65, np.int32))           # more than max_ctx
    assert gpu.n_past == 0
    gpu.close()


@needs_ref
def test_state_blob_matches_reference(models):
    """After the same prefill, and after the same speculative generation (MTP rows included),
    the GPU engine's state blob is byte-identical to the reference engine's: the blob format,
    the model fingerprint, the transposed recurrent state and every KV row agree."""
    gpu, ref = pair(models["small"])
    prompt = np.random.default_rng(11).integers(0, pqfile.SMALL.vocab, 37)
    gpu.eval(prompt), ref.eval(prompt)
    assert gpu.state_save() == ref.state_save(), "state after prefill"
    gpu.generate(prompt, 20, k=4, draft_vocab=1024)
    ref.generate(prompt, 20, k=4, draft_vocab=1024)
    assert gpu.state_save() == ref.state_save(), "state after a speculative generation"
    gpu.close(), ref.close()


@needs_ref
def test_state_load_across_engines(models):
    """A reference blob loaded into the GPU engine (and a GPU blob into the reference)
    continues bit-identically; a GPU round trip (save, more tokens, reset, load) too."""
    gpu, ref = pair(models["small"])
    rng = np.random.default_rng(12)
    prompt = rng.integers(0, pqfile.SMALL.vocab, 45)
    more = rng.integers(0, pqfile.SMALL.vocab, 9)
    ref.eval(prompt)
    blob_r = ref.state_save()
    gpu.state_load(blob_r)
    assert gpu.n_past == 45
    a, b = gpu.eval(more), ref.eval(more)
    assert np.array_equal(bits(a), bits(b)), "reference blob -> GPU"
    blob_g = gpu.state_save()
    ref.reset()
    ref.state_load(blob_g)
    c, d = ref.eval([3, 4]), gpu.eval([3, 4])
    assert np.array_equal(bits(c), bits(d)), "GPU blob -> reference"
    # round trip on the GPU
    gpu.reset()
    gpu.eval(prompt)
    blob = gpu.state_save()
    x = gpu.eval(more)
    gpu.reset()
    gpu.state_load(blob)
    y = gpu.eval(more)
    assert np.array_equal(bits(x), bits(y)), "GPU round trip"
    # blobs of another shape or corrupted headers are refused
    from nibblemac_amd.pinfer import PinferError
    bad = bytearray(blob)
    bad[0] ^= 1
    with pytest.raises(PinferError):
        gpu.state_load(bytes(bad))
    with pytest.raises(PinferError):
        gpu.state_load(blob[:100])
    gpu.close(), ref.close()


@needs_ref
def test_checkpoint_rewind(models):
    """checkpoint / rewind (engine/include/pinfer.h:153-175): after a rewind, feeding other
    tokens gives exactly what feeding them at the checkpoint gives, on both engines."""
    gpu, ref = pair(models["small"])
    rng = np.random.default_rng(13)
    prefix = rng.integers(0, pqfile.SMALL.vocab, 30)
    a_toks = rng.integers(0, pqfile.SMALL.vocab, 6)
    b_toks = rng.integers(0, pqfile.SMALL.vocab, 4)
    from nibblemac_amd.pinfer import PinferError
    with pytest.raises(PinferError):
        gpu.rewind()                      # no checkpoint yet
    assert gpu.checkpoint_n_past == -1
    for m in (gpu, ref):
        m.eval(prefix)
        m.checkpoint()
        m.eval(a_toks)
        m.rewind()
    assert gpu.n_past == ref.n_past == 30 and gpu.checkpoint_n_past == 30
    x, y = gpu.eval(b_toks), ref.eval(b_toks)
    assert np.array_equal(bits(x), bits(y)), "after rewind vs reference"
    fresh = Model(str(models["small"]), max_ctx=512)
    z = fresh.eval(np.concatenate([prefix, b_toks]))
    assert np.array_equal(bits(x), bits(z)), "after rewind vs a fresh context"
    gpu.rewind()                          # one checkpoint serves any number of rewinds
    tg, _ = gpu.generate(b_toks, 8, k=4, draft_vocab=1024, cont=True)
    ref.rewind()
    tr, _ = ref.generate(b_toks, 8, k=4, draft_vocab=1024, cont=True)
    assert tg == tr
    gpu.reset()                           # reset drops the checkpoint
    assert gpu.checkpoint_n_past == -1
    with pytest.raises(PinferError):
        gpu.rewind()
    fresh.close(), gpu.close(), ref.close()
