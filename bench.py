#!/usr/bin/env python3
"""Benchmark of speculative greedy decoding (draft k = 4, verify + commit) on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-kernels] [--no-accept]
                    [--head-only [--eager] [--copy-mib M]]

Workload (config 5): a 0.8B-shaped Qwen3.5 hybrid (24 layers: 18 Gated DeltaNet + 6 gated full
attention, hidden 1024, FFN 3584, vocab 248320 with the Q4K embedding tied to the LM head, one MTP
layer), random-init weights N(0, 0.02) packed as Q4K_G32 into a .pq file, loaded by libpinfer.so
into HBM. One step is the reference CLI's benchmark (engine/tools/pinfer_run.c:384-430): prefill
a 512-token random prompt, then generate exactly 128 tokens with EOS ignored at k = 4 drafts per
verification pass, drafts from the MTP head over the first 32768 ids. `value` is verified tokens
per second of the decode: (128 - 1) per step / decode seconds, over K steps.

`roofline` is the LM head as the verify round launches it (nmx_head_keys: the Q4K x A8 matvec
248320 x 1024 over k + 1 = 5 rows with the fused argmax, leaving partial keys whose reduction and
the acceptance run in the commit's workgroups), four rotating copies of the 143 MB head so no
launch finds it in the 256 MB MALL, timed with HIP events around back-to-back launches on the
stream it runs on (so the time is the kernel's, as a kernel trace reports it; the graph-replay
time is given beside it); the line also carries the same launch with the head resident in the
MALL (one copy). `kernels` holds configs 1-4 (nibblemac_amd/kbench.py). `cpu_baseline` is the
reference engine's own sources with the oracle's threaded Q4K operators
(oracle/_ref/libpinfer_refq4k.so) on the host cores: the config-5 workload itself on the GPU
box's CPU share (16 threads), its tokens checked against the GPU's, plus a 1-thread run on a
bounded sample and the oracle's Q4K matvec of config 1 on 1 thread. With random weights the
drafts are essentially never accepted; `accepting` times the same workload on the same weights
with final norms that make the drafts agree (multi-token commits and deferred DeltaNet replays),
its tokens checked against plain greedy decoding.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from nibblemac_amd import kbench, pqfile, pqtool  # noqa: E402
from nibblemac_amd.nmx import Device  # noqa: E402
from nibblemac_amd.pinfer import Model  # noqa: E402
from nibblemac_amd.synth import QWEN35_08B  # noqa: E402

METRIC = "verified tok/s at draft k=4 (0.8B-shape Q4K); Q4K matvec GB/s vs HBM peak"
HBM_PEAK_GBS = 8000.0
K_DRAFT, DRAFT_VOCAB = 4, 32768
N_PROMPT, N_GEN = 512, 128
CPU_SHARE = 16                       # host threads of one GPU's share of the box
ONE_PROMPT, ONE_GEN = 16, 5          # the bounded 1-thread sample
TRAFFIC_FILE = ROOT / "profiles" / "q4k_head_n5_fused_traffic.json"


def default_leg(paths: dict, prompt: np.ndarray, steps: int) -> dict:
    """What a caller of pinfer_default_spec_params() gets (k = 4, adaptive width, prompt-lookup
    drafts of up to 7 tokens; engine/src/spec.c:385-391) on the config-5 workload, on the
    random-init model (drafts essentially never accepted) and on the agreeing model; the tokens
    are checked against plain greedy decoding (k = 0) of the same model, which is timed too."""
    out = {}
    for name, path in paths.items():
        with Model(str(path), max_ctx=1024) as gpu:
            sp = gpu.default_spec_params()
            plain, _, _, td0 = gpu.bench_generate(prompt, N_GEN, 0, DRAFT_VOCAB)
            gpu.bench_generate(prompt, N_GEN, **sp)
            dec, rounds, ng, acc = 0.0, 0, 0, 0
            for _ in range(steps):
                toks, st, _, td = gpu.bench_generate(prompt, N_GEN, **sp)
                if toks != plain:
                    raise SystemExit(f"bench.py: default leg ({name}): tokens differ from greedy")
                dec, rounds, ng, acc = dec + td, rounds + st.rounds, ng + st.ngram_rounds, \
                    acc + st.accepted
            out[name] = {"tok_s": round(steps * (N_GEN - 1) / dec, 2),
                         "plain_k0_tok_s": round((N_GEN - 1) / td0, 2),
                         "rounds_per_step": rounds / steps, "ngram_rounds_per_step": ng / steps,
                         "accepted_per_step": acc / steps, "tokens_match_greedy": True}
    out["spec_params"] = sp
    return out


def accepting_leg(tmp: str, prompt: np.ndarray, steps: int) -> dict:
    """The same workload on the same shape with final norms that make the MTP drafts agree
    (pqfile.agreeing_norm) and an untied head whose rows past the draft vocabulary are
    N(0, 0.002) (otherwise the same random-init weights), so that multi-token commits and the
    deferred DeltaNet replays run inside the timed rounds. Its tokens are checked against plain
    greedy decoding (k = 0) of the same model."""
    w = pqfile.agreeing_norm(QWEN35_08B.hidden)
    path = Path(tmp) / "qwen35_08b_shape_q4k_agree.pq"
    pqfile.write_model(path, QWEN35_08B, seed=1, overrides={"norm.weight": w,
                                                            "mtp.norm.weight": w},
                       lm_head=(DRAFT_VOCAB, 0.002))
    with Model(str(path), max_ctx=1024) as gpu:
        plain, _, _, td0 = gpu.bench_generate(prompt, N_GEN, 0, DRAFT_VOCAB)
        gpu.bench_generate(prompt, N_GEN, K_DRAFT, DRAFT_VOCAB)
        dec, rounds, drafted, accepted = 0.0, 0, 0, 0
        for _ in range(steps):
            toks, st, _, td = gpu.bench_generate(prompt, N_GEN, K_DRAFT, DRAFT_VOCAB)
            if toks != plain:
                raise SystemExit("bench.py: accepting leg: speculative tokens differ from greedy")
            dec, rounds = dec + td, rounds + st.rounds
            drafted, accepted = drafted + st.drafted, accepted + st.accepted
    leg = {"workload": "as config; final norms pqfile.agreeing_norm, untied head with rows "
                       f">= {DRAFT_VOCAB} N(0, 0.002) (drafts agree)",
           "tok_s": round(steps * (N_GEN - 1) / dec, 2), "steps": steps,
           "rounds_per_step": rounds / steps, "drafted": drafted // steps,
           "accepted": accepted // steps,
           "tokens_per_pass": round(steps * (N_GEN - 1) / rounds, 3),
           "ms_per_pass": round(dec / rounds * 1e3, 4),
           "plain_k0_tok_s": round((N_GEN - 1) / td0, 2), "tokens_match_greedy": True}
    return leg, path


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def host_threads() -> tuple[int, int]:
    """(threads used, CPUs in this process's affinity mask)."""
    aff = len(os.sched_getaffinity(0))
    return max(1, min(CPU_SHARE, aff)), aff


def head_roofline(copies: int = 4, eager: bool = False, copy_mib: int = 0) -> dict:
    """The in-path LM head (nmx_head_accept at 5 rows, 4 drafts, no logits written) over
    `copies` rotating head copies, timed with HIP events over graph replays (eager: stream
    launches, for profiler counter runs; copy_mib: a plain device copy of that many MiB first,
    whose counters scale the HBM traffic readings)."""
    with Device(0) as dev:
        if copy_mib:
            a = dev.zeros(copy_mib << 20, np.uint8)
            b = dev.zeros(copy_mib << 20, np.uint8)
            dev.copy(b, a, copy_mib << 20)
            dev.sync()
            a.free(), b.free()
        if eager:
            return head_eager(dev, copies)
        r = kbench.config4_head(dev, copies=copies)
    line = r["in_path_cold"]
    traffic = None
    if TRAFFIC_FILE.exists():
        traffic = json.loads(TRAFFIC_FILE.read_text()).get("bytes_per_launch")
    gbs = line["GB_s"]
    return {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
            "kernel": r["in_path_kernel"] + ": the LM head 248320x1024 Q4K x 5 A8 rows with the "
                      "fused argmax as the verify round launches it (the keys' reduction and the "
                      "acceptance run in the commit's workgroups); cold",
            "us_per_launch": line["us"], "algorithmic_bytes": r["in_path_algorithmic_bytes"],
            "copies": copies,
            "timing": "HIP events around 40 back-to-back launches on the kernel's stream (the "
                      "kernel's duration); us_graph_replay: the same launches as graph replays",
            "us_graph_replay": line["us_graph_replay"],
            "warm_mall_resident": r["in_path_warm"],
            "api_head_accept_us": {k: v["us"] for k, v in r.items() if k.startswith("accept")}}


def head_eager(dev: Device, copies: int, reps: int = 40) -> dict:
    """Eager launches of the in-path head, nmx_head_keys (for rocprofv3 counter runs)."""
    s, n = QWEN35_08B, K_DRAFT + 1
    W = pqtool.gauss_q4k(7, 10_000, s.vocab, s.hidden, 0.02)
    heads = [dev.to_device(W) for _ in range(copies)]
    X = dev.to_device(np.random.default_rng(4).standard_normal((n, s.hidden)).astype(np.float32))
    q = dev.empty((s.hidden // 32, n, 32), np.int8)
    d = dev.empty((s.hidden // 32, n), np.float32)
    fs = dev.empty((s.hidden // 32, n), np.float32)
    dev.quant_a8(X, n, s.hidden, q, d, fs)
    work = dev.alloc(dev.head_work_bytes(s.vocab, n))
    dcopy, drafts = dev.zeros(16, np.int32), dev.zeros(n - 1, np.int32)
    e0, e1 = dev.event(), dev.event()
    dev.record(e0)
    for r in range(reps):
        dev.head_keys(heads[r % copies], s.vocab, s.hidden, n, q, d, fs, drafts, work, dcopy)
    dev.record(e1)
    dev.sync()
    return {"us_per_call": round(dev.elapsed_ms(e0, e1) / reps * 1e3, 2), "timing": "eager"}


def cpu_baseline(path: Path, gpu_run: tuple, prompt: np.ndarray) -> dict:
    """The reference engine on the host: the config-5 workload on CPU_SHARE threads (tokens and
    statistics checked against the GPU's), a 1-thread run of a bounded sample, and the
    oracle's config-1 matvec on 1 thread."""
    from oracle import refengine  # the checker and CPU baseline live with the oracle

    thr, aff = host_threads()
    full = refengine.bench_generate(path, prompt, N_GEN, K_DRAFT, DRAFT_VOCAB, thr)
    gtoks, gst = gpu_run
    match = full.tokens == gtoks and (full.rounds, full.drafted, full.accepted) == \
        (gst.rounds, gst.drafted, gst.accepted)
    log(f"cpu reference ({thr} threads): prefill {N_PROMPT} tok {full.prefill_s:.2f} s, decode "
        f"{N_GEN} tok {full.decode_s:.2f} s ({(N_GEN - 1) / full.decode_s:.3f} tok/s), GPU "
        f"tokens match: {match}")
    if not match:
        raise SystemExit("bench.py: GPU tokens differ from the reference engine")
    one = refengine.bench_generate(path, prompt[:ONE_PROMPT], ONE_GEN, K_DRAFT, DRAFT_VOCAB, 1)
    log(f"cpu reference (1 thread): prefill {ONE_PROMPT} tok {one.prefill_s:.2f} s, decode "
        f"{ONE_GEN} tok {one.decode_s:.2f} s ({(ONE_GEN - 1) / one.decode_s:.4f} tok/s)")
    mv = cpu_matvec_1t()
    log(f"cpu oracle Q4K matvec 3584x1024 n=1, 1 thread: {mv['us']:.0f} us, {mv['GB_s']} GB/s")
    ks = cpu_kernels(thr)
    log(f"cpu oracle configs 2-4: {json.dumps(ks)}")
    return {"value": round((N_GEN - 1) / full.decode_s, 4), "unit": "tok/s", "cores": thr,
            "kind": "reference", "tokens_match_gpu": match, "affinity_cpus": aff,
            "prefill_tok_s": round(N_PROMPT / full.prefill_s, 2),
            "sample": f"the config-5 workload itself: reference engine sources (Q4K operators from "
                      f"the oracle's scalar C restatement; the reference's Q4K kernels are "
                      f"NEON-only) on {thr} threads (this GPU's share of the host; {aff} CPUs in "
                      f"the affinity mask): prefill {N_PROMPT} random ids, then {N_GEN} tokens at "
                      f"k={K_DRAFT}, draft vocab {DRAFT_VOCAB}, EOS ignored; decode timed",
            "one_thread": {"value": round((ONE_GEN - 1) / one.decode_s, 4), "unit": "tok/s",
                           "sample": f"prefill {ONE_PROMPT} ids, then {ONE_GEN} tokens at k={K_DRAFT}"},
            "matvec_config1_1t": mv, "configs2to4": ks}


def cpu_kernels(thr: int) -> dict:
    """Configs 2-4 on the oracle (the reference's Q4K / A8, DeltaNet and acceptance arithmetic
    restated in scalar C, oracle/), on 1 thread and on thr threads (rows split; the output is
    the same bit for bit), with the inputs of the GPU's kernel lines."""
    import oracle

    s, n = QWEN35_08B, K_DRAFT + 1
    H, F = s.hidden, s.ffn
    rng = np.random.default_rng(2)

    def a8(cols):
        return oracle.quant_a8(rng.standard_normal((n, cols)).astype(np.float32))

    def timed(f):
        t0 = time.perf_counter()
        f()
        return time.perf_counter() - t0

    out = {}
    # config 2: one DeltaNet layer's products at 5 rows: qkv/z/b/a, out, gate, up, down
    mats = [(8224, H), (H, 2048), (F, H), (F, H), (H, F)]
    Ws = [pqtool.gauss_q4k(20 + i, 0, r, c, 0.02) for i, (r, c) in enumerate(mats)]
    acts = {c: a8(c) for c in {c for _, c in mats}}
    wbytes = sum(W.nbytes for W in Ws)
    c2 = {"weight_bytes": wbytes, "shape": "DeltaNet layer 8224x1024 + 1024x2048 + 2 x 3584x1024 "
                                           "+ 1024x3584, Q4K x 5 A8 rows"}
    for t in (1, thr):
        sec = timed(lambda: [oracle.q4k_matmul(W, r, c, *acts[c], n, threads=t)
                             for W, (r, c) in zip(Ws, mats)])
        c2[f"{t}t"] = {"ms": round(sec * 1e3, 2), "GB_s": round(wbytes / sec / 1e9, 3)}
    out["config2_layer"] = c2
    # config 3: 16 heads x 128 x 128, 5 tokens: the logged pass (state after token 0, log rows
    # 1..4), then the replay of the 4 pending rows (a full acceptance)
    heads, dk, dv = 16, 128, 128
    qkv = rng.standard_normal((n, 2 * heads * dk + heads * dv)).astype(np.float32)
    for o in (0, heads * dk):
        qkv[:, o:o + heads * dk] /= np.linalg.norm(
            qkv[:, o:o + heads * dk].reshape(n, heads, dk), axis=-1).repeat(dk, axis=1)
    decay = (0.9 + 0.1 / (1 + np.exp(-rng.standard_normal((n, heads))))).astype(np.float32)
    beta = (1 / (1 + np.exp(-rng.standard_normal((n, heads))))).astype(np.float32)
    S0 = (rng.standard_normal((heads, dk, dv)) * 0.02).astype(np.float32)
    kw = dict(n=n, heads=heads, rep=1, dk=dk, dv=dv)

    def rule_apply():
        S1, _, lg = oracle.lin_rule(qkv, decay, beta, S0, log=True, **kw)
        oracle.lin_apply(S1, lg[1:], n - 1, heads, dk, dv)

    rule_apply()
    reps = 20
    sec = timed(lambda: [rule_apply() for _ in range(reps)]) / reps
    out["config3_deltanet_1t"] = {"us_per_layer_pass": round(sec * 1e6, 1),
                                  "work": "logged pass of 5 tokens + replay of 4 pending rows"}
    # config 4: the LM head with argmax and acceptance (1 thread: a 16384-row sample)
    Wh = pqtool.gauss_q4k(7, 10_000, s.vocab, H, 0.02)
    qh = a8(H)
    c4 = {"bytes_per_call": int(Wh.nbytes)}
    for t, rows in ((1, 16384), (thr, s.vocab)):
        Wr = Wh[:kbench.q4k_bytes(rows, H)]

        def head():
            Y = oracle.q4k_matmul(Wr, rows, H, *qh, n, threads=t)
            oracle.accept(Y, np.array([oracle.argmax(Y[i]) for i in range(n - 1)], np.int32))

        sec = timed(head)
        gbs = Wr.nbytes / sec / 1e9
        c4[f"{t}t"] = {"GB_s": round(gbs, 3), "ms_per_call": round(Wh.nbytes / gbs / 1e6, 1),
                       "sample_rows": rows}
    out["config4_head"] = c4
    return out


def cpu_matvec_1t(reps: int = 20) -> dict:
    """The oracle's scalar Q4K x A8 matvec of config 1 (3584 x 1024, n = 1) on 1 thread."""
    import oracle

    rows, cols = 3584, 1024
    W = pqtool.gauss_q4k(1, 0, rows, cols, 0.02)
    q, d, fs = oracle.quant_a8(np.random.default_rng(1).standard_normal((1, cols)).astype(np.float32))
    oracle.q4k_matmul(W, rows, cols, q, d, fs, 1)
    t0 = time.perf_counter()
    for _ in range(reps):
        oracle.q4k_matmul(W, rows, cols, q, d, fs, 1)
    us = (time.perf_counter() - t0) / reps * 1e6
    algo = kbench.matvec_algo_bytes(rows, cols, 1)
    return {"us": round(us, 1), "GB_s": round(algo / (us * 1e-6) / 1e9, 3), "cores": 1,
            "kind": "port", "algorithmic_bytes": algo}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-kernels", action="store_true", help="skip the config 1-4 lines")
    ap.add_argument("--no-accept", action="store_true", help="skip the accepting-drafts leg")
    ap.add_argument("--head-only", action="store_true",
                    help="only the in-path LM head launches (for counter runs)")
    ap.add_argument("--kernels-only", action="store_true", help="only the config 1-4 lines")
    ap.add_argument("--eager", action="store_true",
                    help="with --head-only / --kernels-only: stream launches, not graph replays")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="with --head-only: a device copy of this size first (counter scale)")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {a.gpus} is not supported "
              "(the multi-GPU sharding is a design, not a measured path)", file=sys.stderr)
        return 2
    if a.head_only:
        roof = head_roofline(eager=a.eager, copy_mib=a.copy_mib)
        log(f"head: {roof}")
        print(json.dumps({"roofline": roof}), flush=True)
        return 0
    if a.kernels_only:
        kbench.EAGER = a.eager
        with Device(0) as dev:
            ks = kbench.run_all(dev)
        print(json.dumps({"kernels": ks}), flush=True)
        return 0
    rng = np.random.default_rng(512)
    prompt = rng.integers(0, QWEN35_08B.vocab, N_PROMPT).astype(np.int32)
    with tempfile.TemporaryDirectory(prefix="nmx_bench_") as tmp:
        path = Path(tmp) / "qwen35_08b_shape_q4k.pq"
        t0 = time.time()
        pqfile.write_model(path, QWEN35_08B, seed=1)
        log(f"model written in {time.time() - t0:.1f} s ({path.stat().st_size / 1e6:.0f} MB)")
        with Model(str(path), max_ctx=1024) as gpu:
            for w in range(a.warmup):
                gpu.bench_generate(prompt, N_GEN, K_DRAFT, DRAFT_VOCAB)
            dec, pre, stats, first, first_st = 0.0, 0.0, [0, 0, 0], None, None
            for s in range(a.steps):
                toks, st, tp, td = gpu.bench_generate(prompt, N_GEN, K_DRAFT, DRAFT_VOCAB)
                first, first_st = first or toks, first_st or st
                if toks != first:
                    raise SystemExit("bench.py: generations differ between steps")
                dec, pre = dec + td, pre + tp
                stats = [stats[0] + st.rounds, stats[1] + st.drafted, stats[2] + st.accepted]
                log(f"step {s}: prefill {tp * 1e3:.1f} ms, decode {td * 1e3:.1f} ms, "
                    f"{(N_GEN - 1) / td:.1f} tok/s, rounds {st.rounds} accepted {st.accepted}")
            tps = a.steps * (N_GEN - 1) / dec
        cpu = None if a.no_cpu else cpu_baseline(path, (first, first_st), prompt)
        accept = default = None
        if not a.no_accept:
            accept, agree_path = accepting_leg(tmp, prompt, a.steps)
            log(f"accepting leg: {json.dumps(accept)}")
            default = default_leg({"random_init": path, "agreeing": agree_path}, prompt,
                                  max(1, min(a.steps, 5)))
            log(f"default spec params leg: {json.dumps(default)}")
    roof = head_roofline()
    log(f"head (in path, cold): {roof['us_per_launch']} us, {roof['achieved']} GB/s")
    kernels = None
    if not a.no_kernels:
        with Device(0) as dev:
            kernels = kbench.run_all(dev)
        for k, v in kernels.items():
            log(f"{k}: {json.dumps(v)}")
    rounds = stats[0] / a.steps
    rec = {
        "metric": METRIC, "value": round(tps, 2), "unit": "tok/s", "n_gpus": 1,
        "steps": a.steps, "warmup": a.warmup, "ms_per_step": round(dec / a.steps * 1e3, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "q4k x int8 -> fp32",
        "data": "synthetic (random-init 0.8B-shape weights N(0,0.02) packed Q4K, random prompt)",
        "config": {"workload": f"speculative greedy decode, k={K_DRAFT}, draft vocab "
                               f"{DRAFT_VOCAB}, prompt {N_PROMPT}, {N_GEN} tokens, EOS ignored",
                   "model": "qwen3.5-0.8b-shape-q4k (24 layers, 1 MTP layer, vocab 248320)",
                   "global_batch": 1, "seq_len": N_PROMPT + N_GEN,
                   "parallelism": "single-gpu"},
        "spec": {"rounds_per_step": rounds, "drafted": stats[1] // a.steps,
                 "accepted": stats[2] // a.steps,
                 "tokens_per_pass": round((N_GEN - 1) / rounds, 3) if rounds else None,
                 "ms_per_pass": round(dec / stats[0] * 1e3, 4) if stats[0] else None},
        "prefill_tok_s": round(a.steps * N_PROMPT / pre, 1),
        "roofline": roof, "cpu_baseline": cpu, "accepting": accept,
        "default_spec_params": default, "kernels": kernels,
    }
    print(json.dumps(rec), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
