#!/usr/bin/env python3
"""Benchmark of speculative greedy decoding (draft k = 4, verify + commit) on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--roofline-only]

Workload: a 0.8B-shaped Qwen3.5 hybrid (24 layers: 18 Gated DeltaNet + 6 gated full attention,
hidden 1024, FFN 3584, vocab 248320 with the Q4K embedding tied to the LM head, one MTP layer),
random-init weights N(0, 0.02) packed as Q4K_G32 into a .pq file, loaded by libpinfer.so into
HBM. One step is the reference CLI's benchmark (engine/tools/pinfer_run.c:384-430): prefill a
512-token random prompt, then generate exactly 128 tokens with EOS ignored at k = 4 drafts per
verification pass, drafts from the MTP head over the first 32768 ids. `value` is verified
tokens per second of the decode: (128 - 1) per step / decode seconds, over K steps.

`roofline` is the Q4K x A8 matvec kernel on the LM-head shape (248320 x 1024, 5 rows = k + 1,
two copies rotating so the 143 MB head never sits in the 256 MB MALL), timed with HIP events on
the stream it runs on. `cpu_baseline` is the reference engine's own sources with the oracle's
threaded Q4K operators (oracle/_ref/libpinfer_refq4k.so) on the host cores, on a bounded sample
of the same workload (shorter prompt and generation); its tokens are checked against the GPU's
on the same sample.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from nibblemac_amd import pqfile, pqtool  # noqa: E402
from nibblemac_amd.nmx import Device  # noqa: E402
from nibblemac_amd.pinfer import Model, SpecParams, SpecStats, load_library  # noqa: E402
from nibblemac_amd.synth import QWEN35_08B  # noqa: E402

METRIC = "verified tok/s at draft k=4 (0.8B-shape Q4K); Q4K matvec GB/s vs HBM peak"
HBM_PEAK_GBS = 8000.0
K_DRAFT, DRAFT_VOCAB = 4, 32768
N_PROMPT, N_GEN = 512, 128
CPU_PROMPT, CPU_GEN = 32, 17
TRAFFIC_FILE = ROOT / "profiles" / "q4k_head_n5_traffic.json"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def host_threads() -> int:
    return max(1, min(16, len(os.sched_getaffinity(0))))


def time_graph(dev: Device, g, reps: int) -> float:
    e0, e1 = dev.event(), dev.event()
    dev.record(e0)
    for _ in range(reps):
        dev.graph_launch(g)
    dev.record(e1)
    return dev.elapsed_ms(e0, e1)


def head_roofline(reps: int = 20, graphs: int = 5, eager: bool = False,
                  copy_mib: int = 0) -> dict:
    """The Q4K matvec of the LM head (248320 x 1024) over k + 1 = 5 A8 rows, logits written,
    two rotating weight copies (cold), `reps` launches per graph, timed with HIP events on the
    stream the kernels run on. eager: plain stream launches instead of graph replays (for
    profiler counter runs); copy_mib: first copy that many MiB device to device (the plain copy
    whose counters scale the HBM traffic readings)."""
    s, n = QWEN35_08B, K_DRAFT + 1
    thr = host_threads()
    with Device(0) as dev:
        if copy_mib:
            a = dev.zeros(copy_mib << 20, np.uint8)
            b = dev.zeros(copy_mib << 20, np.uint8)
            dev.copy(b, a, copy_mib << 20)
            dev.sync()
            a.free(), b.free()
        W = pqtool.gauss_q4k(7, 10_000, s.vocab, s.hidden, 0.02, thr)
        heads = [dev.to_device(W), dev.to_device(W)]
        X = dev.to_device(np.random.default_rng(7).standard_normal((n, s.hidden))
                          .astype(np.float32))
        q = dev.empty((s.hidden // 32, n, 32), np.int8)
        d = dev.empty((s.hidden // 32, n), np.float32)
        fs = dev.empty((s.hidden // 32, n), np.float32)
        dev.quant_a8(X, n, s.hidden, q, d, fs)
        logits = dev.empty((n, s.vocab), np.float32)

        def launches():
            for r in range(reps):
                dev.q4k_matmul(heads[r % 2], s.vocab, s.hidden, n, q, d, fs, logits)

        if eager:
            launches()
            dev.sync()
            e0, e1 = dev.event(), dev.event()
            dev.record(e0)
            for _ in range(graphs):
                launches()
            dev.record(e1)
            ms = dev.elapsed_ms(e0, e1) / (reps * graphs)
        else:
            dev.graph_begin()
            launches()
            g = dev.graph_end()
            dev.graph_launch(g)
            dev.sync()
            ms = time_graph(dev, g, graphs) / (reps * graphs)
        dev.sync()
    wbytes = s.vocab // 4 * (s.hidden // 256) * 576
    algo = wbytes + n * s.hidden + 2 * 4 * n * (s.hidden // 32) + 4 * n * s.vocab
    achieved = algo / (ms * 1e-3) / 1e9
    traffic = None
    if TRAFFIC_FILE.exists():
        traffic = json.loads(TRAFFIC_FILE.read_text()).get("bytes_per_launch")
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
            "kernel": "q4k_mvx_k<5,false> (LM head 248320x1024 Q4K x 5 A8 rows, block dots on the matrix cores, cold)",
            "us_per_launch": round(ms * 1e3, 2), "algorithmic_bytes": algo,
            "timing": "eager stream launches" if eager else "graph replays"}


class PfStop(ctypes.Structure):
    """The reference's stop conditions (engine/src/spec.h:89-96)."""
    _fields_ = [("eos", ctypes.c_int), ("stop_ids", ctypes.c_void_p), ("n_stop", ctypes.c_int),
                ("on_token", ctypes.c_void_p), ("user", ctypes.c_void_p)]


def ref_bench_generate(path: Path, prompt: np.ndarray, n_gen: int, threads: int):
    """The reference engine's benchmark sequence (pinfer_run.c:384-397): pf_spec_prefill, then
    pf_spec_decode with EOS disabled; returns (tokens, stats, prefill s, decode s)."""
    import oracle  # the reference build lives with the checker

    lib = load_library(str(oracle.HERE / "_ref" / "libpinfer_refq4k.so"))
    cd = lib.cdll
    cd.pf_spec_prefill.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                   ctypes.c_void_p, ctypes.c_int]
    cd.pf_spec_decode.argtypes = [ctypes.c_void_p] * 8
    p = lib.pinfer_default_params()
    p.max_ctx, p.n_threads = 1024, threads
    err = ctypes.c_int(0)
    ctx = lib.pinfer_load(str(path).encode(), ctypes.byref(p), ctypes.byref(err))
    if not ctx:
        raise RuntimeError(f"reference pinfer_load failed: {err.value}")
    try:
        prompt = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(n_gen, np.int32)
        sp, st = SpecParams(K_DRAFT, DRAFT_VOCAB, 0, 0), SpecStats()
        stop, status = PfStop(-1, None, 0, None, None), ctypes.c_int(0)
        t0 = time.perf_counter()
        rc = cd.pf_spec_prefill(ctx, prompt.ctypes.data, prompt.size, ctypes.byref(sp), 0)
        t1 = time.perf_counter()
        if rc < 0:
            raise RuntimeError(f"reference prefill failed: {rc}")
        n = cd.pf_spec_decode(ctx, out.ctypes.data, n_gen, ctypes.byref(sp), ctypes.byref(stop),
                              ctypes.byref(st), None, ctypes.byref(status))
        t2 = time.perf_counter()
        if n != n_gen or status.value != 0:
            raise RuntimeError(f"reference decode failed: {n} tokens, status {status.value}")
        return [int(x) for x in out], st, t1 - t0, t2 - t1
    finally:
        lib.pinfer_free(ctx)


def cpu_baseline(path: Path, gpu: Model, prompt: np.ndarray) -> dict:
    thr = host_threads()
    sample = prompt[:CPU_PROMPT]
    toks, st, tp, td = ref_bench_generate(path, sample, CPU_GEN, thr)
    gtoks, gst, _, _ = gpu.bench_generate(sample, CPU_GEN, K_DRAFT, DRAFT_VOCAB)
    match = toks == gtoks and (st.rounds, st.drafted, st.accepted) == \
        (gst.rounds, gst.drafted, gst.accepted)
    log(f"cpu reference: prefill {CPU_PROMPT} tok {tp:.2f} s, decode {CPU_GEN} tok {td:.2f} s "
        f"({(CPU_GEN - 1) / td:.3f} tok/s), GPU tokens match: {match}")
    if not match:
        raise SystemExit("bench.py: GPU tokens differ from the reference engine on the sample")
    return {"value": round((CPU_GEN - 1) / td, 4), "unit": "tok/s", "cores": thr,
            "kind": "reference", "tokens_match_gpu": match,
            "sample": f"reference engine sources + oracle Q4K operators on {thr} threads: "
                      f"prefill {CPU_PROMPT} random ids, then {CPU_GEN} tokens at k={K_DRAFT} "
                      f"(draft vocab {DRAFT_VOCAB}, EOS ignored), decode timed"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--roofline-only", action="store_true",
                    help="only the LM-head matvec launches (for counter runs)")
    ap.add_argument("--eager", action="store_true",
                    help="with --roofline-only: stream launches instead of graph replays")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="with --roofline-only: a device copy of this size first (counter scale)")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {a.gpus} is not supported "
              "(the multi-GPU sharding is a design, not a measured path)", file=sys.stderr)
        return 2
    if a.roofline_only:
        roof = head_roofline(eager=a.eager, copy_mib=a.copy_mib)
        log(f"head matvec: {roof['us_per_launch']} us/launch, {roof['achieved']} GB/s")
        print(json.dumps({"roofline": roof}), flush=True)
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
            dec, pre, stats, first = 0.0, 0.0, [0, 0, 0], None
            for s in range(a.steps):
                toks, st, tp, td = gpu.bench_generate(prompt, N_GEN, K_DRAFT, DRAFT_VOCAB)
                first = first or toks
                if toks != first:
                    raise SystemExit("bench.py: generations differ between steps")
                dec, pre = dec + td, pre + tp
                stats = [stats[0] + st.rounds, stats[1] + st.drafted, stats[2] + st.accepted]
                log(f"step {s}: prefill {tp * 1e3:.1f} ms, decode {td * 1e3:.1f} ms, "
                    f"{(N_GEN - 1) / td:.1f} tok/s, rounds {st.rounds} accepted {st.accepted}")
            tps = a.steps * (N_GEN - 1) / dec
            cpu = None if a.no_cpu else cpu_baseline(path, gpu, prompt)
    roof = head_roofline()
    log(f"head matvec: {roof['us_per_launch']} us/launch, {roof['achieved']} GB/s")
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
        "roofline": roof, "cpu_baseline": cpu,
    }
    print(json.dumps(rec), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
