#!/usr/bin/env python3
"""Benchmark of the speculative-verify hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]

Workload (0.8B-shaped Qwen3.5 hybrid, random-init weights N(0, 0.02) packed as Q4K): one step
is one k = 4 verify round's Q4K weight stream — every matrix of the 24 layers (18 Gated
DeltaNet, 6 gated full attention) applied to k + 1 = 5 activation rows (A8-quantized on the
device), then the 248320-row LM head fused with greedy argmax and draft acceptance. The step is
captured in one HIP graph; inputs are resident in HBM before the timed region.

Printed: ONE JSON line. `value` is the verify weight stream in GB/s (algorithmic weight +
activation bytes per step / step time); `roofline` is the Q4K matvec on the LM-head shape
(5 rows, cold: two copies rotate so the 143 MB head never sits in the 256 MB MALL), timed with
HIP events on the stream the kernels run on; `cpu_baseline` is the oracle (the portable scalar
C restatement) over the same weight stream on the host cores.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from nibblemac_amd import pqtool  # noqa: E402
from nibblemac_amd.nmx import Device  # noqa: E402
from nibblemac_amd.synth import QWEN35_08B  # noqa: E402

METRIC = "verified tok/s at draft k=4 (0.8B-shape Q4K); Q4K matvec GB/s vs HBM peak"
HBM_PEAK_GBS = 8000.0
N_VERIFY = 5  # k + 1


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def host_threads() -> int:
    return max(1, min(16, len(os.sched_getaffinity(0))))


class VerifyStream:
    """Device-resident weights and activations of one verify round's matmuls."""

    def __init__(self, dev: Device, shape=QWEN35_08B, seed: int = 5, keep_host: bool = True):
        self.dev, self.s = dev, shape
        self.layers = []          # per layer: list of (name, rows, cols, device W)
        self.host = {}            # (layer, name) -> host bytes (for the CPU baseline)
        thr = host_threads()
        t0 = time.time()
        stream = 0
        for l in range(shape.layers):
            mats = []
            for name, rows, cols in shape.layer_mats(l):
                W = pqtool.gauss_q4k(seed, stream, rows, cols, 0.02, thr)
                stream += 1
                mats.append((name, rows, cols, dev.to_device(W)))
                if keep_host:
                    self.host[(l, name)] = W
            self.layers.append(mats)
        self.head_host = pqtool.gauss_q4k(seed, 10_000, shape.vocab, shape.hidden, 0.02, thr)
        self.head = dev.to_device(self.head_host)
        self.head2 = dev.to_device(self.head_host)  # second copy: cold-cache rotation
        log(f"weights synthesised and uploaded in {time.time() - t0:.1f} s")
        rng = np.random.default_rng(seed)
        n = N_VERIFY
        self.X = {c: dev.to_device(rng.standard_normal((n, c)).astype(np.float32))
                  for c in {c for l in range(shape.layers) for _, _, c in shape.layer_mats(l)}}
        self.Xh = {c: x.numpy() for c, x in self.X.items()}
        self.A = {c: (dev.empty((c // 32, n, 32), np.int8), dev.empty((c // 32, n), np.float32),
                      dev.empty((c // 32, n), np.float32)) for c in self.X}
        maxrows = max(r for l in range(shape.layers) for _, r, _ in shape.layer_mats(l))
        self.Y = [dev.empty((n, maxrows), np.float32) for _ in range(4)]
        self.logits = dev.empty((n, shape.vocab), np.float32)
        self.drafts = dev.to_device(np.zeros(n - 1, np.int32))
        self.work = dev.zeros(dev.head_work_bytes(shape.vocab, n), np.uint8)
        self.out = dev.zeros(2 + n, np.int32)

    def bytes_per_step(self) -> int:
        n = N_VERIFY
        b = self.s.q4k_bytes()
        for l in range(self.s.layers):
            for _, rows, cols in self.s.layer_mats(l):
                b += n * cols + 2 * 4 * n * (cols // 32) + 4 * n * rows
        return b + n * self.s.hidden * 2 + 4 * (2 + n)

    def enqueue_step(self) -> None:
        dev, n = self.dev, N_VERIFY
        for c, (q, d, fs) in self.A.items():
            dev.quant_a8(self.X[c], n, c, q, d, fs)
        for mats in self.layers:
            by_cols: dict[int, list] = {}
            for name, rows, cols, W in mats:
                by_cols.setdefault(cols, []).append((rows, W))
            for cols, group in by_cols.items():
                q, d, fs = self.A[cols]
                for i in range(0, len(group), 4):
                    part = group[i:i + 4]
                    dev.q4k_matmul_multi([w for _, w in part], [r for r, _ in part],
                                         self.Y[:len(part)], [r for r, _ in part], cols, n, q, d, fs)
        q, d, fs = self.A[self.s.hidden]
        dev.head_accept(self.head, self.s.vocab, self.s.hidden, n, q, d, fs, None, self.drafts,
                        self.work, self.out)


def time_graph(dev: Device, g, reps: int) -> float:
    e0, e1 = dev.event(), dev.event()
    dev.record(e0)
    for _ in range(reps):
        dev.graph_launch(g)
    dev.record(e1)
    return dev.elapsed_ms(e0, e1)


def head_roofline(dev: Device, vs: VerifyStream, reps: int = 20) -> dict:
    """Q4K matvec of the LM head shape over 5 rows, logits materialised, two rotating copies."""
    s, n = vs.s, N_VERIFY
    q, d, fs = vs.A[s.hidden]
    dev.graph_begin()
    for r in range(reps):
        dev.q4k_matmul(vs.head if r % 2 == 0 else vs.head2, s.vocab, s.hidden, n, q, d, fs,
                       vs.logits)
    g = dev.graph_end()
    dev.graph_launch(g)
    dev.sync()
    ms = time_graph(dev, g, 1) / reps
    wbytes = s.vocab // 4 * (s.hidden // 256) * 576
    algo = wbytes + n * s.hidden + 2 * 4 * n * (s.hidden // 32) + 4 * n * s.vocab
    achieved = algo / (ms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
            "kernel": "q4k_mv_k<5> (LM head 248320x1024 Q4K x 5 rows, cold)",
            "us_per_launch": round(ms * 1e3, 2), "algorithmic_bytes": algo}


def cpu_baseline(vs: VerifyStream, budget_s: float = 20.0) -> dict:
    import oracle  # the checker / CPU baseline only

    s, n = vs.s, N_VERIFY
    thr = host_threads()
    A = {c: oracle.quant_a8(x) for c, x in vs.Xh.items()}

    def one_round(threads: int) -> float:
        t0 = time.perf_counter()
        for l in range(s.layers):
            for name, rows, cols in s.layer_mats(l):
                q, d, fs = A[cols]
                oracle.q4k_matmul(vs.host[(l, name)], rows, cols, q, d, fs, n, threads=threads)
        q, d, fs = A[s.hidden]
        Y = oracle.q4k_matmul(vs.head_host, s.vocab, s.hidden, q, d, fs, n, threads=threads)
        oracle.accept(Y, np.zeros(n - 1, np.int32))
        return time.perf_counter() - t0

    t1 = one_round(1)
    tn, rounds = 0.0, 0
    while tn < budget_s / 2 and rounds < 8:
        tn += one_round(thr)
        rounds += 1
    gb = vs.bytes_per_step() / 1e9
    return {"value": round(gb * rounds / tn, 2), "unit": "GB/s", "cores": thr, "kind": "port",
            "value_1thread": round(gb / t1, 3),
            "sample": f"oracle Q4K x A8 over one verify round's weight stream (24 layers + head, "
                      f"5 rows): {rounds} round(s) on {thr} threads, 1 round on 1 thread"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {a.gpus} is not supported "
              "(the multi-GPU sharding is a design, not a measured path)", file=sys.stderr)
        return 2
    with Device(0) as dev:
        log(f"device {dev.name}")
        vs = VerifyStream(dev)
        dev.graph_begin()
        vs.enqueue_step()
        g = dev.graph_end()
        for _ in range(max(a.warmup, 1)):
            dev.graph_launch(g)
        dev.sync()
        ms = time_graph(dev, g, a.steps) / a.steps
        dev.sync()
        gbs = vs.bytes_per_step() / (ms * 1e-3) / 1e9
        log(f"verify weight stream: {ms * 1e3:.1f} us/step, {gbs:.0f} GB/s")
        roof = head_roofline(dev, vs)
        log(f"head matvec: {roof['us_per_launch']} us/launch, {roof['achieved']} GB/s")
        cpu = None if a.no_cpu else cpu_baseline(vs)
    rec = {
        "metric": METRIC, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": a.steps, "warmup": a.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8xq4+fp32",
        "data": "synthetic (random-init N(0,0.02) weights packed Q4K, N(0,1) activations)",
        "config": {"workload": "k=4 verify round Q4K weight stream, 0.8B shape (24 layers + "
                               "248320x1024 head, 5 rows, fused argmax+acceptance)",
                   "model": "qwen3.5-0.8b-shape-q4k", "global_batch": N_VERIFY,
                   "parallelism": "single-gpu"},
        "roofline": roof, "cpu_baseline": cpu,
    }
    print(json.dumps(rec), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
