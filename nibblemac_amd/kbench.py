"""Kernel-level measurements of the verify path on one GPU (the role of the reference's
engine/bench/kbench.c:184-223 and lbench.c:131-210): each config's kernels timed with HIP events
on the stream they run on, over HIP-graph replays, warm (the same weights every launch) and
cold (rotating copies whose total exceeds the 256 MB MALL, so no launch finds its weights in any
cache). Weights are seeded Gaussians N(0, 0.02) packed as Q4K_G32 (include/pqtool.h);
activations N(0, 1).

Algorithmic bytes per unit (what a launch must move at least once):
  Q4K matvec   rows * cols * 0.5625 weight bytes + n * cols * 1.25 A8 bytes (codes + d + fsum
               per 32 columns) + n * rows * 4 output bytes
  DeltaNet     state read + write (2 * heads * dk * dv * 4) + log rows + q/k/v in + o out
  LM head      the matvec bytes with the logits replaced by ~40 B of (a, bonus, tokens)
"""
from __future__ import annotations

import numpy as np

from . import pqtool
from .nmx import A8, Device, LinArgs, LinMixArgs, LinPreArgs
from .synth import QWEN35_08B

HBM_PEAK_GBS = 8000.0
MALL_BYTES = 256 << 20


def q4k_bytes(rows: int, cols: int) -> int:
    return rows // 4 * (cols // 256) * 576


def matvec_algo_bytes(rows: int, cols: int, n: int, out: bool = True) -> int:
    return q4k_bytes(rows, cols) + n * cols + 2 * 4 * n * (cols // 32) + (4 * n * rows if out else 0)


EAGER = False  # stream launches instead of graph replays (profiler counter runs)


def _time_graph(dev: Device, launches, reps: int) -> float:
    """ms per replay of a graph of `launches` (captured once, replayed after one warm-up), or
    per round of stream launches when EAGER."""
    if EAGER:
        launches()
        dev.sync()
        e0, e1 = dev.event(), dev.event()
        dev.record(e0)
        for _ in range(reps):
            launches()
        dev.record(e1)
        dev.sync()
        return dev.elapsed_ms(e0, e1) / reps
    dev.graph_begin()
    launches()
    g = dev.graph_end()
    dev.graph_launch(g)
    dev.sync()
    e0, e1 = dev.event(), dev.event()
    dev.record(e0)
    for _ in range(reps):
        dev.graph_launch(g)
    dev.record(e1)
    dev.sync()
    ms = dev.elapsed_ms(e0, e1) / reps
    dev.graph_destroy(g)
    return ms


def _copies(dev: Device, host: np.ndarray, total_min: int, at_least: int = 1):
    n = max(at_least, -(-total_min // host.nbytes))
    return [dev.to_device(host) for _ in range(n)]


def _time_stream(dev: Device, launches, reps: int) -> float:
    """ms per round of `launches` issued back to back on the stream (after one warm-up round),
    between two HIP events on that stream."""
    launches()
    dev.sync()
    e0, e1 = dev.event(), dev.event()
    dev.record(e0)
    for _ in range(reps):
        launches()
    dev.record(e1)
    dev.sync()
    return dev.elapsed_ms(e0, e1) / reps


def _a8(dev: Device, rng, n: int, cols: int):
    X = dev.to_device(rng.standard_normal((n, cols)).astype(np.float32))
    q = dev.empty((cols // 32, n, 32), np.int8)
    d = dev.empty((cols // 32, n), np.float32)
    fs = dev.empty((cols // 32, n), np.float32)
    dev.quant_a8(X, n, cols, q, d, fs)
    return q, d, fs


def _line(algo: int, us: float) -> dict:
    gbs = algo / (us * 1e-6) / 1e9
    return {"us": round(us, 3), "GB_s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}


def config1_matvec(dev: Device, rows: int = 3584, cols: int = 1024, n: int = 1,
                   reps_per_graph: int = 150, graphs: int = 20) -> dict:
    """Config 1: one Q4K x A8 matvec 3584 x 1024 at n = 1 (nmx_q4k_matmul), warm and cold
    (>= 150 rotating copies, > 300 MB)."""
    rng = np.random.default_rng(1)
    W = pqtool.gauss_q4k(1, 0, rows, cols, 0.02)
    q, d, fs = _a8(dev, rng, n, cols)
    Y = dev.empty((n, rows), np.float32)
    cold = _copies(dev, W, 300 << 20, at_least=150)
    warm = cold[:1]

    def run(ws):
        def launches():
            for r in range(reps_per_graph):
                dev.q4k_matmul(ws[r % len(ws)], rows, cols, n, q, d, fs, Y)
        return _time_graph(dev, launches, graphs) / reps_per_graph * 1e3

    algo = matvec_algo_bytes(rows, cols, n)
    out = {"shape": f"{rows}x{cols} Q4K x {n} A8 row(s)", "algorithmic_bytes": algo,
           "kernel": "q4k_mt_k<1> (nmx_q4k_matmul)",
           "warm": _line(algo, run(warm)),
           "cold": dict(_line(algo, run(cold)), copies=len(cold),
                        arena_mb=round(len(cold) * W.nbytes / 1e6, 1))}
    for b in cold:
        b.free()
    return out


LIN_SHAPES = {  # the 0.8B shape's per-layer matmuls (rows, cols)
    "qkv": (6144, 1024), "z": (2048, 1024), "b": (16, 1024), "a": (16, 1024),
    "out": (1024, 2048), "gate": (3584, 1024), "up": (3584, 1024), "down": (1024, 3584),
}
ATTN_SHAPES = {
    "q": (4096, 1024), "k": (512, 1024), "v": (512, 1024), "o": (1024, 2048),
    "gate": (3584, 1024), "up": (3584, 1024), "down": (1024, 3584),
}


def config2_layer(dev: Device, n: int = 5, graphs: int = 10) -> dict:
    """Config 2: one decoder layer's Q4K matmuls at n = k + 1 = 5, as the verify pass launches
    them (DeltaNet: qkv/z/b/a in one launch, out, gate/up with the SwiGLU + A8 epilogue, down;
    full attention: q/k/v in one launch, o, gate/up, down), over copies of the layer rotating
    through > 300 MB (cold), timed per layer."""
    s = QWEN35_08B
    H, F = s.hidden, s.ffn
    rng = np.random.default_rng(2)
    res = {}
    for kind, shapes in (("deltanet", LIN_SHAPES), ("full_attention", ATTN_SHAPES)):
        host = {k: pqtool.gauss_q4k(2, i, r, c, 0.02) for i, (k, (r, c)) in enumerate(shapes.items())}
        wbytes = sum(v.nbytes for v in host.values())
        ncopy = max(2, -(-(300 << 20) // wbytes))
        layers = [{k: dev.to_device(v) for k, v in host.items()} for _ in range(ncopy)]
        wide = 2048
        a_h, a_w, a_f = _a8(dev, rng, n, H), _a8(dev, rng, n, wide), _a8(dev, rng, n, F)
        first = ["qkv", "z", "b", "a"] if kind == "deltanet" else ["q", "k", "v"]
        Ys = [dev.empty((n, shapes[k][0]), np.float32) for k in first]
        yo = dev.empty((n, H), np.float32)
        tg, tu = dev.empty((n, F), np.float32), dev.empty((n, F), np.float32)
        o_name = "out" if kind == "deltanet" else "o"

        def launches():
            for L in layers:
                dev.q4k_matmul_multi([L[k] for k in first], [shapes[k][0] for k in first], Ys,
                                     [shapes[k][0] for k in first], H, n, *a_h)
                dev.q4k_matmul(L[o_name], H, wide, n, *a_w, yo)
                dev.q4k_swiglu(L["gate"], L["up"], F, H, n, a_f, a8=a_h, a8_tmp=a_h, gate_tmp=tg,
                               up_tmp=tu)
                dev.q4k_matmul(L["down"], H, F, n, *a_f, yo)

        us = _time_graph(dev, launches, graphs) / ncopy * 1e3
        algo = wbytes + sum(n * c + 8 * n * (c // 32) + 4 * n * r for r, c in shapes.values())
        res[kind] = dict(_line(algo, us), weight_bytes=wbytes, algorithmic_bytes=algo,
                         launches_per_layer=4, copies=ncopy)
        # the same over copies that fit the MALL (about 160 MB: above the L2s, below 256 MB)
        full = layers
        layers = full[:max(2, (160 << 20) // wbytes)]
        us_m = _time_graph(dev, launches, graphs) / len(layers) * 1e3
        res[kind]["mall_resident"] = dict(_line(algo, us_m), copies=len(layers))
        layers = full
        for L in layers:
            for b in L.values():
                b.free()
    res["rows"] = n
    res["kernel"] = "q4k_mt_k<5,...> (nmx_q4k_matmul_multi / nmx_q4k_matmul / nmx_q4k_swiglu)"
    return res


def config3_deltanet(dev: Device, n: int = 5, layers: int = 18, graphs: int = 20) -> dict:
    """Config 3: the fused Gated DeltaNet mixer of one verify pass (nmx_lin_mix: conv + gates +
    L2 norms + the recurrence with the deferred replay of `keep` pending rows and the per-token
    log + gated RMSNorm + A8) at 16 heads x dk = dv = 128, n = 5, over 18 layers' states in
    turn, per layer-pass; keep = 0 (nothing accepted last round) and 4 (all accepted)."""
    heads, dk, dv, K = 16, 128, 128, 4
    C = 2 * heads * dk + heads * dv
    cap = 5
    rng = np.random.default_rng(3)

    def f32(*shape, scale=1.0):
        return dev.to_device((rng.standard_normal(shape) * scale).astype(np.float32))

    raw, z = f32(n, C), f32(n, heads * dv)
    b, a = f32(n, heads), f32(n, heads, scale=2.0)
    A_log = dev.to_device(rng.uniform(np.log(0.2), np.log(0.4), heads).astype(np.float32))
    dt = dev.to_device(rng.uniform(-4.5, -3.5, heads).astype(np.float32))
    conv_w = dev.to_device(rng.uniform(-0.5, 0.5, (C, K)).astype(np.float32))
    norm_w = dev.to_device(rng.uniform(0.5, 1.5, dv).astype(np.float32))
    pend_h = (rng.standard_normal((cap, heads, dk + dv + 1)) * 0.1).astype(np.float32)
    pend_h[:, :, dk + dv] = rng.uniform(0.9, 1.0, (cap, heads))
    st = [dict(S=f32(heads, dv, dk, scale=0.05), state=f32(K - 1, C), xin=dev.zeros((cap, C), np.float32),
               log=dev.zeros((cap, heads, dk + dv + 1), np.float32), pend=dev.to_device(pend_h))
          for _ in range(layers)]
    conv, beta, decay = dev.zeros((n, C), np.float32), dev.zeros((n, heads), np.float32), \
        dev.zeros((n, heads), np.float32)
    o, y = dev.zeros((n, heads * dv), np.float32), dev.zeros((n, heads * dv), np.float32)
    nb = heads * dv // 32
    aq, ad, afs = dev.zeros((nb, n, 32), np.int8), dev.zeros((nb, n), np.float32), \
        dev.zeros((nb, n), np.float32)
    res = {"shape": f"{heads} heads x dk {dk} x dv {dv}, {n} tokens, logged",
           "kernel": "lin_mix_k<32> (nmx_lin_mix)"}
    for keep in (0, 4):
        def launches():
            for L in st:
                pre = LinPreArgs(n, C, K, dk, heads * dk, raw.ptr, C, conv.ptr, L["state"].ptr,
                                 conv_w.ptr, L["xin"].ptr, np.float32(1 / np.sqrt(dk)), 1e-6, b.ptr,
                                 a.ptr, heads, heads, A_log.ptr, None, dt.ptr, beta.ptr, decay.ptr)
                rule = LinArgs(n, heads, 1, dk, dv, C, heads * dv, conv.ptr, decay.ptr, beta.ptr,
                               L["S"].ptr, o.ptr, L["log"].ptr, L["pend"].ptr, keep, 0, None)
                dev.lin_mix(LinMixArgs(pre, rule, z.ptr, heads * dv, norm_w.ptr, 1e-6, y.ptr,
                                       heads * dv, A8(aq.ptr, ad.ptr, afs.ptr)))

        us = _time_graph(dev, launches, graphs) / layers * 1e3
        algo = (2 * heads * dk * dv * 4 + (n - 1 + keep) * heads * (dk + dv + 1) * 4
                + n * C * 4 + 2 * n * heads * dv * 4 + n * heads * dv * 1.25)
        res[f"keep{keep}"] = dict(_line(int(algo), us), algorithmic_bytes=int(algo))
    for L in st:
        for v in L.values():
            v.free()
    return res


def config4_head(dev: Device, n: int = 5, copies: int = 4, reps_per_graph: int = 8,
                 graphs: int = 5) -> dict:
    """Config 4: the LM head 248320 x 1024 over k + 1 = 5 A8 rows with the fused argmax and the
    acceptance of the 4 drafts.

    in_path_cold / in_path_warm: the head launch of the verify round (nmx_head_keys: the
    matvec q4k_head_k<5,4,16>, leaving 243 partial argmax keys per row, whose reduction and
    acceptance run inside the round's commit workgroups), over `copies` rotating copies of the
    head (4 x 143 MB, so no launch finds it in the 256 MB MALL), and over one copy (resident in
    the MALL after the first launch). accept<a>of4: the single-call API (nmx_head_accept: the
    same matvec, then head_finish_k's reduction and acceptance), cold, with the acceptance rate
    swept 0 / 50 / 100 % by planting drafts; the outputs are checked against the planted
    answers, and the in-path keys against the same argmax."""
    s = QWEN35_08B
    rows, cols = s.vocab, s.hidden
    rng = np.random.default_rng(4)
    W = pqtool.gauss_q4k(7, 10_000, rows, cols, 0.02)
    heads = [dev.to_device(W) for _ in range(copies)]
    q, d, fs = _a8(dev, rng, n, cols)
    work = dev.alloc(dev.head_work_bytes(rows, n))
    out = dev.zeros(2 + 64, np.int32)
    logits = dev.empty((n, rows), np.float32)
    drafts = dev.zeros(n - 1, np.int32)
    dev.head_accept(heads[0], rows, cols, n, q, d, fs, logits, drafts, work, out)
    dev.sync()
    am = logits.numpy().argmax(axis=1)  # first maximum per row (numpy's argmax)
    res = {"shape": f"{rows}x{cols} Q4K x {n} A8 rows, fused argmax + acceptance of {n - 1} drafts",
           "kernel": "q4k_mvx_k<5,true> + head_finish_k (nmx_head_accept)", "copies": copies}
    algo = matvec_algo_bytes(rows, cols, n, out=False) + 4 * (n - 1) + 4 * (2 + n)
    res["algorithmic_bytes"] = algo
    for a_plant in (0, 2, 4):
        dr = np.array([am[t] if t < a_plant else (am[t] + 1) % rows for t in range(n - 1)],
                      np.int32)
        dev.upload(drafts, dr)

        def launches():
            for r in range(reps_per_graph):
                dev.head_accept(heads[r % copies], rows, cols, n, q, d, fs, None, drafts, work, out)

        us = _time_graph(dev, launches, graphs) / reps_per_graph * 1e3
        got = out.numpy()[:2]
        if int(got[0]) != a_plant or int(got[1]) != int(am[a_plant]):
            raise RuntimeError(f"head acceptance: planted a={a_plant}, got {got.tolist()}")
        res[f"accept{a_plant}of{n - 1}"] = _line(algo, us)
    # the round's head launch: keys only, the drafts copied for the commit's acceptance
    dcopy = dev.zeros(16, np.int32)
    nk = dev.head_nkeys(rows, cols, n)
    algo_k = matvec_algo_bytes(rows, cols, n, out=False) + 2 * 4 * (n - 1)
    res["in_path_algorithmic_bytes"] = algo_k
    res["in_path_kernel"] = f"q4k_head_k<{n},{cols // 256},16> (nmx_head_keys, {nk} keys per row)"
    for name, ncp in (("in_path_cold", copies), ("in_path_warm", 1)):
        def launches_k():
            for r in range(reps_per_graph):
                dev.head_keys(heads[r % ncp], rows, cols, n, q, d, fs, drafts, work, dcopy)

        # back-to-back stream launches: the kernel's own duration (what a kernel trace
        # reports), and graph replays: with the graph node's launch cost the round pays
        us = _time_stream(dev, launches_k, graphs) / reps_per_graph * 1e3
        usg = _time_graph(dev, launches_k, graphs) / reps_per_graph * 1e3
        keys = dev.download(work, np.uint64, (n, nk))
        top = keys.max(axis=1)
        idx = (0xffffffff - (top & 0xffffffff)).astype(np.int64)
        if not np.array_equal(idx, am):
            raise RuntimeError(f"head keys: argmax {idx.tolist()} != {am.tolist()}")
        res[name] = dict(_line(algo_k, us), us_graph_replay=round(usg, 3))
    dcopy.free()
    for b in heads:
        b.free()
    work.free()
    return res


def run_all(dev: Device) -> dict:
    return {"config1_matvec": config1_matvec(dev), "config2_layer": config2_layer(dev),
            "config3_deltanet": config3_deltanet(dev), "config4_head": config4_head(dev)}
