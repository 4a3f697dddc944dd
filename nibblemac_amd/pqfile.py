""".pq model files (engine/FORMAT.md): the header / directory layout and a writer for seeded
synthetic random-init Qwen3.5-hybrid models whose matrices are Q4K_G32.

Layout (FORMAT.md "Layout"): a 4096-byte header, the tensor directory (128-byte entries), then
tensor data from a 4096-aligned data_offset, every tensor 64-byte aligned. Norm vectors are
stored as the effective multiplier (1 + w); the gated-norm weight is stored as is.
"""
from __future__ import annotations

import os
import struct
from dataclasses import replace
from pathlib import Path

import numpy as np

from . import pqtool
from .synth import QWEN35_08B, Shape

MAGIC = b"PINFERQ\0"
HEADER_FMT = "<8sIIQQ" + "I" * 18 + "ff"   # the header struct of engine/FORMAT.md
ENTRY_FMT = "<80sII4IQQ8x"                 # one 128-byte directory entry
F32, BF16, Q4K = 0, 1, 4


def tensors(shape: Shape, seed: int, random_norms: bool, mtp: bool = True,
            lm_head: tuple[int, float] | None = None):
    """(name, dtype, dims, producer) for every tensor the engine maps, in file order. Matrices
    are N(0, 0.02) packed as Q4K; norms 1 (or U(0.8, 1.2) with random_norms); conv weights
    U(-0.5, 0.5); A_log / dt_bias so that the decay exp(-exp(A_log) softplus(a + dt_bias))
    stays in (0.9, 1) for |a| up to ~3. lm_head = (rows, std): an untied output head whose
    first `rows` rows are N(0, 0.02) and the others N(0, std)."""
    rng = np.random.default_rng(seed)
    H, F = shape.hidden, shape.ffn
    stream = [0]
    out = []

    def mat(name, rows, cols):
        s = stream[0]
        stream[0] += 1
        out.append((name, Q4K, [rows, cols],
                    lambda r=rows, c=cols, s=s: pqtool.gauss_q4k(seed, s, r, c, 0.02)))

    def vec(name, dims, lo=None, hi=None, value=None):
        if value is not None:
            data = np.full(dims, value, np.float32)
        else:
            data = rng.uniform(lo, hi, dims).astype(np.float32)
        out.append((name, F32, list(dims), lambda d=data: d))

    def norm(name, n):
        if random_norms:
            vec(name, [n], 0.8, 1.2)
        else:
            vec(name, [n], value=1.0)

    def block(p, is_full):
        norm(p + "input_layernorm.weight", H)
        norm(p + "post_attention_layernorm.weight", H)
        mat(p + "mlp.gate_proj.weight", F, H)
        mat(p + "mlp.up_proj.weight", F, H)
        mat(p + "mlp.down_proj.weight", H, F)
        if is_full:
            hd = shape.head_dim
            mat(p + "self_attn.q_proj.weight", shape.n_heads * hd * 2, H)
            mat(p + "self_attn.k_proj.weight", shape.n_kv * hd, H)
            mat(p + "self_attn.v_proj.weight", shape.n_kv * hd, H)
            mat(p + "self_attn.o_proj.weight", H, shape.n_heads * hd)
            norm(p + "self_attn.q_norm.weight", hd)
            norm(p + "self_attn.k_norm.weight", hd)
            return
        nv = shape.lin_v_heads
        mat(p + "linear_attn.in_proj_qkv.weight", shape.conv_dim, H)
        mat(p + "linear_attn.in_proj_z.weight", shape.vd, H)
        mat(p + "linear_attn.in_proj_b.weight", nv, H)
        mat(p + "linear_attn.in_proj_a.weight", nv, H)
        mat(p + "linear_attn.out_proj.weight", H, shape.vd)
        vec(p + "linear_attn.A_log", [nv], np.log(0.2), np.log(0.4))
        vec(p + "linear_attn.dt_bias", [nv], -4.5, -3.5)
        if random_norms:
            vec(p + "linear_attn.norm.weight", [shape.lin_v_dim], 0.8, 1.2)
        else:
            vec(p + "linear_attn.norm.weight", [shape.lin_v_dim], value=1.0)
        vec(p + "linear_attn.conv1d.weight", [shape.conv_dim, shape.conv_k], -0.5, 0.5)

    mat("embed_tokens.weight", shape.vocab, H)
    if lm_head:
        hot, std = lm_head
        if hot % 4 or not 0 < hot < shape.vocab:
            raise ValueError(f"lm_head rows {hot}: a multiple of 4 inside the vocabulary")
        s = 1 << 20  # streams of their own: every other tensor keeps its values
        out.append(("lm_head.weight", Q4K, [shape.vocab, H], lambda s=s: np.concatenate(
            [pqtool.gauss_q4k(seed, s, hot, H, 0.02),
             pqtool.gauss_q4k(seed, s + 1, shape.vocab - hot, H, std)])))
    norm("norm.weight", H)
    for i in range(shape.layers):
        block(f"layers.{i}.", shape.is_full(i))
    if mtp:
        mat("mtp.fc.weight", H, 2 * H)
        for n in ("pre_fc_norm_embedding", "pre_fc_norm_hidden", "norm"):
            norm(f"mtp.{n}.weight", H)
        block("mtp.layers.0.", True)
    return out


def nbytes(dtype: int, dims: list[int]) -> int:
    if dtype == Q4K:
        return dims[0] // 4 * (dims[1] // 256) * 576
    return int(np.prod(dims)) * (4 if dtype == F32 else 2)


def write_model(path: str | os.PathLike, shape: Shape = QWEN35_08B, seed: int = 1,
                random_norms: bool = False, mtp: bool = True,
                overrides: dict[str, np.ndarray] | None = None,
                lm_head: tuple[int, float] | None = None) -> Path:
    """Write a synthetic model; returns the path. `overrides` replaces the values of named F32
    tensors (same element count); `lm_head` writes an untied output head (see tensors)."""
    path = Path(path)
    ts = tensors(shape, seed, random_norms, mtp, lm_head)
    for name, value in (overrides or {}).items():
        i = next((i for i, t in enumerate(ts) if t[0] == name), None)
        if i is None or ts[i][1] != F32:
            raise ValueError(f"override {name}: no F32 tensor of that name")
        data = np.ascontiguousarray(value, np.float32).reshape(ts[i][2])
        ts[i] = (name, F32, ts[i][2], lambda d=data: d)
    mask = sum(1 << i for i in range(shape.layers) if shape.is_full(i))
    dir_off = 4096
    data_off = -(-(dir_off + 128 * len(ts)) // 4096) * 4096
    offs, off = [], data_off
    for _, dt, dims, _ in ts:
        offs.append(off)
        off = -(-(off + nbytes(dt, dims)) // 64) * 64
    hdr = struct.pack(HEADER_FMT, MAGIC, 1, len(ts), dir_off, data_off, 1, shape.hidden,
                      shape.layers, shape.vocab, shape.ffn, shape.n_heads, shape.n_kv,
                      shape.head_dim, shape.rot, shape.lin_k_heads, shape.lin_v_heads,
                      shape.lin_k_dim, shape.lin_v_dim, shape.conv_k, mask, shape.eos_id,
                      0 if lm_head else 1,
                      1 if mtp else 0, shape.rms_eps, shape.rope_theta)
    with path.open("wb") as f:
        f.write(hdr.ljust(4096, b"\0"))
        for (name, dt, dims, _), o in zip(ts, offs):
            d4 = dims + [0] * (4 - len(dims))
            f.write(struct.pack(ENTRY_FMT, name.encode(), dt, len(dims), *d4, o, nbytes(dt, dims)))
        for (name, dt, dims, make), o in zip(ts, offs):
            f.write(b"\0" * (o - f.tell()))
            data = make()
            assert data.nbytes == nbytes(dt, dims), name
            f.write(data.tobytes())
    return path


def agreeing_norm(hidden: int, j: int = 2) -> np.ndarray:
    """A final-norm weight vector that keeps (almost) only hidden coordinate j: the logits are
    then about x_j * head[:, j], so the main model and the MTP head (both read through the same
    head) pick one of the same two tokens, by the sign of their x_j, and MTP drafts are often
    accepted. Pass it as the override of both "norm.weight" and "mtp.norm.weight". When the
    drafts are restricted to the first rows of the head, write an untied head whose other rows
    are small (write_model's lm_head), so that the main model's choice lies among them too."""
    w = np.full(hidden, 1e-3, np.float32)
    w[j] = 1.0
    return w


SMALL = replace(QWEN35_08B, hidden=256, layers=4, ffn=768, vocab=2048, n_heads=4, n_kv=2,
                head_dim=64, rot=16, lin_k_heads=2, lin_v_heads=4, lin_k_dim=64, lin_v_dim=64,
                eos_id=2047)
"""A small model with the 0.8B layer pattern (3 Gated DeltaNet + 1 full attention), GQA 2:1,
lin_v_heads = 2 lin_k_heads: the kernels' every dimension relation at test size."""
