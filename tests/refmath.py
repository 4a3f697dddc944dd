"""Exact arithmetic helpers for pinning the oracle: binary32 rounding of exact rationals (so a
fused multiply-add can be evaluated with one rounding), the Q4K layout written from the format
description (engine/FORMAT.md:107-136) independently of the oracle's C code, and brute-force
integer references."""
from __future__ import annotations

from fractions import Fraction

import numpy as np


def round_f32(x: Fraction) -> np.float32:
    """Round an exact rational to the nearest binary32, ties to even (normal and subnormal)."""
    if x == 0:
        return np.float32(0.0)
    sign = -1 if x < 0 else 1
    a = -x if x < 0 else x
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    if Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, -126)                  # subnormal range keeps the 2^-149 quantum
    q = Fraction(2) ** (e - 23)       # ulp at this exponent
    m = a / q
    lo = m.numerator // m.denominator
    rem = m - lo
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and lo % 2 == 1):
        lo += 1
    val = Fraction(lo) * q
    if val >= Fraction(2) ** 128:
        return np.float32(sign * np.inf)
    return np.float32(sign * float(val))


def fma32(a, b, c) -> np.float32:
    """fmaf(a, b, c) with a single rounding."""
    return round_f32(Fraction(float(np.float32(a))) * Fraction(float(np.float32(b))) +
                     Fraction(float(np.float32(c))))


def put6(values) -> bytes:
    """32 six-bit values -> 24 bytes (FORMAT.md: byte j < 16 holds values j (low nibble) and
    j + 16 (high nibble); byte 16 + j holds bits 4..5 of values j, j+8, j+16, j+24)."""
    v = [int(x) for x in values]
    out = bytearray(24)
    for j in range(16):
        out[j] = (v[j] & 15) | ((v[j + 16] & 15) << 4)
    for j in range(8):
        out[16 + j] = (v[j] >> 4) | ((v[j + 8] >> 4) << 2) | ((v[j + 16] >> 4) << 4) | ((v[j + 24] >> 4) << 6)
    return bytes(out)


def pack_superblock(D, M, s, m, codes) -> bytes:
    """One Q4K_G32 superblock: D[4], M[4] (floats, stored fp16), s[8][4], m[8][4] (6-bit, [block]
    [row]), codes[4][256] (0..15, [row][col]) -> 576 bytes."""
    line = bytearray(64)
    line[0:8] = np.asarray(D, np.float16).tobytes()
    line[8:16] = np.asarray(M, np.float16).tobytes()
    line[16:40] = put6(np.asarray(s).reshape(32))   # index 4k + i
    line[40:64] = put6(np.asarray(m).reshape(32))
    body = bytearray(512)
    for k in range(8):
        for i in range(4):
            for j in range(16):
                body[64 * k + 16 * i + j] = codes[i][32 * k + j] | (codes[i][32 * k + j + 16] << 4)
    return bytes(line + body)


def unpack_q4k(W: np.ndarray, rows: int, cols: int):
    """-> (u [rows][cols] nibbles, s, m [rows][cols/32] 6-bit, D, M [rows][cols/256] float32),
    decoded with numpy straight from the byte layout."""
    nsb = cols // 256
    sb = W.reshape(rows // 4, nsb, 576)
    D = sb[:, :, 0:8].copy().view(np.float16).astype(np.float32)      # [t][sb][4]
    M = sb[:, :, 8:16].copy().view(np.float16).astype(np.float32)

    def get6(arr):  # arr [t][sb][24] -> [t][sb][32]
        lo = np.concatenate([arr[..., :16] & 15, arr[..., :16] >> 4], axis=-1).astype(np.int32)
        j = np.arange(32)
        hi = (arr[..., 16 + j % 8] >> (2 * (j // 8))) & 3
        return lo | (hi.astype(np.int32) << 4)

    s = get6(sb[:, :, 16:40]).reshape(rows // 4, nsb, 8, 4)   # [t][sb][k][i]
    m = get6(sb[:, :, 40:64]).reshape(rows // 4, nsb, 8, 4)
    body = sb[:, :, 64:].reshape(rows // 4, nsb, 8, 4, 16)   # [t][sb][k][i][j]
    lo, hi = body & 15, body >> 4
    u = np.concatenate([lo, hi], axis=-1)                    # [t][sb][k][i][32]
    u = u.transpose(0, 3, 1, 2, 4).reshape(rows, cols)
    s = s.transpose(0, 3, 1, 2).reshape(rows, cols // 32)
    m = m.transpose(0, 3, 1, 2).reshape(rows, cols // 32)
    D = D.transpose(0, 2, 1).reshape(rows, nsb)
    M = M.transpose(0, 2, 1).reshape(rows, nsb)
    return u.astype(np.int64), s, m, D, M


def state_offsets(heads: int, dk: int, dv: int) -> np.ndarray:
    """Offsets [h][j][i] of the DeltaNet state element (head h, value column j, key i) in the
    device layout, restated from its description in include/nmx.h: per head the columns in
    groups of 16, and within a group of W columns the float4 slot k (keys 4k .. 4k + 3 of a
    quarter c of dk/4 keys) of every lane 4 (j mod 16) + c contiguous."""
    dk4 = dk // 4
    h = np.arange(heads)[:, None, None]
    j = np.arange(dv)[None, :, None]
    i = np.arange(dk)[None, None, :]
    g = j // 16
    w = np.minimum(16, dv - 16 * g)
    lane = 4 * (j % 16) + i // dk4
    k = (i % dk4) // 4
    return (h * dv + 16 * g) * dk + (k * 4 * w + lane) * 4 + i % 4


def state_to_dev(S, heads: int, dk: int, dv: int) -> np.ndarray:
    """oracle layout [h][dk][dv] -> the device layout (flat)."""
    out = np.empty(heads * dk * dv, np.float32)
    out[state_offsets(heads, dk, dv)] = np.asarray(S, np.float32).reshape(heads, dk, dv).transpose(0, 2, 1)
    return out


def state_from_dev(S, heads: int, dk: int, dv: int) -> np.ndarray:
    """the device layout (flat) -> oracle layout [h][dk][dv]."""
    flat = np.asarray(S, np.float32).ravel()
    return np.ascontiguousarray(flat[state_offsets(heads, dk, dv)].transpose(0, 2, 1))
