/* ORACLE — test infrastructure only (see oracle.h). Scalar numeric primitives. */
#include <math.h>
#include <string.h>

#include "oracle.h"

/* binary32 -> binary16, round to nearest even with subnormals (the conversion __fp16 casts
 * perform in engine/bench/kbench_util.c:117 and engine/src/forward_kv.c:35-59). */
uint16_t orc_f32_to_f16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    const uint32_t sign = (u >> 16) & 0x8000u, e32 = (u >> 23) & 0xffu;
    uint32_t man = u & 0x7fffffu;
    const int exp = (int)e32 - 127 + 15;
    if (e32 == 0xffu) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u | (man >> 13) : 0));
    if (exp >= 31) return (uint16_t)(sign | 0x7c00u);
    if (exp <= 0) {
        if (exp < -10) return (uint16_t)sign;
        man |= 0x800000u;
        const uint32_t shift = (uint32_t)(14 - exp), half = 1u << (shift - 1);
        uint32_t h = man >> shift;
        const uint32_t rem = man & ((1u << shift) - 1);
        if (rem > half || (rem == half && (h & 1))) h++;
        return (uint16_t)(sign | h);
    }
    uint32_t h = sign | ((uint32_t)exp << 10) | (man >> 13);
    const uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1))) h++;
    return (uint16_t)h;
}

float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu, u;
    if (exp == 0) {
        if (!man) {
            u = sign;
        } else {
            int s = 0;
            while (!(man & 0x400u)) { man <<= 1; s++; }
            u = sign | ((uint32_t)(113 - s) << 23) | ((man & 0x3ffu) << 13);
        }
    } else if (exp == 31) {
        u = sign | 0x7f800000u | (man << 13);
    } else {
        u = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* First index of the maximum (engine/src/forward_ops.c:387-409): pass 1 finds the maximum
 * with `>` (so the first of equal values is kept), pass 2 returns the first i with v[i] ==
 * max; -0 == +0, so the earliest zero of either sign wins. */
int orc_argmax(const float *v, int n) {
    if (!v || n <= 0) return -1;
    float mx = v[0];
    for (int i = 1; i < n; i++)
        if (v[i] > mx) mx = v[i];
    for (int i = 0; i < n; i++)
        if (v[i] == mx) return i;
    return 0;
}

/* Acceptance of one verify pass (engine/src/spec.c:340-345): a = 0, g = argmax(row 0);
 * while a < k and the draft for row a + 1 equals g: a++, g = argmax(row a). */
int orc_accept(const float *logits, int V, const int32_t *drafts, int k, int32_t *bonus,
               int32_t *argmax_rows) {
    if (argmax_rows)
        for (int t = 0; t <= k; t++) argmax_rows[t] = orc_argmax(logits + (size_t)t * V, V);
    int a = 0, g = orc_argmax(logits, V);
    while (a < k && drafts[a] == g) {
        a++;
        g = orc_argmax(logits + (size_t)a * V, V);
    }
    if (bonus) *bonus = g;
    return a;
}

/* pf_expf (engine/src/forward_ops.c:26-56): clamp, ln2 range reduction in two parts,
 * degree-6 polynomial, exponent assembled from the integer part; no fused operations. */
float orc_expf_cephes(float x) {
    x = x < -87.0f ? -87.0f : x > 88.0f ? 88.0f : x;
    const float fx = rintf(x * 1.44269504088896341f);
    float r = x - fx * 0.693145751953125f;
    r = r - fx * 1.428606765330187e-06f;
    float p = 1.9875691500e-4f;
    p = p * r + 1.3981999507e-3f;
    p = p * r + 8.3334519073e-3f;
    p = p * r + 4.1665795894e-2f;
    p = p * r + 1.6666665459e-1f;
    p = p * r + 5.0000001201e-1f;
    float y = p * (r * r) + r;
    y = y + 1.0f;
    const uint32_t bits = (uint32_t)((int)fx + 127) << 23;
    float s;
    memcpy(&s, &bits, 4);
    return y * s;
}

/* top1_prob (engine/src/spec.c:93-97): mx = max (pf_softmax_max: greater-than scan, any order
 * gives the same value); s = sum of pf_expf(l_i - mx) as pf_softmax_exp forms it: partial
 * sum j over e[4m + j] for the first n / 4 * 4 elements, s = (c0 + c1) + (c2 + c3), then the
 * tail sequentially into t, s + t (forward_ops.c:320-353). */
float orc_top1_prob(const float *l, int n) {
    float mx = -INFINITY;
    for (int i = 0; i < n; i++)
        if (l[i] > mx) mx = l[i];
    float c[4] = {0.0f, 0.0f, 0.0f, 0.0f}, t = 0.0f;
    const int q4 = n / 4 * 4;
    for (int i = 0; i < q4; i++) c[i % 4] = c[i % 4] + orc_expf_cephes(l[i] - mx);
    for (int i = q4; i < n; i++) t = t + orc_expf_cephes(l[i] - mx);
    const float s = ((c[0] + c[1]) + (c[2] + c[3])) + t;
    return s > 0.0f ? 1.0f / s : 0.0f;
}

/* ---- gate exp / log1p: binary64 evaluation, one rounding to binary32 -------------------
 * exp: Cody-Waite reduction x = k ln2 + r (ln2 split so k * LN2_HI is exact for |k| < 2^20),
 * |r| <= ln2/2, Taylor polynomial of degree 13 in Horner form (truncation < 2e-17), then the
 * power of two assembled in the exponent field. log1p: 1 + y is exact in binary64 for binary32
 * y >= 1e-4 in magnitude; log(m 2^e) = e ln2 + 2 atanh(s), s = (m-1)/(m+1), m in
 * [sqrt(1/2), sqrt(2)), atanh series to s^25 (Abramowitz & Stegun 4.1.28 form). Small |y| use
 * the log1p series to y^6. The error of the binary64 value is a few units of 2^-53, so the
 * final rounding to binary32 is the correctly rounded result except within ~1e-16 of a
 * rounding midpoint. */
#define G_LN2_HI 6.93147180369123816490e-01 /* 0x3fe62e42fee00000 */
#define G_LN2_LO 1.90821492927058770002e-10 /* 0x3dea39ef35793c76 */
#define G_INV_LN2 1.44269504088896338700e+00

static double pow2i(int k) { /* 2^k for -1022 <= k <= 1023 */
    const uint64_t bits = (uint64_t)(k + 1023) << 52;
    double d;
    memcpy(&d, &bits, 8);
    return d;
}

float orc_gate_expf(float xf) {
    if (xf != xf) return xf;
    if (xf > 89.0f) return INFINITY;
    if (xf < -104.0f) return 0.0f;
    const double x = (double)xf;
    const double k = rint(x * G_INV_LN2);
    double r = x - k * G_LN2_HI;
    r = r - k * G_LN2_LO;
    double p = 1.0 / 6227020800.0;       /* 1/13! */
    p = p * r + 1.0 / 479001600.0;       /* 1/12! */
    p = p * r + 1.0 / 39916800.0;        /* 1/11! */
    p = p * r + 1.0 / 3628800.0;         /* 1/10! */
    p = p * r + 1.0 / 362880.0;          /* 1/9! */
    p = p * r + 1.0 / 40320.0;           /* 1/8! */
    p = p * r + 1.0 / 5040.0;            /* 1/7! */
    p = p * r + 1.0 / 720.0;             /* 1/6! */
    p = p * r + 1.0 / 120.0;             /* 1/5! */
    p = p * r + 1.0 / 24.0;              /* 1/4! */
    p = p * r + 1.0 / 6.0;               /* 1/3! */
    p = p * r + 0.5;                     /* 1/2! */
    p = p * r + 1.0;
    p = p * r + 1.0;
    return (float)(p * pow2i((int)k));
}

float orc_gate_log1pf(float yf) {
    if (yf != yf) return yf;
    if (yf <= -1.0f) return yf == -1.0f ? -INFINITY : NAN;
    if (yf == INFINITY) return yf;
    const double y = (double)yf;
    if (fabs(y) < 1e-4) {
        double p = -1.0 / 6.0;
        p = p * y + 1.0 / 5.0;
        p = p * y - 1.0 / 4.0;
        p = p * y + 1.0 / 3.0;
        p = p * y - 1.0 / 2.0;
        p = p * y + 1.0;
        return (float)(p * y);
    }
    const double u = 1.0 + y; /* exact */
    uint64_t bits;
    memcpy(&bits, &u, 8);
    int e = (int)((bits >> 52) & 0x7ff) - 1023;
    bits = (bits & 0x000fffffffffffffull) | 0x3ff0000000000000ull; /* m in [1, 2) */
    double m;
    memcpy(&m, &bits, 8);
    if (m > 1.41421356237309504880) { m = m * 0.5; e += 1; }
    const double s = (m - 1.0) / (m + 1.0), s2 = s * s;
    double t = 1.0 / 25.0;
    t = t * s2 + 1.0 / 23.0;
    t = t * s2 + 1.0 / 21.0;
    t = t * s2 + 1.0 / 19.0;
    t = t * s2 + 1.0 / 17.0;
    t = t * s2 + 1.0 / 15.0;
    t = t * s2 + 1.0 / 13.0;
    t = t * s2 + 1.0 / 11.0;
    t = t * s2 + 1.0 / 9.0;
    t = t * s2 + 1.0 / 7.0;
    t = t * s2 + 1.0 / 5.0;
    t = t * s2 + 1.0 / 3.0;
    t = t * s2 + 1.0;
    const double logm = 2.0 * s * t;
    const double de = (double)e;
    return (float)((de * G_LN2_HI + logm) + de * G_LN2_LO);
}
