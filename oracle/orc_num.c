/* ORACLE — test infrastructure only (see oracle.h). Scalar numeric primitives. */
#include <math.h>
#include <pthread.h>
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

/* ---- gate exp / log1p: the host C library's, operation for operation ------------------
 * The reference computes the DeltaNet gates with libm expf / log1pf (forward_lin.c:18-19,
 * 59-66). On this platform (x86-64, glibc 2.35) those are:
 *   expf: the table method of Arm's optimized-routines (Szabolcs Nagy), which glibc adopted:
 *     z = x N / ln2 (N = 32) split as k + r by adding and subtracting 1.5 * 2^52 (round to
 *     nearest even), 2^(k/N) from a 32-entry table of 2^(i/32) (bit pattern minus i << 47, so
 *     that adding k << 47 supplies the exponent), 2^(r/N) by a cubic, all in binary64; glibc
 *     selects its FMA build on this hardware, so z + shift, z - kd and the cubic's three
 *     multiply-adds are fused (the multiplication x N / ln2 fused into both of its uses);
 *   log1pf: Sun's fdlibm s_log1pf.c, in binary32 without fused operations: 1 + x split into
 *     2^k (1 + f) with a correction term c for the rounding of 1 + x, log(1 + f) = f - hfsq +
 *     s (hfsq + R) with s = f / (2 + f) and R a degree-7 polynomial in s^2, k ln2 in two
 *     parts.
 * Both are checked against the host's expf / log1pf over every binary32 input (0 differences;
 * orc_libm_mismatches). */
static uint64_t g_exp2_tab[32]; /* bits of 2^(i/32) minus i << 47 */
static pthread_once_t g_exp2_once = PTHREAD_ONCE_INIT;

static void exp2_tab_init(void) {
    for (int i = 0; i < 32; i++) {
        /* 2^(i/32) rounded to binary64: the 64-bit-mantissa value is within 2^-64 relative
         * and no entry lies that close to a binary64 rounding midpoint (checked in tests) */
        const double v = (double)exp2l((long double)i / 32.0L);
        uint64_t b;
        memcpy(&b, &v, 8);
        g_exp2_tab[i] = b - ((uint64_t)i << 47);
    }
}

uint64_t orc_exp2_tab(int i) {
    pthread_once(&g_exp2_once, exp2_tab_init);
    return g_exp2_tab[i & 31];
}

static uint32_t f2u(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
static float u2f(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

float orc_gate_expf(float x) {
    static const double inv_ln2_n = 0x1.71547652b82fep+5, shift = 0x1.8p+52;
    static const double c0 = 0x1.c6af84b912394p-20, c1 = 0x1.ebfce50fac4f3p-13,
                        c2 = 0x1.62e42ff0c52d6p-6;
    pthread_once(&g_exp2_once, exp2_tab_init);
    const uint32_t top = (f2u(x) >> 20) & 0x7ff;
    if (top >= (f2u(88.0f) >> 20)) { /* |x| >= 88, inf or nan */
        if (f2u(x) == f2u(-INFINITY)) return 0.0f;
        if (top >= (f2u(INFINITY) >> 20)) return x + x;
        if (x > 0x1.62e42ep6f) return INFINITY;   /* overflow */
        if (x < -0x1.9fe368p6f) return 0.0f;      /* underflow */
    }
    const double xd = (double)x;
    double kd = fma(inv_ln2_n, xd, shift);
    uint64_t ki;
    memcpy(&ki, &kd, 8);
    kd -= shift;
    const double r = fma(inv_ln2_n, xd, -kd);
    const uint64_t t = g_exp2_tab[ki % 32] + (ki << 47);
    double s;
    memcpy(&s, &t, 8);
    const double z = fma(c0, r, c1), r2 = r * r;
    double y = fma(c2, r, 1.0);
    y = fma(z, r2, y);
    return (float)(y * s);
}

float orc_gate_log1pf(float x) {
    static const float ln2_hi = 6.9313812256e-01f, ln2_lo = 9.0580006145e-06f;
    static const float lp1 = 6.6666668653e-01f, lp2 = 4.0000000596e-01f,
                       lp3 = 2.8571429849e-01f, lp4 = 2.2222198546e-01f,
                       lp5 = 1.8183572590e-01f, lp6 = 1.5313838422e-01f,
                       lp7 = 1.4798198640e-01f;
    const int32_t hx = (int32_t)f2u(x), ax = hx & 0x7fffffff;
    int32_t k = 1, hu = 0;
    float f = 0.0f, c = 0.0f;
    if (hx < 0x3ed413d7) {                     /* x < 0.41422 */
        if (ax >= 0x3f800000) return x == -1.0f ? -INFINITY : NAN; /* x <= -1 */
        if (ax < 0x31000000) {                 /* |x| < 2^-29 */
            if (ax < 0x24800000) return x;     /* |x| < 2^-54 */
            return x - x * x * 0.5f;
        }
        if (hx > 0 || hx <= (int32_t)0xbe95f61f) { /* -0.2929 < x < 0.41422 */
            k = 0;
            f = x;
            hu = 1;
        }
    } else if (hx >= 0x7f800000) {
        return x + x;
    }
    if (k != 0) {
        float u;
        if (hx < 0x5a000000) {
            u = 1.0f + x;
            hu = (int32_t)f2u(u);
            k = (hu >> 23) - 127;
            c = k > 0 ? 1.0f - (u - x) : x - (u - 1.0f); /* the rounding error of 1 + x */
            c /= u;
        } else {
            u = x;
            hu = (int32_t)f2u(u);
            k = (hu >> 23) - 127;
            c = 0.0f;
        }
        hu &= 0x007fffff;
        if (hu < 0x3504f7) {
            u = u2f((uint32_t)hu | 0x3f800000u);              /* 1 + f in [1, sqrt 2) */
        } else {
            k += 1;
            u = u2f((uint32_t)hu | 0x3f000000u);              /* (1 + f) / 2 */
            hu = (0x00800000 - hu) >> 2;
        }
        f = u - 1.0f;
    }
    const float hfsq = 0.5f * f * f;
    const float fk = (float)k;
    if (hu == 0) { /* |f| < 2^-20 */
        if (f == 0.0f) {
            if (k == 0) return 0.0f;
            c += fk * ln2_lo;
            return fk * ln2_hi + c;
        }
        const float R = hfsq * (1.0f - 0.66666666666666666f * f);
        if (k == 0) return f - R;
        return fk * ln2_hi - ((R - (fk * ln2_lo + c)) - f);
    }
    const float s = f / (2.0f + f), z = s * s;
    const float R = z * (lp1 + z * (lp2 + z * (lp3 + z * (lp4 + z * (lp5 + z * (lp6 + z * lp7))))));
    if (k == 0) return f - (hfsq - s * (hfsq + R));
    return fk * ln2_hi - ((hfsq - (s * (hfsq + R) + (fk * ln2_lo + c))) - f);
}

/* The number of binary32 inputs (NaNs excluded; a NaN result equals any NaN) on which
 * orc_gate_expf (which = 0) or orc_gate_log1pf (1) differs from the host C library's expf /
 * log1pf, over all 2^32 bit patterns, on `threads` threads. */
typedef struct {
    uint64_t lo, hi;
    int which;
    long long bad;
} libm_job;

static void *libm_scan(void *p) {
    libm_job *j = (libm_job *)p;
    for (uint64_t u = j->lo; u < j->hi; u++) {
        const float x = u2f((uint32_t)u);
        if (x != x) continue;
        const float a = j->which ? log1pf(x) : expf(x);
        const float b = j->which ? orc_gate_log1pf(x) : orc_gate_expf(x);
        if (f2u(a) != f2u(b) && !(a != a && b != b)) j->bad++;
    }
    return NULL;
}

long long orc_libm_mismatches(int which, int threads) {
    pthread_once(&g_exp2_once, exp2_tab_init);
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    pthread_t t[64];
    libm_job J[64];
    const uint64_t span = (1ull << 32) / (uint64_t)threads + 1;
    for (int i = 0; i < threads; i++) {
        const uint64_t lo = span * (uint64_t)i, hi = lo + span;
        J[i] = (libm_job){lo, hi < (1ull << 32) ? hi : (1ull << 32), which, 0};
        pthread_create(&t[i], NULL, libm_scan, &J[i]);
    }
    long long bad = 0;
    for (int i = 0; i < threads; i++) {
        pthread_join(t[i], NULL);
        bad += J[i].bad;
    }
    return bad;
}

/* y[i] = the host C library's expf (which = 0) or log1pf (1) of the binary32 input with bit
 * pattern first + i, for i < n, on `threads` threads: the reference values of a device sweep. */
typedef struct {
    int which;
    uint32_t first;
    long lo, hi;
    float *y;
} libm_fill;

static void *libm_fill_run(void *p) {
    const libm_fill *j = (const libm_fill *)p;
    for (long i = j->lo; i < j->hi; i++) {
        const float x = u2f(j->first + (uint32_t)i);
        j->y[i] = j->which ? log1pf(x) : expf(x);
    }
    return NULL;
}

void orc_libm_eval(int which, uint32_t first, long n, float *y, int threads) {
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    pthread_t t[64];
    libm_fill J[64];
    const long span = n / threads + 1;
    for (int i = 0; i < threads; i++) {
        const long lo = span * i < n ? span * i : n, hi = lo + span < n ? lo + span : n;
        J[i] = (libm_fill){which, first, lo, hi, y};
        pthread_create(&t[i], NULL, libm_fill_run, &J[i]);
    }
    for (int i = 0; i < threads; i++) pthread_join(t[i], NULL);
}
