/* Device scalar primitives shared by the nmx kernels.
 *
 * nmx_expf_cephes: the reference's pf_expf (engine/src/forward_ops.c:26-56) operation for
 *   operation (clamp, two-part ln2 reduction, degree-6 polynomial, exponent bits); every SiLU,
 *   sigmoid and softmax exponential of the forward pass.
 * nmx_gate_expf / nmx_gate_log1pf: exp and log1p for the 16 per-layer DeltaNet gates, where the
 *   reference calls the C library (engine/src/forward_lin.c:18-19,59-66). They restate, operation
 *   for operation, the functions the reference calls on this platform (glibc 2.35, x86-64):
 *   expf is the table method of Arm's optimized-routines that glibc adopted, as glibc's FMA
 *   build evaluates it (binary64; z = x 32 / ln2 rounded to an integer k by adding and
 *   subtracting 1.5 * 2^52, r = z - k with the product fused into both, 2^(k/32) from a table
 *   of 2^(i/32) whose entries hold their bit pattern minus i << 47, 2^(r/32) by a cubic with
 *   fused multiply-adds); log1pf is Sun's fdlibm s_log1pf.c in binary32 with no fused
 *   operation. Both equal the host library on every binary32 input (the oracle's copy is
 *   checked over all 2^32 inputs on the CPU, this one over the same sweep on the GPU). */
#ifndef NMX_MATH_H
#define NMX_MATH_H

#include <hip/hip_runtime.h>
#include <cstdint>

__device__ __forceinline__ float nmx_expf_cephes(float x) {
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
    return y * __uint_as_float((uint32_t)((int)fx + 127) << 23);
}

/* pf_silu / pf_sigmoid (forward_ops.c:58-59): x / (1 + exp(-x)), 1 / (1 + exp(-x)). */
__device__ __forceinline__ float nmx_silu(float x) { return x / (1.0f + nmx_expf_cephes(-x)); }
__device__ __forceinline__ float nmx_sigmoid(float x) { return 1.0f / (1.0f + nmx_expf_cephes(-x)); }

/* 2^(i/32) rounded to binary64, minus i << 47 (so that adding k << 47 for k = 32 q + i
 * yields 2^(k/32) with the exponent q folded in) */
static __device__ __constant__ const uint64_t nmx_exp2_32[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

/* tab: the 32 entries above, from this constant copy or from a copy in LDS (a kernel that
 * stages them at entry turns each lookup's memory round trip into an LDS read) */
__device__ __forceinline__ float nmx_gate_expf_t(float x, const uint64_t *tab) {
    const uint32_t top = (__float_as_uint(x) >> 20) & 0x7ffu;
    if (top >= (0x42b00000u >> 20)) { /* |x| >= 88, inf or nan */
        if (__float_as_uint(x) == 0xff800000u) return 0.0f;
        if (top >= 0x7f8u) return x + x;
        if (x > 0x1.62e42ep6f) return __uint_as_float(0x7f800000u); /* overflow */
        if (x < -0x1.9fe368p6f) return 0.0f;                        /* underflow */
    }
    const double xd = (double)x;
    double kd = __builtin_fma(0x1.71547652b82fep+5, xd, 0x1.8p+52);
    const uint64_t ki = (uint64_t)__double_as_longlong(kd);
    kd -= 0x1.8p+52;
    const double r = __builtin_fma(0x1.71547652b82fep+5, xd, -kd);
    const uint64_t t = tab[ki % 32] + (ki << 47);
    const double s = __longlong_as_double((long long)t);
    const double z = __builtin_fma(0x1.c6af84b912394p-20, r, 0x1.ebfce50fac4f3p-13), r2 = r * r;
    double y = __builtin_fma(0x1.62e42ff0c52d6p-6, r, 1.0);
    y = __builtin_fma(z, r2, y);
    return (float)(y * s);
}

__device__ __forceinline__ float nmx_gate_expf(float x) { return nmx_gate_expf_t(x, nmx_exp2_32); }

__device__ __forceinline__ float nmx_gate_log1pf(float x) {
    const float ln2_hi = 6.9313812256e-01f, ln2_lo = 9.0580006145e-06f;
    const int32_t hx = (int32_t)__float_as_uint(x), ax = hx & 0x7fffffff;
    int32_t k = 1, hu = 0;
    float f = 0.0f, c = 0.0f;
    if (hx < 0x3ed413d7) {                                   /* x < 0.41422 */
        if (ax >= 0x3f800000)                                /* x <= -1 */
            return x == -1.0f ? __uint_as_float(0xff800000u) : __uint_as_float(0x7fc00000u);
        if (ax < 0x31000000) return ax < 0x24800000 ? x : x - x * x * 0.5f; /* |x| < 2^-29 */
        if (hx > 0 || hx <= (int32_t)0xbe95f61f) {           /* -0.2929 < x < 0.41422 */
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
            hu = (int32_t)__float_as_uint(u);
            k = (hu >> 23) - 127;
            c = k > 0 ? 1.0f - (u - x) : x - (u - 1.0f); /* the rounding error of 1 + x */
            c /= u;
        } else {
            u = x;
            hu = (int32_t)__float_as_uint(u);
            k = (hu >> 23) - 127;
            c = 0.0f;
        }
        hu &= 0x007fffff;
        if (hu < 0x3504f7) {
            u = __uint_as_float((uint32_t)hu | 0x3f800000u);      /* 1 + f in [1, sqrt 2) */
        } else {
            k += 1;
            u = __uint_as_float((uint32_t)hu | 0x3f000000u);      /* (1 + f) / 2 */
            hu = (0x00800000 - hu) >> 2;
        }
        f = u - 1.0f;
    }
    const float hfsq = 0.5f * f * f, fk = (float)k;
    if (hu == 0) { /* |f| < 2^-20 */
        if (f == 0.0f) return k == 0 ? 0.0f : fk * ln2_hi + (c + fk * ln2_lo);
        const float R = hfsq * (1.0f - 0.66666666666666666f * f);
        return k == 0 ? f - R : fk * ln2_hi - ((R - (fk * ln2_lo + c)) - f);
    }
    const float s = f / (2.0f + f), z = s * s;
    const float R = z * (6.6666668653e-01f +
                    z * (4.0000000596e-01f +
                    z * (2.8571429849e-01f +
                    z * (2.2222198546e-01f +
                    z * (1.8183572590e-01f + z * (1.5313838422e-01f + z * 1.4798198640e-01f))))));
    if (k == 0) return f - (hfsq - s * (hfsq + R));
    return fk * ln2_hi - ((hfsq - (s * (hfsq + R) + (fk * ln2_lo + c))) - f);
}

/* fp16 bits at p (little endian) -> float, exact */
__device__ __forceinline__ float nmx_half(const uint8_t *p) {
    const unsigned short b = (unsigned short)(p[0] | (p[1] << 8));
    _Float16 f;
    __builtin_memcpy(&f, &b, 2);
    return (float)f;
}

/* value j of a packed 6-bit array (engine/src/kern_act.c:47-50): low nibble of byte j for
 * j < 16, high nibble of byte j - 16 otherwise, and bits 2 (j / 8) of byte 16 + j % 8. Both
 * reads are unconditional, so they are requested together (a select between two loads waited
 * for each one in turn). */
__device__ __forceinline__ int nmx_get6(const uint8_t *p, int j) {
    const int lo = (p[j & 15] >> (4 * (j >> 4))) & 15;
    return lo | (((p[16 + (j & 7)] >> (2 * (j >> 3))) & 3) << 4);
}

#endif
