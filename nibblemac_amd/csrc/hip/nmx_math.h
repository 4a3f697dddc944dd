/* Device scalar primitives shared by the nmx kernels.
 *
 * nmx_expf_cephes: the reference's pf_expf (engine/src/forward_ops.c:26-56) operation for
 *   operation (clamp, two-part ln2 reduction, degree-6 polynomial, exponent bits); every SiLU,
 *   sigmoid and softmax exponential of the forward pass.
 * nmx_gate_expf / nmx_gate_log1pf: exp and log1p for the 16 per-layer DeltaNet gates, where the
 *   reference calls glibc (engine/src/forward_lin.c:18-19,59-66). Evaluated in binary64 and
 *   rounded once to binary32: Cody-Waite reduction x = k ln2 + r with a degree-13 Taylor
 *   polynomial; log(m 2^e) = e ln2 + 2 atanh((m-1)/(m+1)) with the atanh series to s^25, and
 *   the log1p series below 1e-4. The binary64 error is a few units of 2^-53, so the result is
 *   the correctly rounded binary32 except within ~1e-16 of a rounding midpoint. */
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

__device__ __forceinline__ double nmx_pow2i(int k) {
    return __longlong_as_double((long long)((uint64_t)(k + 1023) << 52));
}

__device__ __forceinline__ float nmx_gate_expf(float xf) {
    if (xf != xf) return xf;
    if (xf > 89.0f) return __int_as_float(0x7f800000);
    if (xf < -104.0f) return 0.0f;
    const double x = (double)xf;
    const double k = rint(x * 1.44269504088896338700e+00);
    double r = x - k * 6.93147180369123816490e-01;
    r = r - k * 1.90821492927058770002e-10;
    double p = 1.0 / 6227020800.0;
    p = p * r + 1.0 / 479001600.0;
    p = p * r + 1.0 / 39916800.0;
    p = p * r + 1.0 / 3628800.0;
    p = p * r + 1.0 / 362880.0;
    p = p * r + 1.0 / 40320.0;
    p = p * r + 1.0 / 5040.0;
    p = p * r + 1.0 / 720.0;
    p = p * r + 1.0 / 120.0;
    p = p * r + 1.0 / 24.0;
    p = p * r + 1.0 / 6.0;
    p = p * r + 0.5;
    p = p * r + 1.0;
    p = p * r + 1.0;
    return (float)(p * nmx_pow2i((int)k));
}

__device__ __forceinline__ float nmx_gate_log1pf(float yf) {
    if (yf != yf) return yf;
    if (yf <= -1.0f) return yf == -1.0f ? __int_as_float(0xff800000) : __int_as_float(0x7fc00000);
    if (yf == __int_as_float(0x7f800000)) return yf;
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
    const double u = 1.0 + y;
    uint64_t bits = (uint64_t)__double_as_longlong(u);
    int e = (int)((bits >> 52) & 0x7ff) - 1023;
    bits = (bits & 0x000fffffffffffffull) | 0x3ff0000000000000ull;
    double m = __longlong_as_double((long long)bits);
    if (m > 1.41421356237309504880) {
        m = m * 0.5;
        e += 1;
    }
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
    return (float)((de * 6.93147180369123816490e-01 + logm) + de * 1.90821492927058770002e-10);
}

/* fp16 bits at p (little endian) -> float, exact */
__device__ __forceinline__ float nmx_half(const uint8_t *p) {
    const unsigned short b = (unsigned short)(p[0] | (p[1] << 8));
    _Float16 f;
    __builtin_memcpy(&f, &b, 2);
    return (float)f;
}

/* value j of a packed 6-bit array (engine/src/kern_act.c:47-50) */
__device__ __forceinline__ int nmx_get6(const uint8_t *p, int j) {
    const int lo = j < 16 ? (p[j] & 15) : (p[j - 16] >> 4);
    return lo | (((p[16 + (j & 7)] >> (2 * (j >> 3))) & 3) << 4);
}

#endif
