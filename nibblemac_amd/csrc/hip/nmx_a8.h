/* A8 activation quantization of one 32-column block held by a 32-lane half-wave (lane =
 * column), shared by every kernel that produces a matmul input (engine/src/kern_act.c:14-42):
 * amax = max |x|, id = 127 / amax (0 when amax is 0), codes round-half-even(x * id),
 * d = amax / 127, fsum = d * sum(codes).
 *
 * The two reductions (max, integer sum) are exact in any order; they run as DPP lane moves
 * (nmx_lanes.h) instead of five LDS-crossbar shuffles each. Every lane of the half-wave must be
 * active. */
#ifndef NMX_A8_H
#define NMX_A8_H

#include <hip/hip_runtime.h>
#include <cstdint>

#include "nmx_lanes.h"

/* Quantize the half-wave's block: lane j writes q[j]; lane 0 writes *d and *fs. */
__device__ __forceinline__ void nmx_a8_store(float x, int8_t *q, float *d, float *fs) {
    const int j = threadIdx.x & 31;
    const float amax = nmx_max32(fabsf(x));
    const float id = amax > 0.0f ? 127.0f / amax : 0.0f;
    const int c = (int)rintf(x * id);
    const int sum = nmx_sum32(c);
    q[j] = (int8_t)(c > 127 ? 127 : c < -128 ? -128 : c);
    if (j == 0) {
        const float dd = amax / 127.0f;
        *d = dd;
        *fs = dd * (float)sum;
    }
}

/* Two blocks at once (one value of each per lane): both blocks' reductions and divides are
 * computed before any store, so the two dependent chains interleave. */
__device__ __forceinline__ void nmx_a8_store2(float x1, int8_t *q1, float *d1, float *fs1,
                                              float x2, int8_t *q2, float *d2, float *fs2) {
    const int j = threadIdx.x & 31;
    const float am1 = nmx_max32(fabsf(x1)), am2 = nmx_max32(fabsf(x2));
    const float id1 = am1 > 0.0f ? 127.0f / am1 : 0.0f, id2 = am2 > 0.0f ? 127.0f / am2 : 0.0f;
    const int c1 = (int)rintf(x1 * id1), c2 = (int)rintf(x2 * id2);
    const int s1 = nmx_sum32(c1), s2 = nmx_sum32(c2);
    const float dd1 = am1 / 127.0f, dd2 = am2 / 127.0f;
    const float f1 = dd1 * (float)s1, f2 = dd2 * (float)s2;
    q1[j] = (int8_t)(c1 > 127 ? 127 : c1 < -128 ? -128 : c1);
    q2[j] = (int8_t)(c2 > 127 ? 127 : c2 < -128 ? -128 : c2);
    if (j == 0) {
        *d1 = dd1, *fs1 = f1;
        *d2 = dd2, *fs2 = f2;
    }
}

#endif
