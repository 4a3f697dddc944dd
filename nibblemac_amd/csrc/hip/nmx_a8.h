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

#endif
