/* A8 activation quantization of one 32-column block held by a 32-lane half-wave (lane =
 * column), shared by every kernel that produces a matmul input (engine/src/kern_act.c:14-42):
 * amax = max |x|, id = 127 / amax (0 when amax is 0), codes round-half-even(x * id),
 * d = amax / 127, fsum = d * sum(codes).
 *
 * The two reductions (max, integer sum) are exact in any order; they run as DPP quad
 * permutes and row mirrors inside each 16-lane row (VALU-speed lane exchanges) and one
 * ds_swizzle across the two rows of the half-wave, instead of five LDS-crossbar shuffles each.
 * Every lane of the half-wave must be active. */
#ifndef NMX_A8_H
#define NMX_A8_H

#include <hip/hip_runtime.h>
#include <cstdint>

template <int CTRL>
__device__ __forceinline__ int nmx_dpp(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, true);
}

/* lane ^ 16 within each 32-lane group (swizzle bit mode: and 0x1f, or 0, xor 0x10) */
__device__ __forceinline__ int nmx_swz16(int v) { return __builtin_amdgcn_ds_swizzle(v, 0x401F); }

constexpr int NMX_DPP_XOR1 = 0xB1;        /* quad_perm [1, 0, 3, 2] */
constexpr int NMX_DPP_XOR2 = 0x4E;        /* quad_perm [2, 3, 0, 1] */
constexpr int NMX_DPP_HALF_MIRROR = 0x141; /* lane i <- 7 - i within 8 */
constexpr int NMX_DPP_MIRROR = 0x140;      /* lane i <- 15 - i within 16 */

__device__ __forceinline__ float nmx_max32(float v) {
    v = fmaxf(v, __int_as_float(nmx_dpp<NMX_DPP_XOR1>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(nmx_dpp<NMX_DPP_XOR2>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(nmx_dpp<NMX_DPP_HALF_MIRROR>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(nmx_dpp<NMX_DPP_MIRROR>(__float_as_int(v))));
    return fmaxf(v, __int_as_float(nmx_swz16(__float_as_int(v))));
}

__device__ __forceinline__ int nmx_sum32(int v) {
    v += nmx_dpp<NMX_DPP_XOR1>(v);
    v += nmx_dpp<NMX_DPP_XOR2>(v);
    v += nmx_dpp<NMX_DPP_HALF_MIRROR>(v);
    v += nmx_dpp<NMX_DPP_MIRROR>(v);
    return v + nmx_swz16(v);
}

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
