/* Cross-lane helpers for gfx950 wave64 kernels.
 *
 * nmx_dpp<CTRL>: a DPP lane move (row_mask / bank_mask all, bound_ctrl); nmx_swz16: lane ^ 16
 * within each 32-lane group (ds_swizzle). nmx_max32 / nmx_sum32 reduce over each 32-lane
 * half-wave (every lane of the half active): DPP quad permutes and row mirrors inside the
 * 16-lane rows, one swizzle across them; max and integer sums are exact in any order.
 * nmx_quad_chain: a left-to-right fp32 sum over a quad of lanes, lane c holding the c-th
 * quarter of the terms; the running sum moves to the next lane by a DPP broadcast of lane c
 * (quad_perm [c, c, c, c]), so the adds are one sequential chain. */
#ifndef NMX_LANES_H
#define NMX_LANES_H

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

/* Maximum of a float over the wave (every lane active; exact in any order), returned to
 * every lane: nmx_max32 within each half, then the halves through readlane. */
__device__ __forceinline__ float nmx_max_f32_wave(float v) {
    const float m = nmx_max32(v);
    return fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 0)),
                 __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 32)));
}

/* Maximum of a 64-bit unsigned key over the wave (every lane active), returned to every
 * lane: DPP quad swaps and row mirrors within 16 lanes, a swizzle across the 16-lane rows
 * of each half, then the two halves through readlane. No LDS permutes. */
__device__ __forceinline__ void nmx_max_u64_step(uint32_t &lo, uint32_t &hi, uint32_t olo,
                                                 uint32_t ohi) {
    const bool take = ohi > hi || (ohi == hi && olo > lo);
    lo = take ? olo : lo;
    hi = take ? ohi : hi;
}

__device__ __forceinline__ unsigned long long nmx_max_u64_wave(unsigned long long key) {
    uint32_t lo = (uint32_t)key, hi = (uint32_t)(key >> 32);
#define NMX_MAX64_DPP(C)                                                                      \
    nmx_max_u64_step(lo, hi, (uint32_t)nmx_dpp<C>((int)lo), (uint32_t)nmx_dpp<C>((int)hi))
    NMX_MAX64_DPP(NMX_DPP_XOR1);
    NMX_MAX64_DPP(NMX_DPP_XOR2);
    NMX_MAX64_DPP(NMX_DPP_HALF_MIRROR);
    NMX_MAX64_DPP(NMX_DPP_MIRROR);
#undef NMX_MAX64_DPP
    nmx_max_u64_step(lo, hi, (uint32_t)nmx_swz16((int)lo), (uint32_t)nmx_swz16((int)hi));
    uint32_t lo0 = (uint32_t)__builtin_amdgcn_readlane((int)lo, 0);
    uint32_t hi0 = (uint32_t)__builtin_amdgcn_readlane((int)hi, 0);
    nmx_max_u64_step(lo0, hi0, (uint32_t)__builtin_amdgcn_readlane((int)lo, 32),
                     (uint32_t)__builtin_amdgcn_readlane((int)hi, 32));
    return ((unsigned long long)hi0 << 32) | lo0;
}

/* The row of the greatest of nk argmax keys (order-preserving value bits over the complemented
 * row index, so the greatest key is the first maximum): what head_finish_k resolves for one
 * vector. Every lane of the calling wave gets it; the first 512 keys (the draft head over 32768
 * rows leaves 512) are requested together. */
__device__ __forceinline__ int nmx_keys_token(const unsigned long long *keys, int nk) {
    const int lane = threadIdx.x & 63;
    unsigned long long k[8], m = 0ull;
#pragma unroll
    for (int u = 0; u < 8; u++) {
        const int i = lane + 64 * u;
        k[u] = keys[i < nk ? i : nk - 1];
    }
#pragma unroll
    for (int u = 0; u < 8; u++) m = k[u] > m ? k[u] : m;
    for (int i = lane + 512; i < nk; i += 64) m = keys[i] > m ? keys[i] : m;
    m = nmx_max_u64_wave(m);
    return (int)(0xffffffffu - (uint32_t)(m & 0xffffffffull));
}

template <int DK4>
__device__ __forceinline__ float nmx_quad_chain(const float (&p)[DK4]) {
    float carry = 0.0f;
#define NMX_QUAD_SEG(C)                                                                       \
    {                                                                                         \
        float acc = carry;                                                                    \
        _Pragma("unroll") for (int r = 0; r < DK4; r++) acc = acc + p[r];                     \
        carry = __int_as_float(nmx_dpp<(C) * 0x55>(__float_as_int(acc)));                     \
    }
    NMX_QUAD_SEG(0)
    NMX_QUAD_SEG(1)
    NMX_QUAD_SEG(2)
    NMX_QUAD_SEG(3)
#undef NMX_QUAD_SEG
    return carry;
}

#endif
