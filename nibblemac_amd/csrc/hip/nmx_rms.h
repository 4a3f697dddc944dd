/* Row RMSNorm with A8 output shared by the norm kernels and the heads' norm prologues
 * (engine/src/forward_ops.c:191-200, kern_act.c:14-88): the sum of squares as 4 interleaved
 * partial sums in element order plus the cols % 4 tail, combined (s0 + s1) + (s2 + s3) + tail,
 * r = 1 / sqrtf(ss / cols + eps), y = (x * r) * w, and the A8 blocks of y. */
#ifndef NMX_RMS_H
#define NMX_RMS_H

#include <hip/hip_runtime.h>
#include <cstdint>

#include "nmx_math.h"
#include "nmx_lanes.h"

/* The same sum over values stored chain-major: chain l's m-th value at cm[l * s4 + m]
 * (s4 a multiple of 4, so a chain is read as float4), the cols % 4 tail at cm[4 * s4 + k].
 * Two register sets of 32 values take turns: the next set is requested before the current
 * one is added (scheduling barriers keep that order; a request past the end re-reads). */
__device__ inline float ordered_sum4_cm(const float *cm, int cols, int s4, float *red) {
    const int tid = threadIdx.x, m4 = cols >> 2;
    if (tid < 4) {
        const float *ch = cm + tid * s4;
        float c = 0.0f;
        int m = 0;
        auto fetch = [&](float4 (&b)[8], int m0) {
#pragma unroll
            for (int u = 0; u < 8; u++) b[u] = *(const float4 *)(ch + m0 + 4 * u);
        };
        auto add = [&](const float4 (&b)[8]) {
#pragma unroll
            for (int u = 0; u < 8; u++) {
                c = c + b[u].x;
                c = c + b[u].y;
                c = c + b[u].z;
                c = c + b[u].w;
            }
        };
        if (m4 >= 32) {
            float4 ba[8], bb[8];
            fetch(ba, 0);
            for (; m + 64 <= m4; m += 64) {
                __builtin_amdgcn_sched_barrier(0);
                fetch(bb, m + 32);
                __builtin_amdgcn_sched_barrier(0);
                add(ba);
                __builtin_amdgcn_sched_barrier(0);
                fetch(ba, m + 96 <= m4 ? m + 64 : m);
                __builtin_amdgcn_sched_barrier(0);
                add(bb);
            }
            __builtin_amdgcn_sched_barrier(0);
            if (m + 32 <= m4) { /* ba holds values m .. m + 31 */
                add(ba);
                m += 32;
            }
        }
        for (; m < m4; m++) c = c + ch[m];
        red[tid] = c;
    } else if (tid == 4) {
        float t = 0.0f;
        for (int i = m4 * 4; i < cols; i++) t = t + cm[4 * s4 + (i - m4 * 4)];
        red[4] = t;
    }
    __syncthreads();
    const float s = (red[0] + red[1]) + (red[2] + red[3]);
    const float r = s + red[4];
    __syncthreads();
    return r;
}

__host__ __device__ constexpr int cm_stride(int cols) { return (((cols >> 2) + 3) & ~3) + 4; }

/* The same RMSNorm with each thread owning 4 consecutive columns (float4 loads and stores,
 * cols % 4 == 0, 16-byte aligned rows): element 4 j + l is term j of partial sum l, so the squares
 * go to LDS chain-major directly; a 32-column A8 block is 8 consecutive lanes (its amax and the
 * code sum reduced over them by DPP, exact in any order). */
__device__ __forceinline__ void a8_block4(float4 x, int b, int v, int n, int8_t *q, float *d,
                                          float *fs) {
    const size_t u = (size_t)b * n + v;
    const int l8 = threadIdx.x & 7;
    float m = fmaxf(fmaxf(fabsf(x.x), fabsf(x.y)), fmaxf(fabsf(x.z), fabsf(x.w)));
    m = fmaxf(m, __int_as_float(nmx_dpp<NMX_DPP_XOR1>(__float_as_int(m))));
    m = fmaxf(m, __int_as_float(nmx_dpp<NMX_DPP_XOR2>(__float_as_int(m))));
    m = fmaxf(m, __int_as_float(nmx_dpp<NMX_DPP_HALF_MIRROR>(__float_as_int(m))));
    const float id = m > 0.0f ? 127.0f / m : 0.0f;
    const int c0 = (int)rintf(x.x * id), c1 = (int)rintf(x.y * id);
    const int c2 = (int)rintf(x.z * id), c3 = (int)rintf(x.w * id);
    int sum = (c0 + c1) + (c2 + c3);
    sum += nmx_dpp<NMX_DPP_XOR1>(sum);
    sum += nmx_dpp<NMX_DPP_XOR2>(sum);
    sum += nmx_dpp<NMX_DPP_HALF_MIRROR>(sum);
    auto cl = [](int c) { return (uint32_t)(uint8_t)(int8_t)(c > 127 ? 127 : c < -128 ? -128 : c); };
    ((uint32_t *)(q + u * 32))[l8] = cl(c0) | cl(c1) << 8 | cl(c2) << 16 | cl(c3) << 24;
    if (l8 == 0) {
        const float dd = m / 127.0f;
        d[u] = dd;
        fs[u] = dd * (float)sum;
    }
}

/* Columns 4 j .. 4 j + 3 of Q4K row `row` (cols columns), as embed_k computes them. */
__device__ __forceinline__ float4 embed4(const uint8_t *E, int row, int cols, int j) {
    const int c = 4 * j, sb = c >> 8, k = (c & 255) >> 5, jj = c & 31, i = row & 3;
    const uint8_t *p = E + ((size_t)(row >> 2) * (cols >> 8) + sb) * 576;
    const float D = nmx_half(p + 2 * i), M = nmx_half(p + 8 + 2 * i);
    const float dd = D * (float)nmx_get6(p + 16, 4 * k + i);
    const float mm = M * (float)nmx_get6(p + 40, 4 * k + i);
    const uint32_t b4 = *(const uint32_t *)(p + 64 + 64 * k + 16 * i + (jj & 15));
    const uint32_t u4 = jj < 16 ? (b4 & 0x0f0f0f0fu) : ((b4 >> 4) & 0x0f0f0f0fu);
    return make_float4(dd * (float)(u4 & 0xffu) - mm, dd * (float)((u4 >> 8) & 0xffu) - mm,
                       dd * (float)((u4 >> 16) & 0xffu) - mm, dd * (float)(u4 >> 24) - mm);
}

/* rms4_row in two steps: rms4_load requests the row (x, add, w; P4 float4 per thread, indexes
 * clamped in-bounds) so that a caller can issue other loads before the first use, and
 * rms4_finish adds, squares, reduces and writes y and the A8 blocks. rms4_load_w requests the
 * norm weights alone, for callers whose row address waits for a load (a token); rms4_load<P4,
 * true> then leaves wv as it is. */
template <int P4>
__device__ __forceinline__ void rms4_load_w(const float *w, int cols, float4 (&wv)[P4]) {
    const int tid = threadIdx.x, c4 = cols >> 2;
#pragma unroll
    for (int u = 0; u < P4; u++) {
        const int j = tid + 256 * u, jc = j < c4 ? j : c4 - 1;
        wv[u] = ((const float4 *)w)[jc];
    }
}

template <int P4, bool HAVE_W = false>
__device__ __forceinline__ void rms4_load(const float *xr, const float *ar, const float *w,
                                          int cols, float4 (&v)[P4], float4 (&a)[P4],
                                          float4 (&wv)[P4], const uint8_t *E = nullptr,
                                          int er = 0) {
    const int tid = threadIdx.x, c4 = cols >> 2;
    if constexpr (!HAVE_W) rms4_load_w<P4>(w, cols, wv);
#pragma unroll
    for (int u = 0; u < P4; u++) {
        const int j = tid + 256 * u, jc = j < c4 ? j : c4 - 1;
        v[u] = E ? embed4(E, er, cols, jc) : ((const float4 *)xr)[jc];
        a[u] = ar ? ((const float4 *)ar)[jc] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
}

template <int P4>
__device__ __forceinline__ void rms4_finish(float4 (&v)[P4], const float4 (&a)[P4],
                                            const float4 (&wv)[P4], bool add, float *xo, int cols,
                                            float eps, float *__restrict__ y,
                                            int8_t *__restrict__ q, float *__restrict__ d,
                                            float *__restrict__ fs, int n, int row, float *sq,
                                            float *red) {
    const int tid = threadIdx.x;
    const int c4 = cols >> 2, s4 = cm_stride(cols);
    if (add) {
#pragma unroll
        for (int u = 0; u < P4; u++)
            v[u] = make_float4(v[u].x + a[u].x, v[u].y + a[u].y, v[u].z + a[u].z, v[u].w + a[u].w);
    }
#pragma unroll
    for (int u = 0; u < P4; u++) {
        const int j = tid + 256 * u;
        if (j >= c4) continue;
        if (xo) ((float4 *)xo)[j] = v[u];
        sq[j] = v[u].x * v[u].x;
        sq[s4 + j] = v[u].y * v[u].y;
        sq[2 * s4 + j] = v[u].z * v[u].z;
        sq[3 * s4 + j] = v[u].w * v[u].w;
    }
    __syncthreads();
    const float ss = ordered_sum4_cm(sq, cols, s4, red);
    const float r = 1.0f / sqrtf(ss / (float)cols + eps);
#pragma unroll
    for (int u = 0; u < P4; u++) {
        const int j = tid + 256 * u;
        if (256 * u + (tid & ~7) >= c4) continue; /* whole 8-lane group past the row */
        const float4 o = make_float4((v[u].x * r) * wv[u].x, (v[u].y * r) * wv[u].y,
                                     (v[u].z * r) * wv[u].z, (v[u].w * r) * wv[u].w);
        if (y) ((float4 *)y)[j] = o;
        if (q) a8_block4(o, j >> 3, row, n, q, d, fs);
    }
}

/* One row of rmsnorm4_k (row of the workgroup; sq / red its LDS). E (optional): row `row` is
 * the Q4K embedding row tok[row] of E instead of x's row. */
template <int P4>
__device__ __forceinline__ void rms4_row(const float *x, int x_stride, const float *add,
                                         int add_stride, float *xo, int xo_stride,
                                         const float *__restrict__ w, int cols, float eps,
                                         float *__restrict__ y, int y_stride, int8_t *__restrict__ q,
                                         float *__restrict__ d, float *__restrict__ fs, int n,
                                         int row, float *sq, float *red,
                                         const uint8_t *E = nullptr, const int32_t *tok = nullptr) {
    float4 v[P4], a[P4], wv[P4];
    rms4_load_w<P4>(w, cols, wv); /* before the token the embedding row waits for */
    rms4_load<P4, true>(x + (size_t)row * x_stride, add ? add + (size_t)row * add_stride : nullptr,
                        w, cols, v, a, wv, E, E ? tok[row] : 0);
    rms4_finish<P4>(v, a, wv, add != nullptr, xo ? xo + (size_t)row * xo_stride : nullptr, cols,
                    eps, y ? y + (size_t)row * y_stride : nullptr, q, d, fs, n, row, sq, red);
}

#endif
