/* Q4K_G32 x A8 matvec / small-batch matmul and A8 activation quantization for gfx950.
 *
 * Exactness contract (the reference's kern_q4k, engine/src/kern_quant.c:148-245): for every
 * output row r and vector v the fp32 accumulator runs over the 32-column blocks in column
 * order, acc = fma((float)dot, (D*s)*d_v, acc); acc = fma(-(M*m), fsum_v, acc), with dot the
 * exact int32 sum of 32 nibble x int8 products. The integer part may be computed in any order;
 * the float chain may not, so one lane owns one (row, vector) chain.
 *
 * Mapping (one wave64 = 64 consecutive rows = 16 four-row tiles of the native .pq layout):
 *   - lane l reads its row's 16-byte code chunk of block k (bytes 64 + 64k + 16i of the
 *     superblock, i = row % 4): the 4 lanes of a tile read one contiguous 64-byte run, a wave
 *     16 runs per instruction, and over the 8 blocks of a superblock every byte of the tile's
 *     576-byte superblock is consumed once (128-bit loads, no repack);
 *   - every lane of a wave works on the same column block at the same time, so the A8
 *     activations (32 int8 + d + fsum per vector) are wave-uniform and are read with scalar
 *     loads into SGPRs, shared by all 64 rows; the integer dot is 8 v_dot4_i32_i8 per vector;
 *   - the 6-bit sub-scales / sub-mins of the lane's row are decoded from the 64-byte scale line
 *     once per superblock.
 * Several matrices that share one input run in one launch (segment table). */
#include <mutex>

#include "nmx_internal.h"
#include "nmx_a8.h"
#include "nmx_lanes.h"
#include "nmx_rms.h"

namespace {

constexpr int SB_BYTES = 576;
constexpr int MAX_NV = 8; /* vectors per register pass */

struct Seg {
    const uint8_t *W;
    float *Y;
    int rows;
    int ystride;
    int wave0; /* first global wave of this matrix */
    int pad;
};

struct SegTable {
    Seg s[NMX_MAX_SEGS];
    int count;
    int total_waves;
};

__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
    const unsigned short b = (unsigned short)h;
    _Float16 f;
    __builtin_memcpy(&f, &b, 2);
    return (float)f;
}

/* 6-bit values s[4k + i], k = 0..7, of one row i from a packed array (engine/FORMAT.md: 16 B
 * of low nibbles, then 8 B of high bit pairs): L0..L3 the low-nibble dwords, H0/H1 the
 * high-pair dwords, sh8 = 8 * i. */
__device__ __forceinline__ void decode6(uint32_t L0, uint32_t L1, uint32_t L2, uint32_t L3,
                                        uint32_t H0, uint32_t H1, int sh8, int out[8]) {
    const uint32_t b0 = (L0 >> sh8) & 0xffu, b1 = (L1 >> sh8) & 0xffu;
    const uint32_t b2 = (L2 >> sh8) & 0xffu, b3 = (L3 >> sh8) & 0xffu;
    const uint32_t h0 = (H0 >> sh8) & 0xffu, h1 = (H1 >> sh8) & 0xffu;
    const uint32_t lo[8] = {b0 & 15u, b1 & 15u, b2 & 15u, b3 & 15u,
                            b0 >> 4, b1 >> 4, b2 >> 4, b3 >> 4};
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const uint32_t h = (k & 1) ? h1 : h0;
        out[k] = (int)(lo[k] | (((h >> (2 * (k >> 1))) & 3u) << 4));
    }
}

/* 64-bit argmax key: high word = the value's bits made order-preserving as unsigned (-0 folded
 * into +0 so equal values tie), low word = ~index (a smaller index wins among equal values). */
__device__ __forceinline__ unsigned long long argmax_key(float v, int idx) {
    const float c = v == 0.0f ? 0.0f : v;
    uint32_t u = __float_as_uint(c);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)u << 32) | (unsigned long long)(0xffffffffu - (uint32_t)idx);
}

/* AMAX: also reduce to one (max value, first index) key per vector and workgroup (the head's
 * fused greedy argmax, finished by head_finish_k); Y may then be NULL (logits not
 * materialised). */
template <int NV, bool DOTS, bool AMAX>
__global__ __launch_bounds__(256) void q4k_mv_k(SegTable tab, int cols, int n, int v0,
                                                const int8_t *__restrict__ q,
                                                const float *__restrict__ d,
                                                const float *__restrict__ fs,
                                                int32_t *__restrict__ dots,
                                                unsigned long long *__restrict__ amax_key) {
    const int wave_raw = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (!AMAX && wave_raw >= tab.total_waves) return;
    const bool wave_live = wave_raw < tab.total_waves;
    const int wave = wave_live ? wave_raw : tab.total_waves - 1;
    const int lane = threadIdx.x & 63;

    /* segment of this wave (uniform) */
    const uint8_t *W = tab.s[0].W;
    float *Y = tab.s[0].Y;
    int rows = tab.s[0].rows, ystride = tab.s[0].ystride, wave0 = tab.s[0].wave0;
#pragma unroll
    for (int t = 1; t < NMX_MAX_SEGS; t++)
        if (t < tab.count && wave >= tab.s[t].wave0) {
            W = tab.s[t].W;
            Y = tab.s[t].Y;
            rows = tab.s[t].rows;
            ystride = tab.s[t].ystride;
            wave0 = tab.s[t].wave0;
        }

    const int row_raw = (wave - wave0) * 64 + lane;
    const bool valid = wave_live && row_raw < rows;
    const int row = row_raw < rows ? row_raw : rows - 1; /* clamped: the wave stays convergent */
    const int i = row & 3, sh8 = 8 * i;
    const int nsb = cols >> 8, nb = cols >> 5;
    const uint4 *tp = (const uint4 *)(W + (size_t)(row >> 2) * nsb * SB_BYTES);

    float acc[NV];
#pragma unroll
    for (int v = 0; v < NV; v++) acc[v] = 0.0f;

    for (int sb = 0; sb < nsb; sb++) {
        const uint4 *p = tp + sb * (SB_BYTES / 16);
        const uint4 a0 = p[0], a1 = p[1], a2 = p[2], a3 = p[3];
        uint4 c[8];
#pragma unroll
        for (int k = 0; k < 8; k++) c[k] = p[4 + 4 * k + i];

        const uint32_t dw = (i & 2) ? a0.y : a0.x, mw = (i & 2) ? a0.w : a0.z;
        const float D = half_bits_to_float(dw >> (16 * (i & 1)));
        const float M = half_bits_to_float(mw >> (16 * (i & 1)));
        int s6[8], m6[8];
        decode6(a1.x, a1.y, a1.z, a1.w, a2.x, a2.y, sh8, s6);
        decode6(a2.z, a2.w, a3.x, a3.y, a3.z, a3.w, sh8, m6);

#pragma unroll
        for (int k = 0; k < 8; k++) {
            const float sc = D * (float)s6[k]; /* exact: 6-bit x 11-bit mantissa */
            const float of = M * (float)m6[k];
            const int lo0 = (int)(c[k].x & 0x0f0f0f0fu), hi0 = (int)((c[k].x >> 4) & 0x0f0f0f0fu);
            const int lo1 = (int)(c[k].y & 0x0f0f0f0fu), hi1 = (int)((c[k].y >> 4) & 0x0f0f0f0fu);
            const int lo2 = (int)(c[k].z & 0x0f0f0f0fu), hi2 = (int)((c[k].z >> 4) & 0x0f0f0f0fu);
            const int lo3 = (int)(c[k].w & 0x0f0f0f0fu), hi3 = (int)((c[k].w >> 4) & 0x0f0f0f0fu);
            const int blk = sb * 8 + k;
#pragma unroll
            for (int v = 0; v < NV; v++) {
                const size_t ai = (size_t)blk * n + v0 + v;
                const int *xa = (const int *)(q + ai * 32);
                int dot = __builtin_amdgcn_sdot4(lo0, xa[0], 0, false);
                dot = __builtin_amdgcn_sdot4(lo1, xa[1], dot, false);
                dot = __builtin_amdgcn_sdot4(lo2, xa[2], dot, false);
                dot = __builtin_amdgcn_sdot4(lo3, xa[3], dot, false);
                dot = __builtin_amdgcn_sdot4(hi0, xa[4], dot, false);
                dot = __builtin_amdgcn_sdot4(hi1, xa[5], dot, false);
                dot = __builtin_amdgcn_sdot4(hi2, xa[6], dot, false);
                dot = __builtin_amdgcn_sdot4(hi3, xa[7], dot, false);
                acc[v] = __builtin_fmaf((float)dot, sc * d[ai], acc[v]);
                acc[v] = __builtin_fmaf(-of, fs[ai], acc[v]);
                if (DOTS && valid) dots[((size_t)(v0 + v) * rows + row) * nb + blk] = dot;
            }
        }
    }
    if (valid && Y) {
#pragma unroll
        for (int v = 0; v < NV; v++) Y[(size_t)(v0 + v) * ystride + row] = acc[v];
    }
    if (AMAX) {
        /* (value, index) order: larger value first, then the smaller index, so the winner is
         * the first index whose value equals the maximum (engine/src/forward_ops.c:387-409;
         * -0 == +0 compare equal, finite logits assumed as in the reference). Keys: 64-bit
         * (order-preserving value bits, complemented index), so the order is an unsigned max.
         * Per wave (shuffles), then per workgroup (LDS): one partial key per (vector,
         * workgroup), plain stores; head_finish_k reduces them after the kernel boundary. */
        __shared__ unsigned long long wkeys[4][MAX_NV];
        const int wv = threadIdx.x >> 6;
#pragma unroll
        for (int v = 0; v < NV; v++) {
            const unsigned long long key = nmx_max_u64_wave(valid ? argmax_key(acc[v], row) : 0ull);
            if (lane == 0) wkeys[wv][v] = key;
        }
        __syncthreads();
        if (threadIdx.x < NV) {
            unsigned long long key = wkeys[0][threadIdx.x];
            for (int w = 1; w < 4; w++) key = wkeys[w][threadIdx.x] > key ? wkeys[w][threadIdx.x] : key;
            amax_key[(size_t)(v0 + threadIdx.x) * gridDim.x + blockIdx.x] = key;
        }
    }
}

__global__ void copy_i32_k(const int32_t *__restrict__ src, int32_t *__restrict__ dst, int n) {
    for (int t = threadIdx.x; t < n; t += 64) dst[t] = src[t];
}

/* Bytes i (the lane's row in its tile) of four dwords, gathered into one dword. */
__device__ __forceinline__ uint32_t gather_byte4(uint32_t x0, uint32_t x1, uint32_t x2, uint32_t x3,
                                                 uint32_t sel) {
    const uint32_t t01 = __builtin_amdgcn_perm(x1, x0, sel); /* [x0.i, x1.i, 0, 0] */
    const uint32_t t23 = __builtin_amdgcn_perm(x3, x2, sel); /* [x2.i, x3.i, 0, 0] */
    return __builtin_amdgcn_perm(t23, t01, 0x05040100u);     /* [x0.i, x1.i, x2.i, x3.i] */
}

/* decode6 for one row, four values per dword: lo = bytes s[0..3], hi = bytes s[4..7]. sel
 * gathers byte i of two dwords into bytes 0-1, sel2 builds [h0, h1, h0, h1] from the two
 * high-pair dwords; the 2-bit fields of s[k] sit at bit 2 (k >> 1) of h(k & 1). */
__device__ __forceinline__ void decode6x4(uint32_t L0, uint32_t L1, uint32_t L2, uint32_t L3,
                                          uint32_t H0, uint32_t H1, uint32_t sel, uint32_t sel2,
                                          uint32_t &lo, uint32_t &hi) {
    const uint32_t P = gather_byte4(L0, L1, L2, L3, sel);
    const uint32_t Q = __builtin_amdgcn_perm(H1, H0, sel2);
    const uint32_t q03 = (Q & 0x0000ffffu) | ((Q >> 2) & 0xffff0000u);
    const uint32_t q47 = ((Q >> 4) & 0x0000ffffu) | ((Q >> 6) & 0xffff0000u);
    lo = (P & 0x0f0f0f0fu) | ((q03 & 0x03030303u) << 4);
    hi = ((P >> 4) & 0x0f0f0f0fu) | ((q47 & 0x03030303u) << 4);
}

__device__ __forceinline__ float byte_f(uint32_t w, int b) { return (float)((w >> (8 * b)) & 0xffu); }

/* The same matvec with the int32 block dots on the matrix cores, for 3..MAX_NV vectors (the
 * verify head). Row per lane as in q4k_mv_k: each lane still owns its row's (row, vector)
 * chains, in registers, in block order.
 *
 * One v_mfma_i32_32x32x32_i8 per half block (16 columns) gives every lane the dots of its own
 * row with all the vectors, because the activation operand is block-diagonal. B operand: lane
 * l supplies column l % 32 and K group l / 32 (16 bytes), here its own row's 16 nibbles as
 * bytes. Result: lane l holds C[m][l % 32] for m = 8 i + 4 (l / 32) + j in element 4 i + j.
 * A operand: lane l' supplies row m = l' % 32 of K group l' / 32. A[m][group g] is set to
 * vector v(m) = 4 (m / 8) + m % 4 only where g = (m / 4) % 2, and to zero elsewhere. Then
 * C[m][n] in lane n + 32 g takes only lane n + 32 g's own B bytes, so element v of every lane
 * is the dot of the lane's row with vector v. The K order is the B layout's (low then high
 * nibbles of code dwords 2h, 2h + 1), which the activation table copies.
 *
 * That table holds [block][half][vector] 16-byte rows and an all-zero copy of the same size.
 * Every workgroup builds it in LDS after its first superblock's weight loads are issued; lanes
 * whose A entries must be zero read the zero copy. Each block's operand reads are ordered
 * after the previous block's chain steps (an empty asm on the LDS offset), and each superblock's
 * weight loads after the last one's. Left alone, the compiler hoists every block's MFMAs and
 * holds all their results, which halves the waves per SIMD. WPG waves per workgroup share one
 * table and one partial argmax key per vector. */
template <int NV, bool AMAX, int WPG>
__global__ __launch_bounds__(64 * WPG) void q4k_mvx_k(SegTable tab, int cols, int n, int v0,
                                                 const int8_t *__restrict__ q,
                                                 const float *__restrict__ d,
                                                 const float *__restrict__ fs,
                                                 unsigned long long *__restrict__ amax_key) {
    typedef int v4i __attribute__((ext_vector_type(4)));
    typedef int v16i __attribute__((ext_vector_type(16)));
    extern __shared__ __align__(16) uint8_t xt[];
    const int nb = cols >> 5, ent = nb * 2 * NV, tbytes = ent * 16;
    const int wave_raw = blockIdx.x * WPG + (threadIdx.x >> 6);
    const bool wave_live = wave_raw < tab.total_waves; /* every wave reaches the barrier */
    const int wave = wave_live ? wave_raw : tab.total_waves - 1;
    const int lane = threadIdx.x & 63;
    const uint8_t *W = tab.s[0].W;
    float *Y = tab.s[0].Y;
    int rows = tab.s[0].rows, ystride = tab.s[0].ystride, wave0 = tab.s[0].wave0;
#pragma unroll
    for (int t = 1; t < NMX_MAX_SEGS; t++)
        if (t < tab.count && wave >= tab.s[t].wave0) {
            W = tab.s[t].W;
            Y = tab.s[t].Y;
            rows = tab.s[t].rows;
            ystride = tab.s[t].ystride;
            wave0 = tab.s[t].wave0;
        }
    const int row_raw = (wave - wave0) * 64 + lane;
    const bool valid = wave_live && row_raw < rows;
    const int row = row_raw < rows ? row_raw : rows - 1;
    const uint32_t i = (uint32_t)(row & 3);
    const int nsb = cols >> 8;
    const uint4 *tp = (const uint4 *)(W + (size_t)(row >> 2) * nsb * SB_BYTES);
    uint4 a0 = tp[0], a1 = tp[1], a2 = tp[2], a3 = tp[3], c[8];
#pragma unroll
    for (int k = 0; k < 8; k++) c[k] = tp[4 + 4 * k + i];

    for (int e = threadIdx.x; e < ent; e += 64 * WPG) {
        const int v = e % NV, bp = e / NV, h = bp & 1, blk = bp >> 1;
        const uint32_t *x = (const uint32_t *)(q + ((size_t)blk * n + v0 + v) * 32);
        *(uint4 *)(xt + (size_t)e * 16) = make_uint4(x[2 * h], x[4 + 2 * h], x[2 * h + 1], x[5 + 2 * h]);
        *(uint4 *)(xt + tbytes + (size_t)e * 16) = make_uint4(0, 0, 0, 0);
    }
    __syncthreads();
    const int m = lane & 31, vl = 4 * (m >> 3) + (m & 3);
    const bool diag = ((m >> 2) & 1) == (lane >> 5) && vl < NV;
    const uint8_t *xl = xt + (diag ? vl * 16 : tbytes);
    const uint32_t sel = 0x0c0c0400u | i | (i << 8), sel2 = i | ((i + 4) << 8) | (i << 16) | ((i + 4) << 24);
    const v16i zero = {};

    float acc[NV];
#pragma unroll
    for (int v = 0; v < NV; v++) acc[v] = 0.0f;
    for (int sb = 0; sb < nsb; sb++) {
        const uint32_t dw = (i & 2) ? a0.y : a0.x, mw = (i & 2) ? a0.w : a0.z;
        const float D = half_bits_to_float(dw >> (16 * (i & 1)));
        const float M = half_bits_to_float(mw >> (16 * (i & 1)));
        uint32_t S03, S47, M03, M47;
        decode6x4(a1.x, a1.y, a1.z, a1.w, a2.x, a2.y, sel, sel2, S03, S47);
        decode6x4(a2.z, a2.w, a3.x, a3.y, a3.z, a3.w, sel, sel2, M03, M47);
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const float sc = D * byte_f(k < 4 ? S03 : S47, k & 3); /* exact: 6-bit x 11-bit */
            const float of = M * byte_f(k < 4 ? M03 : M47, k & 3);
            const int blk = sb * 8 + k;
            const uint4 w = c[k];
            const v4i b0 = {(int)(w.x & 0x0f0f0f0fu), (int)((w.x >> 4) & 0x0f0f0f0fu),
                            (int)(w.y & 0x0f0f0f0fu), (int)((w.y >> 4) & 0x0f0f0f0fu)};
            const v4i b1 = {(int)(w.z & 0x0f0f0f0fu), (int)((w.z >> 4) & 0x0f0f0f0fu),
                            (int)(w.w & 0x0f0f0f0fu), (int)((w.w >> 4) & 0x0f0f0f0fu)};
            int xo = blk * 2 * NV * 16;
#pragma unroll
            for (int v = 0; v < NV; v++) asm volatile("" : "+v"(xo) : "v"(acc[v]));
            const v4i x0 = *(const v4i *)(xl + xo);
            const v4i x1 = *(const v4i *)(xl + xo + NV * 16);
            v16i C = __builtin_amdgcn_mfma_i32_32x32x32_i8(x0, b0, zero, 0, 0, 0);
            C = __builtin_amdgcn_mfma_i32_32x32x32_i8(x1, b1, C, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < NV; v++) {
                const size_t ai = (size_t)blk * n + v0 + v;
                acc[v] = __builtin_fmaf((float)C[v], sc * d[ai], acc[v]);
                acc[v] = __builtin_fmaf(-of, fs[ai], acc[v]);
            }
        }
        if (sb + 1 < nsb) {
            int nxt = (sb + 1) * (SB_BYTES / 16);
            asm volatile("" : "+v"(nxt) : "v"(acc[0]), "v"(acc[NV - 1]));
            const uint4 *p = tp + nxt;
            a0 = p[0], a1 = p[1], a2 = p[2], a3 = p[3];
#pragma unroll
            for (int k = 0; k < 8; k++) c[k] = p[4 + 4 * k + i];
        }
    }
    if (valid && Y) {
#pragma unroll
        for (int v = 0; v < NV; v++) Y[(size_t)(v0 + v) * ystride + row] = acc[v];
    }
    if (AMAX) { /* as in q4k_mv_k */
        __shared__ unsigned long long wkeys[WPG][MAX_NV];
        const int wv = threadIdx.x >> 6;
#pragma unroll
        for (int v = 0; v < NV; v++) {
            const unsigned long long key = nmx_max_u64_wave(valid ? argmax_key(acc[v], row) : 0ull);
            if (lane == 0) wkeys[wv][v] = key;
        }
        __syncthreads();
        if (threadIdx.x < NV) {
            unsigned long long key = wkeys[0][threadIdx.x];
            for (int w = 1; w < WPG; w++) key = wkeys[w][threadIdx.x] > key ? wkeys[w][threadIdx.x] : key;
            amax_key[(size_t)(v0 + threadIdx.x) * gridDim.x + blockIdx.x] = key;
        }
    }
}

/* The verify head (one matrix, cols = NSB x 256 known at compile time, 3..MAX_NV vectors): the
 * dots and chains of q4k_mvx_k, with the weight loads kept in flight across the arithmetic.
 * Superblock sb + 1's scale line is requested right after sb's scales are decoded, and its
 * code chunk k right after block k of sb has been unpacked into MFMA operands (the registers
 * are reused); every block's MFMA pair is issued one block ahead of the previous block's chain
 * steps. Scheduling barriers keep each block's work together, so each in-order wait on the
 * load counter names only what that block needs, and every wave has about one superblock of
 * requests outstanding all the time instead of one superblock at a time. The activation
 * table's sources are requested before the first weights and stored to LDS after them.
 * Results equal q4k_mvx_k's bit for bit (same operations per (row, vector) chain, in order).
 * Leading arguments are what the first requests need (preloaded into SGPRs). dcopy (not NULL):
 * workgroup 0 copies drafts[0..ndr) there, so that a consumer that also rewrites the drafts'
 * row (the accept commit writes the bonus to vt[a + 1]) reads them from a copy no workgroup of
 * its own launch writes. */
template <int NV, int NSB, int WPG, bool ONEPASS>
__global__ __launch_bounds__(64 * WPG) void q4k_head_k(const uint8_t *__restrict__ W,
                                                     const int8_t *__restrict__ q,
                                                     const float *__restrict__ d,
                                                     const float *__restrict__ fs,
                                                     unsigned long long *__restrict__ amax_key,
                                                     int rows, int n_arg, int v0_arg,
                                                     float *__restrict__ Y,
                                                     const int32_t *__restrict__ drafts,
                                                     int32_t *__restrict__ dcopy, int ndr) {
    /* ONEPASS (n == NV, v0 == 0): the activations' (d, fsum) offsets are compile-time
     * constants, so each block's scalar loads are few wide ones instead of 2 NV computed ones */
    const int n = ONEPASS ? NV : n_arg, v0 = ONEPASS ? 0 : v0_arg;
    typedef int v4i __attribute__((ext_vector_type(4)));
    typedef int v16i __attribute__((ext_vector_type(16)));
    constexpr int NB = NSB * 8, ENT = NB * 2 * NV, TB = ENT * 16;
    constexpr int TPT = (ENT + 64 * WPG - 1) / (64 * WPG);
    __shared__ __align__(16) uint8_t xt[2 * TB + 16]; /* table, zero copy, one junk slot */
    const int total_waves = (rows + 63) / 64;
    const int wave_raw = blockIdx.x * WPG + (threadIdx.x >> 6);
    const bool wave_live = wave_raw < total_waves; /* every wave reaches the barriers */
    const int wave = wave_live ? wave_raw : total_waves - 1;
    const int lane = threadIdx.x & 63;
    const int row_raw = wave * 64 + lane;
    const bool valid = wave_live && row_raw < rows;
    const int row = row_raw < rows ? row_raw : rows - 1;
    const uint32_t i = (uint32_t)(row & 3);
    /* the activation table's sources: entry e = (block, half, vector), 16 bytes each */
    uint2 ta[TPT], tb[TPT];
#pragma unroll
    for (int t = 0; t < TPT; t++) {
        const int e = threadIdx.x + t * 64 * WPG;
        const int ee = e < ENT ? e : ENT - 1;
        const int v = ee % NV, bp = ee / NV, h = bp & 1, blk = bp >> 1;
        const uint32_t *x = (const uint32_t *)(q + ((size_t)blk * n + v0 + v) * 32);
        ta[t] = *(const uint2 *)(x + 2 * h);
        tb[t] = *(const uint2 *)(x + 4 + 2 * h);
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    const uint4 *tp = (const uint4 *)(W + (size_t)(row >> 2) * NSB * SB_BYTES);
    uint4 a0 = tp[0], a1 = tp[1], a2 = tp[2], a3 = tp[3], c[8];
#pragma unroll
    for (int k = 0; k < 8; k++) c[k] = tp[4 + 4 * k + i];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < TPT; t++) {
        const int e = threadIdx.x + t * 64 * WPG;
        const int o0 = e < ENT ? e * 16 : 2 * TB, o1 = e < ENT ? TB + e * 16 : 2 * TB;
        *(uint4 *)(xt + o0) = make_uint4(ta[t].x, tb[t].x, ta[t].y, tb[t].y);
        *(uint4 *)(xt + o1) = make_uint4(0, 0, 0, 0);
    }
    __syncthreads();
    const int m = lane & 31, vl = 4 * (m >> 3) + (m & 3);
    const bool diag = ((m >> 2) & 1) == (lane >> 5) && vl < NV;
    const uint8_t *xl = xt + (diag ? vl * 16 : TB);
    const uint32_t sel = 0x0c0c0400u | i | (i << 8), sel2 = i | ((i + 4) << 8) | (i << 16) | ((i + 4) << 24);
    const v16i zero = {};
    float acc[NV];
#pragma unroll
    for (int v = 0; v < NV; v++) acc[v] = 0.0f;
    auto unpack = [](const uint4 w, v4i &b0, v4i &b1) {
        b0 = v4i{(int)(w.x & 0x0f0f0f0fu), (int)((w.x >> 4) & 0x0f0f0f0fu),
                 (int)(w.y & 0x0f0f0f0fu), (int)((w.y >> 4) & 0x0f0f0f0fu)};
        b1 = v4i{(int)(w.z & 0x0f0f0f0fu), (int)((w.z >> 4) & 0x0f0f0f0fu),
                 (int)(w.w & 0x0f0f0f0fu), (int)((w.w >> 4) & 0x0f0f0f0fu)};
    };
    v16i Cc; /* block 0's products, then always one block ahead of the chain */
    {
        v4i b0, b1;
        unpack(c[0], b0, b1);
        const v4i x0 = *(const v4i *)(xl), x1 = *(const v4i *)(xl + NV * 16);
        Cc = __builtin_amdgcn_mfma_i32_32x32x32_i8(x0, b0, zero, 0, 0, 0);
        Cc = __builtin_amdgcn_mfma_i32_32x32x32_i8(x1, b1, Cc, 0, 0, 0);
    }
#pragma unroll
    for (int sb = 0; sb < NSB; sb++) {
        const uint32_t dw = (i & 2) ? a0.y : a0.x, mw = (i & 2) ? a0.w : a0.z;
        const float D = half_bits_to_float(dw >> (16 * (i & 1)));
        const float M = half_bits_to_float(mw >> (16 * (i & 1)));
        uint32_t S03, S47, M03, M47;
        decode6x4(a1.x, a1.y, a1.z, a1.w, a2.x, a2.y, sel, sel2, S03, S47);
        decode6x4(a2.z, a2.w, a3.x, a3.y, a3.z, a3.w, sel, sel2, M03, M47);
        const uint4 *p = tp + (sb + 1) * (SB_BYTES / 16);
        __builtin_amdgcn_sched_barrier(0);
        if (sb + 1 < NSB) { /* the next scale line and chunk 0 (block 0's unpack is done) */
            a0 = p[0], a1 = p[1], a2 = p[2], a3 = p[3];
            c[0] = p[4 + i];
        }
#pragma unroll
        for (int k = 0; k < 8; k++) {
            __builtin_amdgcn_sched_barrier(0);
            const int blk = sb * 8 + k;
            v16i Cn = Cc;
            if (blk + 1 < NB) { /* the next block's products */
                const int kn = (k + 1) & 7;
                v4i b0, b1;
                unpack(c[kn], b0, b1);
                if (kn != 0 && sb + 1 < NSB) c[kn] = p[4 + 4 * kn + i];
                int xo = (blk + 1) * 2 * NV * 16;
                asm volatile("" : "+v"(xo) : "v"(Cc[0])); /* keeps the MFMAs in block order */
                const v4i x0 = *(const v4i *)(xl + xo);
                const v4i x1 = *(const v4i *)(xl + xo + NV * 16);
                Cn = __builtin_amdgcn_mfma_i32_32x32x32_i8(x0, b0, zero, 0, 0, 0);
                Cn = __builtin_amdgcn_mfma_i32_32x32x32_i8(x1, b1, Cn, 0, 0, 0);
            }
            const float sc = D * byte_f(k < 4 ? S03 : S47, k & 3); /* exact: 6-bit x 11-bit */
            const float of = M * byte_f(k < 4 ? M03 : M47, k & 3);
#pragma unroll
            for (int v = 0; v < NV; v++) {
                const size_t ai = (size_t)blk * n + v0 + v;
                acc[v] = __builtin_fmaf((float)Cc[v], sc * d[ai], acc[v]);
                acc[v] = __builtin_fmaf(-of, fs[ai], acc[v]);
            }
            Cc = Cn;
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    if (valid && Y) {
#pragma unroll
        for (int v = 0; v < NV; v++) Y[(size_t)(v0 + v) * rows + row] = acc[v];
    }
    if (dcopy && blockIdx.x == 0 && threadIdx.x < ndr) dcopy[threadIdx.x] = drafts[threadIdx.x];
    __shared__ unsigned long long wkeys[WPG][MAX_NV];
    const int wv = threadIdx.x >> 6;
#pragma unroll
    for (int v = 0; v < NV; v++) {
        const unsigned long long key = nmx_max_u64_wave(valid ? argmax_key(acc[v], row) : 0ull);
        if (lane == 0) wkeys[wv][v] = key;
    }
    __syncthreads();
    if (threadIdx.x < NV) {
        unsigned long long key = wkeys[0][threadIdx.x];
        for (int w = 1; w < WPG; w++) key = wkeys[w][threadIdx.x] > key ? wkeys[w][threadIdx.x] : key;
        amax_key[(size_t)(v0 + threadIdx.x) * gridDim.x + blockIdx.x] = key;
    }
}

/* The commit of the accepted run that head_finish_k can apply itself (engine/src/spec.c:
 * 346-351): vt[a + 1] = bonus, ctl[1] = e = a + 1, and the host mailbox [a, bonus, vt[0..nvt)
 * after the update] followed by mb[2 + nvt] = 1 with a system-scope release. vt NULL: none. */
struct FinishCommit {
    int32_t *vt, *ctl, *mb;
    int nvt;
    int32_t *adv; /* not NULL: adv[0] += adv[1] last (a round's n_past += e) */
};

/* The one-row head with its input's RMSNorm inside (nmx_head_row_accept_to): row *idx + off of
 * x (+ add), clamped to [0, nrows), normed with w (rms4_load / rms4_finish: the arithmetic of
 * nmx_rmsnorm_row) into y (written by workgroup 0) and into a one-vector A8 in LDS; then the
 * dots of the row against 64 rows of W per workgroup, split over the cols / 256 superblocks: wave
 * s requests superblock s of its 64 rows at entry (right behind the norm's row), computes that
 * superblock's exact int32 block dots with v_dot4 (activations from LDS) and its (float)dot,
 * (D s) d, -(M m), fsum records in registers, and the fp32 chain then runs wave 0 -> 1 -> ... in
 * column order, the running accumulator handed over through LDS, so each (row) chain performs
 * the reference's operations in its order (engine/src/kern_quant.c:148-245) while every
 * superblock's loads are in flight at once. One partial argmax key per workgroup. cols <= 1024
 * (64 cols / 4 threads: the norm's float4 per thread); W has rows rows. The leading arguments
 * are what the first requests need (preloaded with the wave). */
constexpr int MVR_MAX_COLS = 1024;

__global__ __launch_bounds__(256) void q4k_mvr_k(const int32_t *__restrict__ idx,
                                                 const float *__restrict__ x,
                                                 const float *__restrict__ add,
                                                 const float *__restrict__ w,
                                                 const uint8_t *__restrict__ W, int off, int nrows,
                                                 int x_stride, int add_stride, int cols, int rows,
                                                 float eps, float *__restrict__ y,
                                                 unsigned long long *__restrict__ amax_key) {
    __shared__ __align__(16) int8_t s_q[MVR_MAX_COLS];
    __shared__ float s_d[MVR_MAX_COLS / 32], s_fs[MVR_MAX_COLS / 32];
    __shared__ __align__(16) float s_sq[4 * cm_stride(MVR_MAX_COLS) + 4];
    __shared__ float s_red[8], hand[64];
    /* the norm's row first */
    const int ri = *idx + off;
    const size_t r = (size_t)(ri < 0 ? 0 : ri >= nrows ? nrows - 1 : ri);
    float4 xv[1], av[1], wv[1];
    rms4_load<1>(x + r * x_stride, add ? add + r * add_stride : nullptr, w, cols, xv, av, wv);

    const int sb = threadIdx.x >> 6, nsb = cols >> 8; /* this wave's superblock */
    const int lane = threadIdx.x & 63;
    const int row_raw = blockIdx.x * 64 + lane;
    const bool valid = row_raw < rows;
    const int row = valid ? row_raw : rows - 1;
    const int i = row & 3, sh8 = 8 * i;
    const uint4 *p = (const uint4 *)(W + ((size_t)(row >> 2) * nsb + sb) * SB_BYTES);
    const uint4 a0 = p[0], a1 = p[1], a2 = p[2], a3 = p[3];
    uint4 c[8];
#pragma unroll
    for (int k = 0; k < 8; k++) c[k] = p[4 + 4 * k + i];

    rms4_finish<1>(xv, av, wv, add != nullptr, nullptr, cols, eps, blockIdx.x == 0 ? y : nullptr,
                   s_q, s_d, s_fs, 1, 0, s_sq, s_red);
    __syncthreads(); /* the A8 row is in LDS */

    const uint32_t dw = (i & 2) ? a0.y : a0.x, mw = (i & 2) ? a0.w : a0.z;
    const float D = half_bits_to_float(dw >> (16 * (i & 1)));
    const float M = half_bits_to_float(mw >> (16 * (i & 1)));
    int s6[8], m6[8];
    decode6(a1.x, a1.y, a1.z, a1.w, a2.x, a2.y, sh8, s6);
    decode6(a2.z, a2.w, a3.x, a3.y, a3.z, a3.w, sh8, m6);
    float tf[8], tm[8], to[8], tfs[8];
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const int blk = sb * 8 + k;
        const int4 x0 = *(const int4 *)(s_q + blk * 32), x1 = *(const int4 *)(s_q + blk * 32 + 16);
        int dot = __builtin_amdgcn_sdot4((int)(c[k].x & 0x0f0f0f0fu), x0.x, 0, false);
        dot = __builtin_amdgcn_sdot4((int)(c[k].y & 0x0f0f0f0fu), x0.y, dot, false);
        dot = __builtin_amdgcn_sdot4((int)(c[k].z & 0x0f0f0f0fu), x0.z, dot, false);
        dot = __builtin_amdgcn_sdot4((int)(c[k].w & 0x0f0f0f0fu), x0.w, dot, false);
        dot = __builtin_amdgcn_sdot4((int)((c[k].x >> 4) & 0x0f0f0f0fu), x1.x, dot, false);
        dot = __builtin_amdgcn_sdot4((int)((c[k].y >> 4) & 0x0f0f0f0fu), x1.y, dot, false);
        dot = __builtin_amdgcn_sdot4((int)((c[k].z >> 4) & 0x0f0f0f0fu), x1.z, dot, false);
        dot = __builtin_amdgcn_sdot4((int)((c[k].w >> 4) & 0x0f0f0f0fu), x1.w, dot, false);
        tf[k] = (float)dot;
        tm[k] = (D * (float)s6[k]) * s_d[blk]; /* exact: 6-bit x 11-bit mantissa, then d */
        to[k] = -(M * (float)m6[k]);
        tfs[k] = s_fs[blk];
    }
    /* the chain: acc = fma((float)dot, (D*s)*d, acc); acc = fma(-(M*m), fsum, acc), block by
     * block, superblock 0 first */
    float acc = 0.0f;
    for (int turn = 0; turn < nsb; turn++) {
        if (turn == sb) {
            if (sb > 0) acc = hand[lane];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                acc = __builtin_fmaf(tf[k], tm[k], acc);
                acc = __builtin_fmaf(to[k], tfs[k], acc);
            }
            if (sb + 1 < nsb) hand[lane] = acc;
        }
        __syncthreads();
    }
    /* the argmax key of the workgroup's 64 rows, from the last superblock's wave */
    if (sb == nsb - 1) {
        const unsigned long long key = nmx_max_u64_wave(valid ? argmax_key(acc, row) : 0ull);
        if (lane == 0) amax_key[blockIdx.x] = key;
    }
}

/* Argmax of every row from the per-workgroup partial keys, then the acceptance loop of the
 * reference (engine/src/spec.c:340-345): a = 0; g = argmax(row 0); while a < k and
 * drafts[a] == g: a++, g = argmax(row a). out = [a, g, argmax(row 0..n-1)]; then the commit
 * fc when given. One workgroup of 1024 threads; the drafts (and vt for the mailbox) are
 * requested first, every partial is loaded once, all loads issued before the reduction, so
 * the acceptance loop reads LDS only. */
__global__ __launch_bounds__(1024) void head_finish_k(const unsigned long long *__restrict__ keys,
                                                      int nblk, int n,
                                                      const int32_t *drafts,
                                                      int32_t *__restrict__ out,
                                                      int32_t *__restrict__ tok_dst,
                                                      FinishCommit fc) {
    __shared__ unsigned long long red[16][8];
    __shared__ int am[64], sdr[64], svt[1024];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    bool staged = false;
    for (int t0 = 0; t0 < n; t0 += 8) {
        unsigned long long k[8];
#pragma unroll
        for (int j = 0; j < 8; j++) k[j] = 0ull;
        for (int b = tid; b < nblk; b += 1024) {
            unsigned long long o[8]; /* every row's load issued before the first compare */
#pragma unroll
            for (int j = 0; j < 8; j++)
                if (t0 + j < n) o[j] = keys[(size_t)(t0 + j) * nblk + b];
#pragma unroll
            for (int j = 0; j < 8; j++)
                if (t0 + j < n) k[j] = o[j] > k[j] ? o[j] : k[j];
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
            if (t0 + j >= n) break; /* uniform: only the pass's vectors */
            k[j] = nmx_max_u64_wave(k[j]);
            if (lane == 0) red[wv][j] = k[j];
        }
        if (!staged) { /* the drafts and vt after the first keys: loads complete in order, so
                        * their LDS stores cannot hold back the key requests */
            const int dr = drafts && tid < n - 1 ? drafts[tid] : 0;
            const int vv = fc.mb && tid < fc.nvt ? fc.vt[tid] : 0;
            if (tid < n - 1) sdr[tid] = dr;
            if (tid < fc.nvt) svt[tid] = vv;
            staged = true;
        }
        __syncthreads();
        if (tid < 8 && t0 + tid < n) {
            unsigned long long m = red[0][tid];
            for (int w = 1; w < 16; w++) m = red[w][tid] > m ? red[w][tid] : m;
            am[t0 + tid] = (int)(0xffffffffu - (unsigned)(m & 0xffffffffull));
        }
        __syncthreads();
    }
    if (tid == 0) {
        int a = 0, g = am[0];
        while (a < n - 1 && sdr[a] == g) {
            a++;
            g = am[a];
        }
        out[0] = a;
        out[1] = g;
        for (int t = 0; t < n; t++) out[2 + t] = am[t];
        if (tok_dst) *tok_dst = g;
        if (fc.vt) {
            fc.vt[a + 1] = g;
            fc.ctl[1] = a + 1;
            if (fc.mb) {
                fc.mb[0] = a;
                fc.mb[1] = g;
                for (int i = 0; i < fc.nvt; i++) fc.mb[2 + i] = i == a + 1 ? g : svt[i];
                __hip_atomic_store(fc.mb + 2 + fc.nvt, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
            }
        }
        if (fc.adv) fc.adv[0] = fc.adv[0] + fc.adv[1];
    }
}

/* K-split variant for matrices with few rows (the per-layer projections): a workgroup owns
 * 64 rows x ONE vector and KS waves split the superblocks (SBW each). Every wave computes its
 * blocks' int dots with the same wave-uniform activations and keeps (float)dot, (D*s)*d and
 * -(M*m) in registers; then the fp32 chain runs wave 0 -> 1 -> ... -> KS-1 in column order, the
 * running accumulator handed over through LDS, so the per-(row, vector) operation sequence is
 * exactly the reference's. Grid: (64-row groups over all segments) x vectors. */
template <int SBW, bool DOTS>
__global__ __launch_bounds__(1024) void q4k_mv_ks_k(SegTable tab, int cols, int n, int KS,
                                                   const int8_t *__restrict__ q,
                                                   const float *__restrict__ d,
                                                   const float *__restrict__ fs,
                                                   int32_t *__restrict__ dots) {
    __shared__ float hand[64];
    const int grp = blockIdx.x, v = blockIdx.y;
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;

    const uint8_t *W = tab.s[0].W;
    float *Y = tab.s[0].Y;
    int rows = tab.s[0].rows, ystride = tab.s[0].ystride, grp0 = tab.s[0].wave0;
#pragma unroll
    for (int t = 1; t < NMX_MAX_SEGS; t++)
        if (t < tab.count && grp >= tab.s[t].wave0) {
            W = tab.s[t].W;
            Y = tab.s[t].Y;
            rows = tab.s[t].rows;
            ystride = tab.s[t].ystride;
            grp0 = tab.s[t].wave0;
        }
    const int row_raw = (grp - grp0) * 64 + lane;
    const bool valid = row_raw < rows;
    const int row = valid ? row_raw : rows - 1;
    const int i = row & 3, sh8 = 8 * i;
    const int nsb = cols >> 8, nb = cols >> 5;
    const int sb0 = w * SBW;
    const uint4 *tp = (const uint4 *)(W + (size_t)(row >> 2) * nsb * SB_BYTES);

    float tf[SBW * 8], tm[SBW * 8], to[SBW * 8], tfs[SBW * 8];
#pragma unroll
    for (int u = 0; u < SBW; u++) {
        const int sb = sb0 + u;
        if (sb >= nsb) { /* uniform: a short last wave */
#pragma unroll
            for (int k = 0; k < 8; k++) tf[u * 8 + k] = tm[u * 8 + k] = to[u * 8 + k] = tfs[u * 8 + k] = 0.0f;
            continue;
        }
        const uint4 *p = tp + sb * (SB_BYTES / 16);
        const uint4 a0 = p[0], a1 = p[1], a2 = p[2], a3 = p[3];
        uint4 c[8];
#pragma unroll
        for (int k = 0; k < 8; k++) c[k] = p[4 + 4 * k + i];
        const uint32_t dw = (i & 2) ? a0.y : a0.x, mw = (i & 2) ? a0.w : a0.z;
        const float D = half_bits_to_float(dw >> (16 * (i & 1)));
        const float M = half_bits_to_float(mw >> (16 * (i & 1)));
        int s6[8], m6[8];
        decode6(a1.x, a1.y, a1.z, a1.w, a2.x, a2.y, sh8, s6);
        decode6(a2.z, a2.w, a3.x, a3.y, a3.z, a3.w, sh8, m6);
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int blk = sb * 8 + k;
            const size_t ai = (size_t)blk * n + v;
            const int *xa = (const int *)(q + ai * 32);
            int dot = __builtin_amdgcn_sdot4((int)(c[k].x & 0x0f0f0f0fu), xa[0], 0, false);
            dot = __builtin_amdgcn_sdot4((int)(c[k].y & 0x0f0f0f0fu), xa[1], dot, false);
            dot = __builtin_amdgcn_sdot4((int)(c[k].z & 0x0f0f0f0fu), xa[2], dot, false);
            dot = __builtin_amdgcn_sdot4((int)(c[k].w & 0x0f0f0f0fu), xa[3], dot, false);
            dot = __builtin_amdgcn_sdot4((int)((c[k].x >> 4) & 0x0f0f0f0fu), xa[4], dot, false);
            dot = __builtin_amdgcn_sdot4((int)((c[k].y >> 4) & 0x0f0f0f0fu), xa[5], dot, false);
            dot = __builtin_amdgcn_sdot4((int)((c[k].z >> 4) & 0x0f0f0f0fu), xa[6], dot, false);
            dot = __builtin_amdgcn_sdot4((int)((c[k].w >> 4) & 0x0f0f0f0fu), xa[7], dot, false);
            if (DOTS && valid) dots[((size_t)v * rows + row) * nb + blk] = dot;
            tf[u * 8 + k] = (float)dot;
            tm[u * 8 + k] = (D * (float)s6[k]) * d[ai];
            to[u * 8 + k] = -(M * (float)m6[k]);
            tfs[u * 8 + k] = fs[ai];
        }
    }

    float acc = 0.0f;
    for (int turn = 0; turn < KS; turn++) {
        if (turn == w) {
            if (w > 0) acc = hand[lane];
#pragma unroll
            for (int j = 0; j < SBW * 8; j++) {
                if (sb0 + j / 8 < nsb) {
                    acc = __builtin_fmaf(tf[j], tm[j], acc);
                    acc = __builtin_fmaf(to[j], tfs[j], acc);
                }
            }
            if (w + 1 < KS) hand[lane] = acc;
            else if (valid) Y[(size_t)v * ystride + row] = acc;
        }
        __syncthreads();
    }
}

/* Prefill chunks (more than 8 vectors): the int32 block dots on the matrix cores, one
 * v_mfma_i32_16x16x32_i8 per (16 rows, 16 vectors, 32-column block), then the reference's
 * ordered per-block FMA pair on the 16 x 16 result in registers.
 *
 * A wave owns 16 rows (four 4-row tiles) and NT tiles of 16 vectors; a workgroup of WAVES waves
 * shares the activations of its vectors, staged in LDS one superblock at a time; the weights and
 * activations of superblock sb + DIST are loaded into registers while sb is used (DIST = 2 for
 * single-wave workgroups, whose latency nothing else on the CU hides; 1 where VGPRs are
 * short).
 * MFMA operand layout (16x16x32 i8, checked on gfx950): lane l supplies row (A) / column (B)
 * l % 16 and the 8 K values of group g = l / 16; the result C[4 (l / 16) + j][l % 16] lands in
 * the lane's element j. The 32 columns of a block may be dealt to the K positions in any order
 * that is the same for both operands, since the int32 sum is exact: group g takes the low
 * nibbles of code bytes 4g..4g+3 (columns 4g..4g+3) and their high nibbles (columns
 * 16+4g..16+4g+3), and the staged activations are permuted to the same order. The lane's four
 * result rows are the four rows of tile l / 16, whose 6-bit scales and mins for block k are
 * decoded four at a time (one byte per row). Per (row, vector) the lane then runs
 * acc = fma((float)dot, (D*s)*d, acc); acc = fma(-(M*m), fsum, acc) block by block. */
template <int NT, int WAVES, int DIST>
__global__ __launch_bounds__(64 * WAVES) void q4k_mm_k(SegTable tab, int cols, int n,
                                                       const int8_t *__restrict__ q,
                                                       const float *__restrict__ d,
                                                       const float *__restrict__ fs) {
    typedef int v4i __attribute__((ext_vector_type(4)));
    constexpr int NV16 = NT * 16, T = 64 * WAVES;
    constexpr int SE = (8 * NV16 + T - 1) / T; /* staged (block, vector) entries per thread */
    __shared__ __align__(16) uint8_t xs[8 * NV16 * 32]; /* [block][vector][g][8 B] */
    __shared__ float2 xdf[8 * NV16];                    /* (d, fsum) per [block][vector] */
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int grp_raw = blockIdx.x * WAVES + w; /* 16-row group over all segments */
    const bool live = grp_raw < tab.total_waves;
    const int grp = live ? grp_raw : tab.total_waves - 1;
    const uint8_t *W = tab.s[0].W;
    float *Y = tab.s[0].Y;
    int rows = tab.s[0].rows, ystride = tab.s[0].ystride, grp0 = tab.s[0].wave0;
#pragma unroll
    for (int t = 1; t < NMX_MAX_SEGS; t++)
        if (t < tab.count && grp >= tab.s[t].wave0) {
            W = tab.s[t].W;
            Y = tab.s[t].Y;
            rows = tab.s[t].rows;
            ystride = tab.s[t].ystride;
            grp0 = tab.s[t].wave0;
        }
    const int nsb = cols >> 8;
    const int row0 = (grp - grp0) * 16;
    const int vt0 = blockIdx.y * NV16, nvw = n - vt0 < NV16 ? n - vt0 : NV16;
    const int g = lane >> 4, c16 = lane & 15;
    /* operand A: row row0 + c16 (clamped into the matrix), code dword g of each block */
    const int arow = row0 + c16 < rows ? row0 + c16 : rows - 1;
    const uint8_t *ap = W + (size_t)(arow >> 2) * nsb * SB_BYTES + 64 + 16 * (arow & 3) + 4 * g;
    /* result rows: tile g of the group (clamped), vector vt0 + 16 t + c16 */
    const int erow0 = row0 + 4 * g < rows ? row0 + 4 * g : rows - 4;
    const uint4 *hp = (const uint4 *)(W + (size_t)(erow0 >> 2) * nsb * SB_BYTES);

    /* one superblock's inputs; DIST sets, loaded DIST superblocks ahead of their use */
    struct Buf {
        uint32_t cw[8];
        uint4 h[4], x0[SE], x1[SE];
        float2 df[SE];
    };
    auto fetch = [&](Buf &B, int sb) {
#pragma unroll
        for (int k = 0; k < 8; k++) B.cw[k] = *(const uint32_t *)(ap + (size_t)sb * SB_BYTES + 64 * k);
#pragma unroll
        for (int u = 0; u < 4; u++) B.h[u] = hp[sb * 36 + u];
#pragma unroll
        for (int u = 0; u < SE; u++) {
            const int e = u * T + tid, k = e / NV16, v = e - k * NV16;
            B.x0[u] = B.x1[u] = make_uint4(0, 0, 0, 0);
            B.df[u] = make_float2(0.0f, 0.0f);
            if (e < 8 * NV16 && v < nvw) {
                const size_t ai = (size_t)(sb * 8 + k) * n + vt0 + v;
                B.x0[u] = *(const uint4 *)(q + ai * 32);
                B.x1[u] = *(const uint4 *)(q + ai * 32 + 16);
                B.df[u] = make_float2(d[ai], fs[ai]);
            }
        }
    };

    float acc[NT][4];
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[t][j] = 0.0f;
    const v4i zero = {0, 0, 0, 0};

    /* superblock sb from buffer B, whose set is then refilled with superblock sb + DIST */
    auto step = [&](Buf &B, int sb) {
        uint32_t cw[8];
#pragma unroll
        for (int k = 0; k < 8; k++) cw[k] = B.cw[k];
        const uint4 h0 = B.h[0], h1 = B.h[1], h2 = B.h[2], h3 = B.h[3];
        __syncthreads(); /* the previous superblock's activations are consumed */
#pragma unroll
        for (int u = 0; u < SE; u++) {
            const int e = u * T + tid;
            if (e < 8 * NV16) {
                uint2 *dst = (uint2 *)(xs + (size_t)e * 32);
                dst[0] = make_uint2(B.x0[u].x, B.x1[u].x);
                dst[1] = make_uint2(B.x0[u].y, B.x1[u].y);
                dst[2] = make_uint2(B.x0[u].z, B.x1[u].z);
                dst[3] = make_uint2(B.x0[u].w, B.x1[u].w);
                xdf[e] = B.df[u];
            }
        }
        if (sb + DIST < nsb) fetch(B, sb + DIST);
        __syncthreads();
        float Dj[4], Mj[4];
        Dj[0] = half_bits_to_float(h0.x), Dj[1] = half_bits_to_float(h0.x >> 16);
        Dj[2] = half_bits_to_float(h0.y), Dj[3] = half_bits_to_float(h0.y >> 16);
        Mj[0] = half_bits_to_float(h0.z), Mj[1] = half_bits_to_float(h0.z >> 16);
        Mj[2] = half_bits_to_float(h0.w), Mj[3] = half_bits_to_float(h0.w >> 16);
        const uint32_t SL[4] = {h1.x, h1.y, h1.z, h1.w}, SH[2] = {h2.x, h2.y};
        const uint32_t ML[4] = {h2.z, h2.w, h3.x, h3.y}, MH[2] = {h3.z, h3.w};
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t c = cw[k];
            const long a = (long)(c & 0x0f0f0f0fu) | ((long)((c >> 4) & 0x0f0f0f0fu) << 32);
            /* 6-bit scale / min of block k for the tile's rows 0..3, one byte each */
            const int sl = 4 * (k >> 2), sh = 2 * (k >> 1);
            const uint32_t s4 = ((SL[k & 3] >> sl) & 0x0f0f0f0fu) | (((SH[k & 1] >> sh) & 0x03030303u) << 4);
            const uint32_t m4 = ((ML[k & 3] >> sl) & 0x0f0f0f0fu) | (((MH[k & 1] >> sh) & 0x03030303u) << 4);
            float sc[4], of[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                sc[j] = Dj[j] * (float)((s4 >> (8 * j)) & 0xffu); /* exact: 6-bit x 11-bit */
                of[j] = Mj[j] * (float)((m4 >> (8 * j)) & 0xffu);
            }
#pragma unroll
            for (int t = 0; t < NT; t++) {
                const int e = k * NV16 + 16 * t + c16;
                const long b = *(const long *)(xs + (size_t)e * 32 + 8 * g);
                const v4i dot = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, zero, 0, 0, 0);
                const float2 df = xdf[e];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    acc[t][j] = __builtin_fmaf((float)dot[j], sc[j] * df.x, acc[t][j]);
                    acc[t][j] = __builtin_fmaf(-of[j], df.y, acc[t][j]);
                }
            }
        }
    };

    if constexpr (DIST == 2) {
        Buf A, B;
        fetch(A, 0);
        if (nsb > 1) fetch(B, 1);
        for (int sb = 0; sb < nsb; sb += 2) {
            step(A, sb);
            if (sb + 1 < nsb) step(B, sb + 1);
        }
    } else {
        Buf A;
        fetch(A, 0);
        for (int sb = 0; sb < nsb; sb++) step(A, sb);
    }
    if (!live) return;
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const int v = vt0 + 16 * t + c16;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int row = row0 + 4 * g + j;
            if (v < n && row < rows) Y[(size_t)v * ystride + row] = acc[t][j];
        }
    }
}

/* A8 quantization, one 32-lane half-wave per (block b, vector v) unit; unit index = b * n + v,
 * which is the block-major output index (engine/src/kern.h:19-27). Cross-lane max of |x| and
 * the int sum are exact in any order; 127 / amax and amax / 127 are IEEE divides; the code is
 * round-half-even (engine/src/kern_act.c:14-42, engine/metal/kernels.metal:9-27). */
__global__ __launch_bounds__(256) void quant_a8_k(const float *__restrict__ X, int n, int cols,
                                                  int8_t *__restrict__ q, float *__restrict__ d,
                                                  float *__restrict__ fs) {
    const int unit = (blockIdx.x * 256 + threadIdx.x) >> 5;
    const int nb = cols >> 5;
    if (unit >= nb * n) return; /* the whole half-wave leaves together */
    const int b = unit / n, v = unit - b * n;
    const float x = X[(size_t)v * cols + b * 32 + (threadIdx.x & 31)];
    nmx_a8_store(x, q + (size_t)unit * 32, d + unit, fs + unit);
}

/* Waves per workgroup of the matrix-core matvec: 16 (one 1024-thread workgroup per CU: one
 * activation table per CU instead of about four, and a quarter of the partial argmax keys for
 * the reduction) once the row groups fill MVX_BIG_WAVES waves, else 4 (more CUs for smaller
 * matrices). */
constexpr int MVX_BIG_WAVES = 16 * 200;

bool mvx_used(int nv, int cols, bool dots) { return nv >= 3 && !dots && (size_t)2 * nv * cols <= 65536; }

/* Vectors of the next pass: n vectors in ceil(n / MAX_NV) passes of equal size (+-1), larger
 * first, like the reference's VECTOR_PASSES (engine/src/kern_quant.c:258-274). */
int pass_nv(int left) {
    const int np = (left + MAX_NV - 1) / MAX_NV;
    return (left + np - 1) / np;
}

/* Waves per workgroup of every pass of an n-vector row-per-lane launch: 16 only when every
 * pass runs the matrix-core kernel on enough row groups, so the partial argmax keys of all
 * passes have one layout ([vector][workgroups]). */
int mv_wpg(const SegTable &tab, int n, int cols, bool dots) {
    if (tab.total_waves < MVX_BIG_WAVES) return 4;
    for (int v = 0; v < n;) {
        const int nv = pass_nv(n - v);
        if (!mvx_used(nv, cols, dots)) return 4;
        v += nv;
    }
    return 16;
}

/* The drafts copy of a head launch (q4k_head_k's dcopy): src[0..n) -> dst, by workgroup 0. */
struct HeadCopy {
    const int32_t *src;
    int32_t *dst;
    int n;
};

template <int NV, int NSB, int WPG>
void launch_head(hipStream_t st, unsigned blocks, const Seg &s, int n, int v0, const int8_t *q,
                 const float *d, const float *fs, unsigned long long *am, const HeadCopy &hc) {
    if (n == NV && v0 == 0)
        q4k_head_k<NV, NSB, WPG, true><<<blocks, 64 * WPG, 0, st>>>(
            (const uint8_t *)s.W, q, d, fs, am, s.rows, n, v0, s.Y, hc.src, hc.dst, hc.n);
    else
        q4k_head_k<NV, NSB, WPG, false><<<blocks, 64 * WPG, 0, st>>>(
            (const uint8_t *)s.W, q, d, fs, am, s.rows, n, v0, s.Y, hc.src, hc.dst, hc.n);
}

/* q4k_head_k for one matrix with argmax keys at 1, 2, 4 or 8 superblocks per row; false when
 * the shape is not one of those (q4k_mvx_k then, same results). 8 vectors at 8 superblocks in
 * 16-wave workgroups would need more than the 128 registers a wave may hold there (the
 * compiler spills), so that shape takes q4k_mvx_k too. */
template <int NV>
bool try_head(hipStream_t st, const SegTable &tab, int cols, int n, int v0, const int8_t *q,
              const float *d, const float *fs, unsigned long long *am, int wpg, const HeadCopy &hc) {
    if (tab.count != 1 || tab.s[0].ystride != tab.s[0].rows) return false;
    const unsigned blocks = (unsigned)((tab.total_waves + wpg - 1) / wpg);
    const Seg &s = tab.s[0];
#define NMX_HEAD(NSB)                                                                             do {                                                                                              if (wpg == 16) launch_head<NV, NSB, 16>(st, blocks, s, n, v0, q, d, fs, am, hc);              else launch_head<NV, NSB, 4>(st, blocks, s, n, v0, q, d, fs, am, hc);                     } while (0)
    switch (cols) {
    case 256: NMX_HEAD(1); return true;
    case 512: NMX_HEAD(2); return true;
    case 1024: NMX_HEAD(4); return true;
    case 2048:
        if constexpr (NV < 8) {
            NMX_HEAD(8);
            return true;
        } else {
            if (wpg == 16) return false; /* q4k_mvx_k */
            launch_head<NV, 8, 4>(st, blocks, s, n, v0, q, d, fs, am, hc);
            return true;
        }
    default: return false;
    }
#undef NMX_HEAD
}

/* Returns true when q4k_head_k ran the pass (and with it the drafts copy of hc). */
template <int NV>
bool launch_nv(hipStream_t st, const SegTable &tab, int cols, int n, int v0, const int8_t *q,
               const float *d, const float *fs, int32_t *dots, unsigned long long *am, int wpg,
               const HeadCopy &hc) {
    const unsigned blocks = (unsigned)((tab.total_waves + wpg - 1) / wpg);
    /* 3 or more vectors: the block dots on the matrix cores (bit-identical results; measured at
     * 248320 x 1024, 5 vectors: 30 us against 34-38 us), while its activation table fits in
     * the default 64 KB of LDS */
    if constexpr (NV >= 3) {
        const size_t xbytes = (size_t)2 * NV * cols;
        if (mvx_used(NV, cols, dots != nullptr)) {
            if (am && try_head<NV>(st, tab, cols, n, v0, q, d, fs, am, wpg, hc)) return true;
            if (wpg == 16) {
                if (am) q4k_mvx_k<NV, true, 16><<<blocks, 1024, xbytes, st>>>(tab, cols, n, v0, q, d, fs, am);
                else q4k_mvx_k<NV, false, 16><<<blocks, 1024, xbytes, st>>>(tab, cols, n, v0, q, d, fs, am);
            } else {
                if (am) q4k_mvx_k<NV, true, 4><<<blocks, 256, xbytes, st>>>(tab, cols, n, v0, q, d, fs, am);
                else q4k_mvx_k<NV, false, 4><<<blocks, 256, xbytes, st>>>(tab, cols, n, v0, q, d, fs, am);
            }
            return false;
        }
    }
    if (am) q4k_mv_k<NV, false, true><<<blocks, 256, 0, st>>>(tab, cols, n, v0, q, d, fs, dots, am);
    else if (dots) q4k_mv_k<NV, true, false><<<blocks, 256, 0, st>>>(tab, cols, n, v0, q, d, fs, dots, am);
    else q4k_mv_k<NV, false, false><<<blocks, 256, 0, st>>>(tab, cols, n, v0, q, d, fs, dots, am);
    return false;
}

/* Rows below which the K-split kernel is used (few waves in the row-per-lane kernel). */
constexpr int KSPLIT_MAX_ROWS = 32768;

int launch_ksplit(nmx_ctx *ctx, const SegTable &tab, int total_rows_groups, int cols, int n,
                  const int8_t *q, const float *d, const float *fs, int32_t *dots) {
    const int nsb = cols >> 8;
    const int sbw = nsb <= 8 ? 1 : 2;
    const int KS = (nsb + sbw - 1) / sbw;
    if (KS > 16) return nmx_fail(ctx, "q4k K-split: cols=%d too large", cols);
    dim3 grid((unsigned)total_rows_groups, (unsigned)n);
    dim3 block((unsigned)(64 * KS));
    if (sbw == 1) {
        if (dots) q4k_mv_ks_k<1, true><<<grid, block, 0, ctx->stream>>>(tab, cols, n, KS, q, d, fs, dots);
        else q4k_mv_ks_k<1, false><<<grid, block, 0, ctx->stream>>>(tab, cols, n, KS, q, d, fs, dots);
    } else {
        if (dots) q4k_mv_ks_k<2, true><<<grid, block, 0, ctx->stream>>>(tab, cols, n, KS, q, d, fs, dots);
        else q4k_mv_ks_k<2, false><<<grid, block, 0, ctx->stream>>>(tab, cols, n, KS, q, d, fs, dots);
    }
    NMX_LAUNCHED(ctx, "q4k_mv_ks");
    return 0;
}

/* More than 8 vectors (prefill chunks): the MFMA kernel. Its segment table counts 16-row
 * groups. A wave takes all vector tiles when there are enough row groups to fill the chip,
 * else one tile (four times the waves, the scale decode repeated per tile). */
int launch_mm(nmx_ctx *ctx, const SegTable &tab, int cols, int n, const int8_t *q,
              const float *d, const float *fs) {
    SegTable t16 = tab;
    int groups = 0;
    for (int s = 0; s < tab.count; s++) {
        t16.s[s].wave0 = groups;
        groups += (tab.s[s].rows + 15) / 16;
    }
    t16.total_waves = groups;
    const int vtiles = (n + 15) / 16;
    if (groups < 512) { /* few rows: one vector tile per single-wave workgroup */
        const dim3 grid((unsigned)groups, (unsigned)vtiles);
        q4k_mm_k<1, 1, 2><<<grid, 64, 0, ctx->stream>>>(t16, cols, n, q, d, fs);
    } else {
        const dim3 grid((unsigned)((groups + 3) / 4));
        switch (vtiles) {
        case 4: q4k_mm_k<4, 4, 1><<<grid, 256, 0, ctx->stream>>>(t16, cols, n, q, d, fs); break;
        case 3: q4k_mm_k<3, 4, 1><<<grid, 256, 0, ctx->stream>>>(t16, cols, n, q, d, fs); break;
        case 2: q4k_mm_k<2, 4, 1><<<grid, 256, 0, ctx->stream>>>(t16, cols, n, q, d, fs); break;
        default: q4k_mm_k<1, 4, 1><<<grid, 256, 0, ctx->stream>>>(t16, cols, n, q, d, fs); break;
        }
    }
    NMX_LAUNCHED(ctx, "q4k_mm");
    return 0;
}

/* copied (may be NULL): set to whether the first pass made hc's drafts copy. */
int launch_passes(nmx_ctx *ctx, const SegTable &tab, int cols, int n, const int8_t *q,
                  const float *d, const float *fs, int32_t *dots, unsigned long long *am = nullptr,
                  HeadCopy hc = HeadCopy{nullptr, nullptr, 0}, bool *copied = nullptr) {
    if (copied) *copied = false;
    int total_rows = 0;
    for (int s = 0; s < tab.count; s++) total_rows += tab.s[s].rows;
    if (!am && !dots && n > MAX_NV) return launch_mm(ctx, tab, cols, n, q, d, fs);
    if (!am && !dots && total_rows < KSPLIT_MAX_ROWS) {
        nmx_mt_seg segs[NMX_MAX_SEGS];
        for (int s = 0; s < tab.count; s++)
            segs[s] = nmx_mt_seg{tab.s[s].W, tab.s[s].Y, tab.s[s].rows, tab.s[s].ystride};
        const int rc = nmx_mt_matmul(ctx, tab.count, segs, cols, n, q, d, fs, nullptr, false, nmx_a8{});
        if (rc <= 0) return rc;
    }
    if (!am && total_rows < KSPLIT_MAX_ROWS && cols <= 16 * 2 * 256)
        return launch_ksplit(ctx, tab, tab.total_waves, cols, n, q, d, fs, dots);
    /* every pass performs the same per-vector operations, so the result does not depend on
     * the split (pass_nv) */
    const int wpg = mv_wpg(tab, n, cols, dots != nullptr);
    for (int v = 0; v < n;) {
        const int nv = pass_nv(n - v);
        bool head = false;
        switch (nv) {
        case 8: head = launch_nv<8>(ctx->stream, tab, cols, n, v, q, d, fs, dots, am, wpg, hc); break;
        case 7: head = launch_nv<7>(ctx->stream, tab, cols, n, v, q, d, fs, dots, am, wpg, hc); break;
        case 6: head = launch_nv<6>(ctx->stream, tab, cols, n, v, q, d, fs, dots, am, wpg, hc); break;
        case 5: head = launch_nv<5>(ctx->stream, tab, cols, n, v, q, d, fs, dots, am, wpg, hc); break;
        case 4: head = launch_nv<4>(ctx->stream, tab, cols, n, v, q, d, fs, dots, am, wpg, hc); break;
        case 3: head = launch_nv<3>(ctx->stream, tab, cols, n, v, q, d, fs, dots, am, wpg, hc); break;
        case 2: head = launch_nv<2>(ctx->stream, tab, cols, n, v, q, d, fs, dots, am, wpg, hc); break;
        default: head = launch_nv<1>(ctx->stream, tab, cols, n, v, q, d, fs, dots, am, wpg, hc); break;
        }
        NMX_LAUNCHED(ctx, "q4k_mv");
        if (v == 0 && copied) *copied = head && hc.dst;
        hc.dst = nullptr; /* the drafts are copied by the first pass */
        v += nv;
    }
    return 0;
}

size_t q4k_bytes(int rows, int cols) {
    return (size_t)(rows / 4) * (size_t)(cols / 256) * SB_BYTES;
}

} // namespace

/* The partial argmax keys of nmx_head_accept_noalloc live in this array instead of a
 * caller-provided workspace: one copy per device, at a device address that
 * nmx_head_scratch_init resolves once per device (host code must never pass the array's own
 * name to a kernel: on the host it only stands for the device symbol). Every call of the
 * entry point on a device shares the copy; the keys of a call are all written by its head
 * kernel before head_finish_k reads them, so nothing needs clearing between calls. */
static __device__ __align__(256) unsigned long long scratch[NMX_HEAD_SCRATCH_BYTES / 8];

namespace {
constexpr int SCRATCH_DEVICES = 64;
std::mutex g_scratch_mu;
unsigned long long *g_scratch[SCRATCH_DEVICES]; /* device address of `scratch`, per device */
} // namespace

int nmx_head_scratch_init(nmx_ctx *ctx) {
    if (ctx->device < 0 || ctx->device >= SCRATCH_DEVICES)
        return nmx_fail(ctx, "head scratch: device %d beyond %d", ctx->device, SCRATCH_DEVICES);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch[ctx->device]) return 0;
    int cur = -1;
    NMX_HIP(ctx, hipGetDevice(&cur));
    if (cur != ctx->device) return nmx_fail(ctx, "head scratch: device %d not current", ctx->device);
    void *ptr = nullptr;
    NMX_HIP(ctx, hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    if (!ptr || (uintptr_t)ptr % 256) return nmx_fail(ctx, "head scratch: bad symbol address");
    g_scratch[ctx->device] = (unsigned long long *)ptr;
    return 0;
}

extern "C" {

int nmx_quant_a8(nmx_ctx *ctx, const float *X, int n, int cols, int8_t *q, float *d,
                 float *fsum) {
    if (!ctx) return -1;
    if (!X || !q || !d || !fsum) return nmx_fail(ctx, "nmx_quant_a8: NULL pointer");
    if (n < 1 || n > 4096 || cols < 32 || cols % 32 || cols > (1 << 20))
        return nmx_fail(ctx, "nmx_quant_a8: bad shape n=%d cols=%d", n, cols);
    const size_t xb = (size_t)n * cols * 4, qb = (size_t)n * cols, fb = (size_t)n * (cols / 32) * 4;
    if (nmx_overlap(q, qb, X, xb) || nmx_overlap(d, fb, X, xb) || nmx_overlap(fsum, fb, X, xb) ||
        nmx_overlap(q, qb, d, fb) || nmx_overlap(q, qb, fsum, fb) || nmx_overlap(d, fb, fsum, fb))
        return nmx_fail(ctx, "nmx_quant_a8: aliased buffers");
    const size_t units = (size_t)n * (cols / 32);
    const unsigned blocks = (unsigned)((units + 7) / 8);
    quant_a8_k<<<blocks, 256, 0, ctx->stream>>>(X, n, cols, q, d, fsum);
    NMX_LAUNCHED(ctx, "quant_a8");
    return 0;
}

int nmx_q4k_matmul_multi(nmx_ctx *ctx, int count, const void *const *W, const int *rows,
                         float *const *Y, const int *y_stride, int cols, int n,
                         const int8_t *q, const float *d, const float *fsum) {
    if (!ctx) return -1;
    if (count < 1 || count > NMX_MAX_SEGS || !W || !rows || !Y || !y_stride)
        return nmx_fail(ctx, "nmx_q4k_matmul_multi: bad segment list (count=%d)", count);
    if (!q || !d || !fsum) return nmx_fail(ctx, "nmx_q4k_matmul: NULL activation pointer");
    if (cols <= 0 || cols % 256 || cols > 65536 || n < 1 || n > 64)
        return nmx_fail(ctx, "nmx_q4k_matmul: bad shape cols=%d n=%d", cols, n);
    const size_t qb = (size_t)n * cols, fb = (size_t)n * (cols / 32) * 4;
    SegTable tab = {};
    tab.count = count;
    int waves = 0;
    for (int s = 0; s < count; s++) {
        if (!W[s] || !Y[s]) return nmx_fail(ctx, "nmx_q4k_matmul: NULL matrix %d", s);
        if (rows[s] <= 0 || rows[s] % 4 || rows[s] > (1 << 22) || y_stride[s] < rows[s])
            return nmx_fail(ctx, "nmx_q4k_matmul: bad rows=%d y_stride=%d (matrix %d)", rows[s],
                            y_stride[s], s);
        const size_t wb = q4k_bytes(rows[s], cols), yb = ((size_t)(n - 1) * y_stride[s] + rows[s]) * 4;
        if (nmx_overlap(Y[s], yb, W[s], wb) || nmx_overlap(Y[s], yb, q, qb) ||
            nmx_overlap(Y[s], yb, d, fb) || nmx_overlap(Y[s], yb, fsum, fb))
            return nmx_fail(ctx, "nmx_q4k_matmul: output %d aliases an input", s);
        tab.s[s] = Seg{(const uint8_t *)W[s], Y[s], rows[s], y_stride[s], waves, 0};
        waves += (rows[s] + 63) / 64;
    }
    tab.total_waves = waves;
    return launch_passes(ctx, tab, cols, n, q, d, fsum, nullptr);
}

int nmx_q4k_matmul(nmx_ctx *ctx, const void *W, int rows, int cols, int n, const int8_t *q,
                   const float *d, const float *fsum, float *Y, int y_stride, int32_t *dots) {
    if (!ctx) return -1;
    if (!W || !Y || !q || !d || !fsum) return nmx_fail(ctx, "nmx_q4k_matmul: NULL pointer");
    if (rows <= 0 || rows % 4 || rows > (1 << 22) || cols <= 0 || cols % 256 || cols > 65536 ||
        n < 1 || n > 64 || y_stride < rows)
        return nmx_fail(ctx, "nmx_q4k_matmul: bad shape rows=%d cols=%d n=%d y_stride=%d", rows,
                        cols, n, y_stride);
    const size_t wb = q4k_bytes(rows, cols), qb = (size_t)n * cols, fb = (size_t)n * (cols / 32) * 4;
    const size_t yb = ((size_t)(n - 1) * y_stride + rows) * 4;
    if (nmx_overlap(Y, yb, W, wb) || nmx_overlap(Y, yb, q, qb) || nmx_overlap(Y, yb, d, fb) ||
        nmx_overlap(Y, yb, fsum, fb))
        return nmx_fail(ctx, "nmx_q4k_matmul: output aliases an input");
    if (dots) {
        const size_t db = (size_t)n * rows * (cols / 32) * 4;
        if (nmx_overlap(dots, db, Y, yb) || nmx_overlap(dots, db, W, wb) ||
            nmx_overlap(dots, db, q, qb) || nmx_overlap(dots, db, d, fb) ||
            nmx_overlap(dots, db, fsum, fb))
            return nmx_fail(ctx, "nmx_q4k_matmul: dots aliases a buffer");
    }
    SegTable tab = {};
    tab.count = 1;
    tab.s[0] = Seg{(const uint8_t *)W, Y, rows, y_stride, 0, 0};
    tab.total_waves = (rows + 63) / 64;
    return launch_passes(ctx, tab, cols, n, q, d, fsum, dots);
}

size_t nmx_head_work_bytes(int rows, int n) {
    if (rows <= 0 || n <= 0) return 0;
    const size_t blocks = (size_t)((rows + 63) / 64 + 3) / 4;
    return (size_t)n * blocks * 8; /* [n][workgroups] partial argmax keys */
}

int nmx_head_accept(nmx_ctx *ctx, const void *W, int rows, int cols, int n, const int8_t *q,
                    const float *d, const float *fsum, float *logits, const int32_t *drafts,
                    void *work, int32_t *out) {
    return nmx_head_accept_to(ctx, W, rows, cols, n, q, d, fsum, logits, drafts, work, out, nullptr);
}

int nmx_head_accept_noalloc(nmx_ctx *ctx, const void *W, int rows, int cols, int n,
                            const int8_t *q, const float *d, const float *fsum, float *logits,
                            const int32_t *drafts, int32_t *out) {
    if (!ctx) return -1;
    const size_t kb = nmx_head_work_bytes(rows, n);
    if (kb > NMX_HEAD_SCRATCH_BYTES)
        return nmx_fail(ctx, "nmx_head_accept_noalloc: rows=%d n=%d need %zu scratch bytes, above "
                        "the %d of the static array (use nmx_head_accept with a workspace)",
                        rows, n, kb, NMX_HEAD_SCRATCH_BYTES);
    unsigned long long *keys = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        if (ctx->device >= 0 && ctx->device < SCRATCH_DEVICES) keys = g_scratch[ctx->device];
    }
    if (!keys) return nmx_fail(ctx, "nmx_head_accept_noalloc: head scratch not set up");
    return nmx_head_accept_to(ctx, W, rows, cols, n, q, d, fsum, logits, drafts, keys, out,
                              nullptr);
}

static int head_accept(nmx_ctx *ctx, const void *W, int rows, int cols, int n, const int8_t *q,
                       const float *d, const float *fsum, float *logits, const int32_t *drafts,
                       void *work, int32_t *out, int32_t *tok_dst, FinishCommit fc) {
    if (!ctx) return -1;
    if (!W || !q || !d || !fsum || !work || !out || (n > 1 && !drafts))
        return nmx_fail(ctx, "nmx_head_accept: NULL pointer");
    if (rows <= 0 || rows % 4 || rows > (1 << 22) || cols <= 0 || cols % 256 || cols > 65536 ||
        n < 1 || n > 64)
        return nmx_fail(ctx, "nmx_head_accept: bad shape rows=%d cols=%d n=%d", rows, cols, n);
    const size_t wb = q4k_bytes(rows, cols), qb = (size_t)n * cols, fb = (size_t)n * (cols / 32) * 4;
    const size_t lb = (size_t)n * rows * 4, kb = nmx_head_work_bytes(rows, n);
    const size_t ob = (size_t)(2 + n) * 4;
    if (logits && (nmx_overlap(logits, lb, W, wb) || nmx_overlap(logits, lb, q, qb) ||
                   nmx_overlap(logits, lb, d, fb) || nmx_overlap(logits, lb, fsum, fb) ||
                   nmx_overlap(logits, lb, work, kb) || nmx_overlap(logits, lb, out, ob)))
        return nmx_fail(ctx, "nmx_head_accept: logits alias another buffer");
    if (nmx_overlap(work, kb, W, wb) || nmx_overlap(work, kb, q, qb) || nmx_overlap(work, kb, out, ob) ||
        nmx_overlap(out, ob, W, wb) || nmx_overlap(out, ob, q, qb))
        return nmx_fail(ctx, "nmx_head_accept: work/out alias another buffer");
    SegTable tab = {};
    tab.count = 1;
    tab.s[0] = Seg{(const uint8_t *)W, logits, rows, rows, 0, 0};
    tab.total_waves = (rows + 63) / 64;
    if ((uintptr_t)work % 8) return nmx_fail(ctx, "nmx_head_accept: work not 8-byte aligned");
    const int wpg = mv_wpg(tab, n, cols, false);
    const int blocks = (tab.total_waves + wpg - 1) / wpg; /* launch_passes' workgroups */
    unsigned long long *keys = (unsigned long long *)work;
    if (launch_passes(ctx, tab, cols, n, q, d, fsum, nullptr, keys)) return -1;
    head_finish_k<<<1, 1024, 0, ctx->stream>>>(keys, blocks, n, drafts, out, tok_dst, fc);
    NMX_LAUNCHED(ctx, "head_finish");
    return 0;
}

int nmx_head_nkeys(int rows, int cols, int n) {
    if (rows <= 0 || cols <= 0 || n <= 0) return 0;
    SegTable tab = {};
    tab.count = 1;
    tab.s[0] = Seg{nullptr, nullptr, rows, rows, 0, 0};
    tab.total_waves = (rows + 63) / 64;
    const int wpg = mv_wpg(tab, n, cols, false);
    return (tab.total_waves + wpg - 1) / wpg;
}

int nmx_head_keys(nmx_ctx *ctx, const void *W, int rows, int cols, int n, const int8_t *q,
                  const float *d, const float *fsum, const int32_t *drafts, void *work,
                  int32_t *drafts_copy) {
    if (!ctx) return -1;
    if (!W || !q || !d || !fsum || !work || (n > 1 && (!drafts || !drafts_copy)))
        return nmx_fail(ctx, "nmx_head_keys: NULL pointer");
    if (rows <= 0 || rows % 4 || rows > (1 << 22) || cols <= 0 || cols % 256 || cols > 65536 ||
        n < 1 || n > 16)
        return nmx_fail(ctx, "nmx_head_keys: bad shape rows=%d cols=%d n=%d", rows, cols, n);
    if ((uintptr_t)work % 8) return nmx_fail(ctx, "nmx_head_keys: work not 8-byte aligned");
    const size_t wb = q4k_bytes(rows, cols), kb = nmx_head_work_bytes(rows, n);
    if (nmx_overlap(work, kb, W, wb) || nmx_overlap(work, kb, q, (size_t)n * cols) ||
        (n > 1 && (nmx_overlap(drafts_copy, (size_t)(n - 1) * 4, work, kb) ||
                   nmx_overlap(drafts_copy, (size_t)(n - 1) * 4, drafts, (size_t)(n - 1) * 4))))
        return nmx_fail(ctx, "nmx_head_keys: work or drafts_copy aliases another buffer");
    SegTable tab = {};
    tab.count = 1;
    tab.s[0] = Seg{(const uint8_t *)W, nullptr, rows, rows, 0, 0};
    tab.total_waves = (rows + 63) / 64;
    bool copied = false;
    const HeadCopy hc{drafts, n > 1 ? drafts_copy : nullptr, n - 1};
    if (launch_passes(ctx, tab, cols, n, q, d, fsum, nullptr, (unsigned long long *)work, hc,
                      &copied))
        return -1;
    if (n > 1 && !copied) { /* the first pass ran another kernel (1-2 vectors, other widths) */
        copy_i32_k<<<1, 64, 0, ctx->stream>>>(drafts, drafts_copy, n - 1);
        NMX_LAUNCHED(ctx, "copy_i32");
    }
    return 0;
}

int nmx_head_accept_to(nmx_ctx *ctx, const void *W, int rows, int cols, int n, const int8_t *q,
                       const float *d, const float *fsum, float *logits, const int32_t *drafts,
                       void *work, int32_t *out, int32_t *tok_dst) {
    return head_accept(ctx, W, rows, cols, n, q, d, fsum, logits, drafts, work, out, tok_dst,
                       FinishCommit{nullptr, nullptr, nullptr, 0, nullptr});
}

int nmx_head_row_accept_to(nmx_ctx *ctx, const void *W, int rows, int cols, const float *x,
                           int x_stride, const float *add, int add_stride, const float *w,
                           float eps, const int32_t *idx, int off, int nrows, float *y,
                           void *work, int32_t *out, int32_t *tok_dst, nmx_a8 a8_tmp,
                           int32_t *advance) {
    if (!ctx) return -1;
    if (!W || !x || !w || !idx || !work || !out || nrows < 1 || x_stride < cols ||
        (add && add_stride < cols))
        return nmx_fail(ctx, "nmx_head_row_accept_to: bad arguments");
    auto al = [](const void *p) { return ((uintptr_t)p & 15) == 0; };
    const bool fused = cols > 0 && cols % 256 == 0 && cols <= MVR_MAX_COLS && rows > 0 &&
                       rows % 4 == 0 && rows <= (1 << 22) && al(x) && al(w) && x_stride % 4 == 0 &&
                       (!add || (al(add) && add_stride % 4 == 0)) && (!y || al(y)) &&
                       (uintptr_t)work % 8 == 0;
    if (!fused) { /* the norm, then the head on its A8 */
        if (!a8_tmp.q || !a8_tmp.d || !a8_tmp.fs)
            return nmx_fail(ctx, "nmx_head_row_accept_to: shape needs a8_tmp");
        if (nmx_rmsnorm_row(ctx, x, x_stride, add, add_stride, w, cols, eps, idx, off, nrows, y,
                            a8_tmp))
            return -1;
        if (nmx_head_accept_to(ctx, W, rows, cols, 1, a8_tmp.q, a8_tmp.d, a8_tmp.fs, nullptr,
                               nullptr, work, out, tok_dst))
            return -1;
        return advance ? nmx_ctl_advance(ctx, advance) : 0;
    }
    const int blocks = nmx_head_row_nkeys(rows);
    unsigned long long *keys = (unsigned long long *)work;
    q4k_mvr_k<<<blocks, cols / 4, 0, ctx->stream>>>(idx, x, add, w, (const uint8_t *)W, off,
                                                     nrows, x_stride, add_stride, cols, rows, eps,
                                                     y, keys);
    NMX_LAUNCHED(ctx, "q4k_mvr");
    head_finish_k<<<1, 1024, 0, ctx->stream>>>(keys, blocks, 1, nullptr, out, tok_dst,
                                                FinishCommit{nullptr, nullptr, nullptr, 0, advance});
    NMX_LAUNCHED(ctx, "head_finish");
    return 0;
}

int nmx_head_row_nkeys(int rows) { return rows > 0 ? (rows + 63) / 64 : 0; }

int nmx_head_row_keys(nmx_ctx *ctx, const void *W, int rows, int cols, const float *x,
                      int x_stride, const float *add, int add_stride, const float *w, float eps,
                      const int32_t *idx, int off, int nrows, float *y, void *keys) {
    if (!ctx) return -1;
    auto al = [](const void *p) { return ((uintptr_t)p & 15) == 0; };
    if (!W || !x || !w || !idx || !keys || nrows < 1 || x_stride < cols ||
        (add && add_stride < cols))
        return nmx_fail(ctx, "nmx_head_row_keys: bad arguments");
    if (cols <= 0 || cols % 256 || cols > MVR_MAX_COLS || rows <= 0 || rows % 4 ||
        rows > (1 << 22) || !al(x) || !al(w) || x_stride % 4 ||
        (add && (!al(add) || add_stride % 4)) || (y && !al(y)) ||
        (uintptr_t)keys % 8)
        return nmx_fail(ctx, "nmx_head_row_keys: shape outside the fused kernel (cols %d)", cols);
    q4k_mvr_k<<<nmx_head_row_nkeys(rows), cols / 4, 0, ctx->stream>>>(
        idx, x, add, w, (const uint8_t *)W, off, nrows, x_stride, add_stride, cols, rows, eps, y,
        (unsigned long long *)keys);
    NMX_LAUNCHED(ctx, "q4k_mvr");
    return 0;
}

int nmx_head_step(nmx_ctx *ctx, const void *W, int rows, int cols, const int8_t *q,
                  const float *d, const float *fsum, void *work, int32_t *out, int32_t *vt,
                  int32_t *ctl, int32_t *mailbox, int nvt) {
    if (!ctx) return -1;
    if (!vt || !ctl || (mailbox && (nvt < 2 || nvt > 1024)))
        return nmx_fail(ctx, "nmx_head_step: bad arguments");
    return head_accept(ctx, W, rows, cols, 1, q, d, fsum, nullptr, nullptr, work, out, vt,
                       FinishCommit{vt, ctl, mailbox, mailbox ? nvt : 0, ctl});
}

int nmx_head_accept_commit(nmx_ctx *ctx, const void *W, int rows, int cols, int n,
                           const int8_t *q, const float *d, const float *fsum,
                           const int32_t *drafts, void *work, int32_t *out, int32_t *vt,
                           int32_t *ctl, int32_t *mailbox, int nvt) {
    if (!ctx) return -1;
    if (!vt || !ctl || (mailbox && (nvt < n + 1 || nvt > 1024)))
        return nmx_fail(ctx, "nmx_head_accept_commit: bad arguments");
    return head_accept(ctx, W, rows, cols, n, q, d, fsum, nullptr, drafts, work, out, nullptr,
                       FinishCommit{vt, ctl, mailbox, mailbox ? nvt : 0, nullptr});
}

} /* extern "C" */
