/* Q4K_G32 x A8 products of the verify step's small projections (a few thousand rows, k + 1
 * activation rows) for gfx950, with an optional fused RMSNorm + A8 prologue and an optional
 * fused SwiGLU + A8 epilogue.
 *
 * Exactness contract (the reference's kern_q4k, engine/src/kern_quant.c:148-245): for every
 * output row r and vector v the fp32 accumulator runs over the 32-column blocks in column
 * order, acc = fma((float)dot, (D*s)*d_v, acc); acc = fma(-(M*m), fsum_v, acc), with dot the
 * exact int32 sum of 32 nibble x int8 products.
 *
 * One workgroup owns R output rows and every vector of the pass, so each weight byte is
 * fetched once per launch. Three phases, separated by barriers:
 *   0. the thread's weight unit (one row x half a 256-column superblock: the 64-byte scale
 *      line and the row's four 16-byte code chunks) is loaded first; meanwhile the pass's A8
 *      activations are staged into LDS (copied, or computed by the RMSNorm prologue);
 *   1. every unit decodes its sub-scales and computes its 4 blocks x NV exact int32 dots with
 *      v_dot4_i32_i8, storing one record ((float)dot, (D*s)*d_v, -(M*m), fsum_v) per (block,
 *      vector, row) to LDS laid out [vector][row][block] (a chain's records contiguous, so its
 *      reads take immediate offsets; the 64-row SwiGLU launch stores ((float)dot, (D*s)*d_v)
 *      pairs and -(M*m) separately, laid out the same way, to fit in 160 KB);
 *   2. one lane per (row, vector) runs the fp32 chain over the blocks in column order, two
 *      FMAs per block from one 16-byte LDS read (three reads for SwiGLU), then stores the row
 *      (or, for SwiGLU, the workgroup combines its gate and up halves, silu(g) * u, and
 *      quantizes the result to A8).
 * The RMSNorm prologue restates engine/src/forward_ops.c:168-200 (sumsq as 4 interleaved
 * partial sums + tail, r = 1 / sqrtf(ss / cols + eps), y = (x * r) * w) and the A8 of
 * engine/src/kern_act.c:14-42, so the activations equal those of the separate kernels. */
#include "nmx_internal.h"
#include "nmx_math.h"
#include "nmx_a8.h"

namespace {

constexpr int MT_MAX_NV = 8;
constexpr int MT_MAX_THREADS = 512; /* the SwiGLU launch (64 rows; the dots' VGPR buffers) */
constexpr int MT_LDS = 159 * 1024; /* dynamic LDS per workgroup (gfx950: 160 KB) */
constexpr int MT_NORM_CPT = 8; /* columns per thread in the norm prologue */
constexpr int MT_NORM_THREADS = 512; /* the prologue keeps NV x MT_NORM_CPT values in VGPRs */
constexpr int MT_REC_THREADS = 1024; /* launches of 1- or 2-block units */
constexpr int MT_REC4_THREADS = 256; /* record launches of 4-block units: room for VGPR buffers */

struct MtTab {
    nmx_mt_seg s[NMX_MAX_SEGS];
    int g0[NMX_MAX_SEGS]; /* first workgroup of each segment */
    int count;
};

/* The PAIR prologue's embedding half: the Q4K embedding E and its norm weight (the other half's
 * weight and eps come in nmx_norm_in); keys (one row): its token is the argmax of the nkeys
 * partial keys instead of tok[v0], and workgroup 0 writes it to tok[v0]. */
struct MtPair {
    const uint8_t *E;
    const float *w0;
    const unsigned long long *keys;
    int nkeys;
};

__device__ __forceinline__ float half_bits(uint32_t h) {
    const unsigned short b = (unsigned short)h;
    _Float16 f;
    __builtin_memcpy(&f, &b, 2);
    return (float)f;
}

/* The four 6-bit values s[4k + i], k = 4 half .. 4 half + 3, of row i from a packed array
 * (engine/FORMAT.md: 16 B of low nibbles, then 8 B of high bit pairs): L0..L3 the low-nibble
 * dwords, H0 / H1 the high-pair dwords, sh8 = 8 i. */
__device__ __forceinline__ void decode6_half(uint32_t L0, uint32_t L1, uint32_t L2, uint32_t L3,
                                             uint32_t H0, uint32_t H1, int sh8, int half,
                                             int out[4]) {
    const uint32_t hs = 4u * half; /* nibble of the low bits, and the high-pair shift base */
    const uint32_t b[4] = {(L0 >> sh8) & 0xffu, (L1 >> sh8) & 0xffu, (L2 >> sh8) & 0xffu,
                           (L3 >> sh8) & 0xffu};
    const uint32_t h0 = (H0 >> sh8) & 0xffu, h1 = (H1 >> sh8) & 0xffu;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint32_t h = (k & 1) ? h1 : h0;
        out[k] = (int)(((b[k] >> hs) & 15u) | (((h >> (hs + 2 * (k >> 1))) & 3u) << 4));
    }
}

/* The 32 values of 32-column block b of Q4K row `row` (cols columns), as the embedding
 * kernels compute them (dequantised (D s) q - M m, engine/src/kern_act.c:47-88): the
 * superblock's 64-byte scale line and the row's 16 code bytes in five 16-byte loads. */
__device__ __forceinline__ void q4k_block32(const uint8_t *__restrict__ E, int row, int cols, int b,
                                            float out[32]) {
    const int sb = b >> 3, k = b & 7, i = row & 3;
    const uint4 *p = (const uint4 *)(E + ((size_t)(row >> 2) * (cols >> 8) + sb) * 576);
    const uint4 a0 = p[0], a1 = p[1], a2 = p[2], a3 = p[3], cw = p[4 + 4 * k + i];
    int s6[4], m6[4];
    decode6_half(a1.x, a1.y, a1.z, a1.w, a2.x, a2.y, 8 * i, k >> 2, s6);
    decode6_half(a2.z, a2.w, a3.x, a3.y, a3.z, a3.w, 8 * i, k >> 2, m6);
    const float D = half_bits(((i & 2) ? a0.y : a0.x) >> (16 * (i & 1)));
    const float M = half_bits(((i & 2) ? a0.w : a0.z) >> (16 * (i & 1)));
    const float dd = D * (float)s6[k & 3], mm = M * (float)m6[k & 3];
    const uint32_t w[4] = {cw.x, cw.y, cw.z, cw.w};
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const uint32_t byte = (w[j >> 2] >> (8 * (j & 3))) & 0xffu;
        out[j] = dd * (float)(byte & 15u) - mm;
        out[16 + j] = dd * (float)(byte >> 4) - mm;
    }
}

/* Byte offset of block b's NV x 32 activation codes in LDS: 16 bytes of padding per
 * superblock, so the units of different superblocks read different banks. */
__host__ __device__ constexpr int aq_off(int b, int nv) { return b * nv * 32 + (b >> 3) * 16; }

__host__ __device__ constexpr int cm_stride4(int cols) { return (((cols >> 2) + 3) & ~3) + 4; }

struct MtLayout {
    int aq, ad, afs, work, res, total;
};

__host__ __device__ inline MtLayout mt_layout(int cols, int nv, int R, bool norm, bool swiglu,
                                              bool pair = false) {
    const int nb = cols >> 5;
    MtLayout L{};
    L.aq = 0;
    L.ad = (aq_off(nb, nv) + 15) & ~15;
    L.afs = L.ad + nb * nv * 4;
    L.work = (L.afs + nb * nv * 4 + 15) & ~15;
    /* chain records: (dot, (D*s)*d, -(M*m), fsum) float4 [nv][R][nb | 1] (each chain's blocks
     * contiguous, an odd stride between chains); the SwiGLU launch (64 rows) keeps ((float)dot,
     * (D*s)*d) float2 [nv][R][nb | 1] and -(M*m) [R][nb | 1] to fit */
    int work = swiglu ? (nv * R * 8 + R * 4) * (nb | 1) : nv * R * (nb | 1) * 16;
    /* the norm prologue: chain-major squares, then the summed rows [nv][cols] (PAIR: 2 nv rows
     * of cols / 2) */
    const int nr = pair ? 2 * nv : nv, rc = pair ? cols / 2 : cols;
    const int nwork = nr * (4 * cm_stride4(rc) + 4) * 4 + nr * rc * 4;
    if (norm && nwork > work) work = nwork;
    L.res = L.work + work;
    L.total = L.res + (swiglu ? nv * R * 4 : 0);
    return L;
}

/* The leading arguments are the ones the first memory requests need, in 14 SGPRs: the
 * library is built with kernel-argument preloading, so they arrive in SGPRs with the wave
 * instead of through a load from the argument segment (about 0.2 us on this part). in0 / in1
 * are the A8 codes and scales (q, d), or with NORM the norm input rows x and add; aux is the
 * A8 fsum pointer, or with NORM the row strides of x (low 32 bits) and add (high); W0 / rows0
 * the first segment's weights and rows; T the block size (blockDim lives in the argument
 * segment).
 * PAIR (with NORM): the MTP head's fc input (engine/src/mtp.c:60-75), activation row v =
 * [rmsnorm(embedding row tok[v0 + v] of pr.E, pr.w0) | rmsnorm(row v0 + v of h, nm.w)], each
 * half cols / 2 columns (a multiple of 256, so no A8 block straddles them); in0 = h, in1 =
 * tok, aux = h's row stride; T >= cols / 8 (one float4 of each half per thread). */
template <int NV, bool NORM, bool SWI, int BPU, bool PAIR = false>
__global__ __launch_bounds__(BPU < 4 ? 1024 : NORM ? MT_NORM_THREADS : SWI ? MT_MAX_THREADS : MT_REC4_THREADS) void q4k_mt_k(
    const void *__restrict__ in0, const void *__restrict__ in1, uint64_t aux,
    const uint8_t *__restrict__ W0, int cols, int n, int v0, int R, int T, int rows0,
    MtTab tab, nmx_norm_in nm, int8_t *__restrict__ oq, float *__restrict__ od,
    float *__restrict__ ofs, MtPair pr) {
    static_assert(!PAIR || (NORM && !SWI), "PAIR is a norm prologue of a plain matmul");
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ float red[(PAIR ? 10 : 5) * MT_MAX_NV];
    __shared__ __align__(16) int zl[8]; /* 32 zero bytes: the matrix-core dots' off-diagonal rows */
    const int tid = threadIdx.x;
    if (tid < 8) zl[tid] = 0;
    const int8_t *q = (const int8_t *)in0;
    const float *d = (const float *)in1;
    /* fs (an integer argument) as a pointer to global memory: its loads are then global loads,
     * which a wait can count (a wait for a generic load's result waits for every load in
     * flight, the weights too) */
    const __attribute__((address_space(1))) float *fs =
        (const __attribute__((address_space(1))) float *)(uintptr_t)aux;
    const float *nx = (const float *)in0, *nadd = PAIR ? nullptr : (const float *)in1;
    const int xs = (int)(uint32_t)aux, as = (int)(uint32_t)(aux >> 32);
    const int nb = cols >> 5, nsb = cols >> 8;
    /* norm prologue columns per thread: wide workgroups of 1- or 2-block units need 2 */
    constexpr int CPT = NORM && BPU < 4 ? 2 : MT_NORM_CPT;
    const MtLayout L = mt_layout(cols, NV, R, NORM, SWI);
    int8_t *aq = (int8_t *)(smem + L.aq);
    float *ad = (float *)(smem + L.ad), *afs = (float *)(smem + L.afs);
    constexpr bool REC = !SWI; /* one float4 record per (block, vector, row) */
    float4 *rec = (float4 *)(smem + L.work);  /* [NV][R][nb | 1] (dot, (D*s)*d, -(M*m), fsum) */
    float2 *lp = (float2 *)(smem + L.work);  /* [NV][R][nb | 1] ((float)dot, (D*s)*d) */
    float *lof = (float *)(lp + NV * R * (nb | 1)); /* [R][nb | 1] -(M*m) */

    /* ---- segment and rows of this workgroup (segment 0 from the preloaded arguments: its
     * workgroups are the first ceil(rows0 / R); SwiGLU launches are one segment pair) ---- */
    const int g = blockIdx.x;
    int si = 0;
    if (!SWI && g >= (rows0 + R - 1) / R) { /* uniform */
#pragma unroll
        for (int t = 1; t < NMX_MAX_SEGS; t++)
            if (t < tab.count && g >= tab.g0[t]) si = t;
    }
    const int lg = si == 0 ? g : g - tab.g0[si];

    /* ---- phase 0a: first round of activation / norm-input loads, issued before the weight
     * loads so that waiting for them does not wait for the weights ---- */
    const int nq = nb * NV * 2, ns = nb * NV; /* 16-byte code halves; (block, vector) pairs */
    /* staged per thread and round: NQB code halves, NDB (d, fsum) pairs. One-block units have
     * T >= 8 R nsb threads, so a round needs at most nq / T <= 2 NV / R halves and NV / R pairs
     * per thread: one round for every pass of up to 8 vectors at R >= 4 rows (a second
     * round's loads would be issued only after the first round's have landed) */
    constexpr int NQB = BPU == 1 ? 4 : 8, NDB = BPU == 1 ? 2 : 4;
    int4 buf[NQB];
    float bd[NDB], bf[NDB];
    if constexpr (!NORM) {
#pragma unroll
        for (int u = 0; u < NQB; u++) {
            const int e = u * T + tid;
            buf[u] = make_int4(0, 0, 0, 0);
            if (e < nq) {
                const int b = e / (2 * NV), rem = e - b * 2 * NV;
                buf[u] = *(const int4 *)(q + ((size_t)b * n + v0 + (rem >> 1)) * 32 + 16 * (rem & 1));
            }
        }
#pragma unroll
        for (int u = 0; u < NDB; u++) {
            const int e = u * T + tid;
            const int b = e / NV, v = e - b * NV;
            const int gi = e < ns ? b * n + v0 + v : 0; /* nb n < 2^31 */
            bd[u] = d[gi];
            bf[u] = fs[gi];
        }
    }
    /* the norm inputs: x and add stay in separate registers until the weight loads below are
     * issued (adding them here would wait for their memory round trip first) */
    constexpr bool NX = NORM && !PAIR;
    float xv[NX ? NV : 1][CPT], av[NX ? NV : 1][CPT];
    /* PAIR: float4 tid of each h row, and thread (v, b) = (tid / nbh, tid % nbh) decodes block
     * b of embedding row tok[v0 + v] (its token now, its loads after the weights') */
    const int m4h = cols >> 3, mi = tid < m4h ? tid : m4h - 1, nbh = cols >> 6;
    const int ev = tid / nbh, eb = tid - ev * nbh;
    int etok = 0;
    float4 h4[PAIR ? NV : 1];
    if constexpr (PAIR) {
        if (pr.keys) { /* one row: every wave with a decoding thread, all its lanes */
            if ((tid & ~63) < NV * nbh) {
                etok = nmx_keys_token(pr.keys, pr.nkeys);
                if (blockIdx.x == 0 && tid == 0) ((int32_t *)in1)[v0] = etok;
            }
        } else {
            etok = ((const int32_t *)in1)[v0 + (ev < NV ? ev : NV - 1)];
        }
#pragma unroll
        for (int v = 0; v < NV; v++) h4[v] = ((const float4 *)(nx + (size_t)(v0 + v) * xs))[mi];
    }
    if constexpr (NX) { /* rows v0 .. v0 + NV - 1 (+ add): thread columns c = tid + T j */
#pragma unroll
        for (int j = 0; j < CPT; j++) {
            const int cc = tid + T * j;
            const int ci = cc < cols ? cc : cols - 1;
#pragma unroll
            for (int v = 0; v < NV; v++) xv[v][j] = 0.0f, av[v][j] = 0.0f;
            if (T * j >= cols) continue; /* uniform: slot unused by every thread */
#pragma unroll
            for (int v = 0; v < NV; v++) xv[v][j] = nx[(size_t)(v0 + v) * xs + ci];
            if (nadd) {
#pragma unroll
                for (int v = 0; v < NV; v++) av[v][j] = nadd[(size_t)(v0 + v) * as + ci];
            }
        }
    }

    /* ---- phase 0b: weight unit loads: unit = (row u_r, BPU consecutive blocks u_h of one
     * superblock half; UPS units per superblock) ---- */
    constexpr int UPS = 8 / BPU;
    const bool has_unit = tid < R * UPS * nsb;
    const int u_h = has_unit ? tid / R : 0, u_r = has_unit ? tid - u_h * R : 0;
    const int u_sb = u_h / UPS, u_k0 = BPU * (u_h % UPS);
    int wseg = si, wrow;
    if (SWI) { /* rows [0, R/2) gate, [R/2, R) up, both at output index lg * R/2 + r mod R/2 */
        wseg = u_r < R / 2 ? 0 : 1;
        wrow = lg * (R / 2) + (u_r & (R / 2 - 1));
    } else {
        wrow = lg * R + u_r;
    }
    const int wrows = wseg == 0 ? rows0 : tab.s[wseg].rows;
    const int lrow = wrow < wrows ? wrow : wrows - 1;
    const uint8_t *wbase = wseg == 0 ? W0 : tab.s[wseg].W;
    const uint4 *p = (const uint4 *)(wbase + ((size_t)(lrow >> 2) * nsb + u_sb) * 576);
    const int ti = lrow & 3;
    /* unconditional (a thread without a unit reads unit 0's bytes, in bounds, and ignores
     * them): loads in a branch make every later wait also wait for them, so the norm
     * prologue would hold its squares until the weights had landed */
    const uint4 a0 = p[0], a1 = p[1], a2 = p[2], a3 = p[3];
    uint4 c[BPU];
#pragma unroll
    for (int k = 0; k < BPU; k++) c[k] = p[4 + 4 * (u_k0 + k) + ti];

    float ev32[PAIR ? 32 : 1];
    if constexpr (PAIR) {
        if (ev < NV) q4k_block32(pr.E, etok, cols >> 1, eb, ev32);
    }
    if constexpr (NX) { /* the residual add, now that the weight loads are in flight */
        if (nadd) {
#pragma unroll
            for (int j = 0; j < CPT; j++) {
                if (T * j >= cols) continue;
#pragma unroll
                for (int v = 0; v < NV; v++) xv[v][j] = xv[v][j] + av[v][j];
            }
        }
    }

    /* ---- phase 0c: activations into LDS ---- */
    if constexpr (!NORM) {
        for (int r0 = 0; r0 * NQB * T < nq || r0 * NDB * T < ns; r0++) {
            if (r0 > 0) { /* rare: more than one round (very wide rows) */
#pragma unroll
                for (int u = 0; u < NQB; u++) {
                    const int e = (r0 * NQB + u) * T + tid;
                    if (e < nq) {
                        const int b = e / (2 * NV), rem = e - b * 2 * NV;
                        buf[u] = *(const int4 *)(q + ((size_t)b * n + v0 + (rem >> 1)) * 32 + 16 * (rem & 1));
                    }
                }
#pragma unroll
                for (int u = 0; u < NDB; u++) {
                    const int e = (r0 * NDB + u) * T + tid;
                    const int b = e / NV, v = e - b * NV;
                    const int gi = e < ns ? b * n + v0 + v : 0; /* nb n < 2^31 */
                    bd[u] = d[gi];
                    bf[u] = fs[gi];
                }
            }
#pragma unroll
            for (int u = 0; u < NQB; u++) {
                const int e = (r0 * NQB + u) * T + tid;
                if (e < nq) {
                    const int b = e / (2 * NV), rem = e - b * 2 * NV;
                    *(int4 *)(aq + aq_off(b, NV) + (rem >> 1) * 32 + 16 * (rem & 1)) = buf[u];
                }
            }
#pragma unroll
            for (int u = 0; u < NDB; u++) {
                const int e = (r0 * NDB + u) * T + tid;
                if (e < ns) {
                    ad[e] = bd[u];
                    afs[e] = bf[u];
                }
            }
        }
    }
    if constexpr (NORM) {
        /* RMSNorm (sumsq: 4 interleaved partial sums + tail, chain-major squares in LDS) of NR
         * rows of rc columns: the NV input rows, or (PAIR) the NV embedding rows then the NV h
         * rows, each cols / 2 wide */
        constexpr int NR = PAIR ? 2 * NV : NV;
        const int rc = PAIR ? cols >> 1 : cols;
        const int s4 = cm_stride4(rc), rsz = 4 * s4 + 4, m4 = rc >> 2;
        float *sq = (float *)(smem + L.work);
        float *xs = sq + NR * rsz; /* the summed rows [NR][rc] */
        if constexpr (PAIR) {
            if (tid < m4h) { /* h rows (rows NV..): float4 tid = terms tid of the four chains */
#pragma unroll
                for (int v = 0; v < NV; v++) {
                    const float4 x = h4[v];
                    float *sr = sq + (NV + v) * rsz + tid;
                    sr[0] = x.x * x.x;
                    sr[s4] = x.y * x.y;
                    sr[2 * s4] = x.z * x.z;
                    sr[3 * s4] = x.w * x.w;
                    *(float4 *)(xs + (NV + v) * rc + 4 * tid) = x;
                }
            }
            if (ev < NV) { /* embedding block eb of row ev: terms 8 eb .. 8 eb + 7 of chain l are
                            * its values l, l + 4, .., l + 28 */
                float *sr = sq + ev * rsz + 8 * eb;
#pragma unroll
                for (int l = 0; l < 4; l++) {
                    const float *e = ev32 + l;
                    *(float4 *)(sr + l * s4) = make_float4(e[0] * e[0], e[4] * e[4], e[8] * e[8], e[12] * e[12]);
                    *(float4 *)(sr + l * s4 + 4) = make_float4(e[16] * e[16], e[20] * e[20], e[24] * e[24], e[28] * e[28]);
                }
                float *xr = xs + ev * rc + 32 * eb;
#pragma unroll
                for (int u = 0; u < 8; u++)
                    *(float4 *)(xr + 4 * u) = make_float4(ev32[4 * u], ev32[4 * u + 1], ev32[4 * u + 2], ev32[4 * u + 3]);
            }
        } else {
#pragma unroll
        for (int j = 0; j < CPT; j++) {
            const int cc = tid + T * j;
            if (cc >= cols) continue;
            const int ix = cc < 4 * m4 ? (cc & 3) * s4 + (cc >> 2) : 4 * s4 + (cc - 4 * m4);
#pragma unroll
            for (int v = 0; v < NV; v++) {
                sq[v * rsz + ix] = xv[v][j] * xv[v][j];
                xs[v * cols + cc] = xv[v][j];
                if (nm.x_out && blockIdx.x == 0) nm.x_out[(size_t)(v0 + v) * nm.xo_stride + cc] = xv[v][j];
            }
        }
        }
        __syncthreads();
        if (tid < 4 * NR) { /* chain l of row v: two register sets of 32 terms take turns, the
                             * next set requested before the current one is added (scheduling
                             * barriers keep that order; a request past the end re-reads) */
            const float *ch = sq + (tid >> 2) * rsz + (tid & 3) * s4;
            float a = 0.0f;
            int m = 0;
            auto fetch = [&](float4 (&b)[8], int m0) {
#pragma unroll
                for (int u = 0; u < 8; u++) b[u] = *(const float4 *)(ch + m0 + 4 * u);
            };
            auto add = [&](const float4 (&b)[8]) {
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    a = a + b[u].x;
                    a = a + b[u].y;
                    a = a + b[u].z;
                    a = a + b[u].w;
                }
            };
            /* (the second set would spill at 6 or more rows in 1024-thread launches) */
            constexpr bool TWO = NV <= 5 || BPU == 4;
            if (!TWO) {
                for (; m + 32 <= m4; m += 32) {
                    float4 b[8];
                    fetch(b, m);
                    add(b);
                }
            } else if (m4 >= 32) {
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
                if (m + 32 <= m4) { /* ba holds terms m .. m + 31 */
                    add(ba);
                    m += 32;
                }
            }
            for (; m < m4; m++) a = a + ch[m];
            red[tid] = a;
        } else if (tid < 5 * NR) { /* the rc % 4 tail of row v */
            const int v = tid - 4 * NR;
            float t = 0.0f;
            for (int i = 4 * m4; i < rc; i++) t = t + sq[v * rsz + 4 * s4 + (i - 4 * m4)];
            red[tid] = t;
        }
        __syncthreads();
        /* A8 of y = (x * r) * w: a lane pair per (32-column block, vector), 16 columns each;
         * the block's max and code sum are taken over the pair (exact in any order: the same
         * values as a half-wave's lane reductions), the divisions once per lane */
        for (int e2 = tid; e2 < 2 * nb * NV; e2 += T) { /* T is a multiple of 64: pairs stay whole */
            const int e = e2 >> 1, hf = e2 & 1;
            const int b = e / NV, v = e - b * NV;
            int vr = v, bc = b; /* normed row and its block */
            const float *wr = nm.w;
            if constexpr (PAIR) {
                const int half = b >= (nb >> 1) ? 1 : 0;
                vr = half * NV + v;
                bc = b - half * (nb >> 1);
                wr = half ? nm.w : pr.w0;
            }
            const float sv = (red[4 * vr] + red[4 * vr + 1]) + (red[4 * vr + 2] + red[4 * vr + 3]);
            const float r = 1.0f / sqrtf((sv + red[4 * NR + vr]) / (float)rc + nm.eps);
            const float4 *xp = (const float4 *)(xs + vr * rc + 32 * bc + 16 * hf);
            const float4 *wp = (const float4 *)(wr + 32 * bc + 16 * hf);
            float y[16];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const float4 xx = xp[u], ww = wp[u];
                y[4 * u] = (xx.x * r) * ww.x;
                y[4 * u + 1] = (xx.y * r) * ww.y;
                y[4 * u + 2] = (xx.z * r) * ww.z;
                y[4 * u + 3] = (xx.w * r) * ww.w;
            }
            float amax = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; i++) amax = fmaxf(amax, fabsf(y[i]));
            amax = fmaxf(amax, __int_as_float(nmx_dpp<NMX_DPP_XOR1>(__float_as_int(amax))));
            const float id = amax > 0.0f ? 127.0f / amax : 0.0f;
            int sum = 0;
            uint32_t pk[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                uint32_t w4 = 0;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int c = (int)rintf(y[4 * u + i] * id);
                    sum += c;
                    const int cs = c > 127 ? 127 : c < -128 ? -128 : c;
                    w4 |= ((uint32_t)cs & 0xffu) << (8 * i);
                }
                pk[u] = w4;
            }
            sum += nmx_dpp<NMX_DPP_XOR1>(sum);
            *(int4 *)(aq + aq_off(b, NV) + v * 32 + 16 * hf) =
                make_int4((int)pk[0], (int)pk[1], (int)pk[2], (int)pk[3]);
            if (hf == 0) {
                const float dd = amax / 127.0f;
                ad[b * NV + v] = dd;
                afs[b * NV + v] = dd * (float)sum;
            }
        }
    }
    __syncthreads();

    /* ---- phase 1: exact int32 dots of the unit ---- */
    /* The SwiGLU launch (R = 64: a wave's lanes are the 64 rows of one block pair) computes its
     * dots on the matrix cores, as q4k_head_k does: per block two v_mfma_i32_32x32x32_i8 with
     * B = the lane's own row's 32 nibbles and A = the block's activation codes of vector v(m)
     * in the rows m of K group (m / 4) % 2 (zero elsewhere), so every lane receives its own
     * row's exact int32 dots for all NV vectors (4 matrix instructions per block pair instead
     * of 16 NV v_dot4). Every lane of the wave runs them (lanes without a unit read unit 0's
     * bytes and discard the result). */
    constexpr bool MF = SWI && NV >= 3 && BPU == 2;
    typedef int v4i __attribute__((ext_vector_type(4)));
    typedef int v16i __attribute__((ext_vector_type(16)));
    v16i mfd[MF ? BPU : 1];
    if constexpr (MF) {
        const int lane = tid & 63, m = lane & 31, vl = 4 * (m >> 3) + (m & 3);
        const bool diag = ((m >> 2) & 1) == (lane >> 5) && vl < NV;
        const int blk0 = u_sb * 8 + u_k0;
        const v16i zero = {};
#pragma unroll
        for (int k = 0; k < BPU; k++) {
            /* A: entries [8h .. 8h + 3 | 16 + 8h .. | 8h + 4 .. | 16 + 8h + 4 ..] of half h,
             * matching the nibble order of B below */
            const int8_t *xb = diag ? aq + aq_off(blk0 + k, NV) + vl * 32 : (const int8_t *)zl;
            const uint2 ta0 = *(const uint2 *)xb, tb0 = *(const uint2 *)(xb + 16);
            const uint2 ta1 = *(const uint2 *)(xb + 8), tb1 = *(const uint2 *)(xb + 24);
            const v4i x0 = {(int)ta0.x, (int)tb0.x, (int)ta0.y, (int)tb0.y};
            const v4i x1 = {(int)ta1.x, (int)tb1.x, (int)ta1.y, (int)tb1.y};
            /* B: the low nibbles of code bytes 4u .. 4u + 3 are columns 4u .., the high ones
             * columns 16 + 4u .. */
            const uint4 w = c[k];
            const v4i b0 = {(int)(w.x & 0x0f0f0f0fu), (int)((w.x >> 4) & 0x0f0f0f0fu),
                            (int)(w.y & 0x0f0f0f0fu), (int)((w.y >> 4) & 0x0f0f0f0fu)};
            const v4i b1 = {(int)(w.z & 0x0f0f0f0fu), (int)((w.z >> 4) & 0x0f0f0f0fu),
                            (int)(w.w & 0x0f0f0f0fu), (int)((w.w >> 4) & 0x0f0f0f0fu)};
            mfd[k] = __builtin_amdgcn_mfma_i32_32x32x32_i8(x0, b0, zero, 0, 0, 0);
            mfd[k] = __builtin_amdgcn_mfma_i32_32x32x32_i8(x1, b1, mfd[k], 0, 0, 0);
        }
    }
    if (has_unit) {
        const int sh8 = 8 * ti;
        const uint32_t dw = (ti & 2) ? a0.y : a0.x, mw = (ti & 2) ? a0.w : a0.z;
        const float D = half_bits(dw >> (16 * (ti & 1)));
        const float M = half_bits(mw >> (16 * (ti & 1)));
        int s6[4], m6[4]; /* the 4 blocks of the unit's superblock half */
        decode6_half(a1.x, a1.y, a1.z, a1.w, a2.x, a2.y, sh8, u_k0 >> 2, s6);
        decode6_half(a2.z, a2.w, a3.x, a3.y, a3.z, a3.w, sh8, u_k0 >> 2, m6);
        const int blk0 = u_sb * 8 + u_k0, kh = u_k0 & 3; /* kh: first block within the half */
        /* the unit's BPU blocks x NV scales d and fsum (BPU NV consecutive floats each; as NV
         * float4 for 4-block units, 16-byte aligned), then the activations block by block, the
         * next block's 2 NV reads issued before the current block's dots */
        float sdv[BPU * NV], sfv[BPU * NV];
        if constexpr (BPU == 4) {
#pragma unroll
            for (int i = 0; i < NV; i++) {
                const float4 x = *(const float4 *)(ad + blk0 * NV + 4 * i);
                const float4 y = *(const float4 *)(afs + blk0 * NV + 4 * i);
                sdv[4 * i] = x.x, sdv[4 * i + 1] = x.y, sdv[4 * i + 2] = x.z, sdv[4 * i + 3] = x.w;
                sfv[4 * i] = y.x, sfv[4 * i + 1] = y.y, sfv[4 * i + 2] = y.z, sfv[4 * i + 3] = y.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < BPU * NV; i++) sdv[i] = ad[blk0 * NV + i], sfv[i] = afs[blk0 * NV + i];
        }
        int4 xa[MF ? 1 : NV][2], xn[MF ? 1 : NV][2];
        if constexpr (!MF) {
#pragma unroll
            for (int v = 0; v < NV; v++) {
                const int8_t *xb = aq + aq_off(blk0, NV) + v * 32;
                xa[v][0] = *(const int4 *)xb, xa[v][1] = *(const int4 *)(xb + 16);
            }
        }
#pragma unroll
        for (int k = 0; k < BPU; k++) {
            const int blk = blk0 + k;
            if (!MF && k < BPU - 1) {
#pragma unroll
                for (int v = 0; v < NV; v++) {
                    const int8_t *xb = aq + aq_off(blk + 1, NV) + v * 32;
                    xn[v][0] = *(const int4 *)xb, xn[v][1] = *(const int4 *)(xb + 16);
                }
            }
            const float sc = D * (float)s6[kh + k]; /* exact: 6-bit x 11-bit mantissa */
            const float of = M * (float)m6[kh + k];
            if constexpr (!REC) lof[u_r * (nb | 1) + blk] = -of;
            const int lo0 = (int)(c[k].x & 0x0f0f0f0fu), hi0 = (int)((c[k].x >> 4) & 0x0f0f0f0fu);
            const int lo1 = (int)(c[k].y & 0x0f0f0f0fu), hi1 = (int)((c[k].y >> 4) & 0x0f0f0f0fu);
            const int lo2 = (int)(c[k].z & 0x0f0f0f0fu), hi2 = (int)((c[k].z >> 4) & 0x0f0f0f0fu);
            const int lo3 = (int)(c[k].w & 0x0f0f0f0fu), hi3 = (int)((c[k].w >> 4) & 0x0f0f0f0fu);
            if constexpr (MF) {
#pragma unroll
                for (int v = 0; v < NV; v++)
                    lp[(v * R + u_r) * (nb | 1) + blk] = make_float2((float)mfd[k][v], sc * sdv[k * NV + v]);
                continue;
            }
#pragma unroll
            for (int v = 0; v < NV; v++) {
                const int4 x0 = xa[MF ? 0 : v][0], x1 = xa[MF ? 0 : v][1];
                int dot = __builtin_amdgcn_sdot4(lo0, x0.x, 0, false);
                dot = __builtin_amdgcn_sdot4(lo1, x0.y, dot, false);
                dot = __builtin_amdgcn_sdot4(lo2, x0.z, dot, false);
                dot = __builtin_amdgcn_sdot4(lo3, x0.w, dot, false);
                dot = __builtin_amdgcn_sdot4(hi0, x1.x, dot, false);
                dot = __builtin_amdgcn_sdot4(hi1, x1.y, dot, false);
                dot = __builtin_amdgcn_sdot4(hi2, x1.z, dot, false);
                dot = __builtin_amdgcn_sdot4(hi3, x1.w, dot, false);
                if constexpr (REC)
                    rec[(v * R + u_r) * (nb | 1) + blk] =
                        make_float4((float)dot, sc * sdv[k * NV + v], -of, sfv[k * NV + v]);
                else
                    lp[(v * R + u_r) * (nb | 1) + blk] =
                        make_float2((float)dot, sc * sdv[k * NV + v]);
            }
            if (k < BPU - 1) {
#pragma unroll
                for (int v = 0; v < (MF ? 1 : NV); v++) xa[v][0] = xn[v][0], xa[v][1] = xn[v][1];
            }
        }
    }
    __syncthreads();

    /* ---- phase 2: the fp32 chain of (row, vector) in column order ---- */
    const bool chain = tid < R * NV;
    const int cv = chain ? tid / R : 0;
    const int cr = chain ? tid - cv * R : 0;
    float acc = 0.0f;
    if (chain) {
        /* per block: acc = fma((float)dot, (D*s)*d_v, acc); acc = fma(-(M*m), fsum_v, acc) */
        if constexpr (REC) {
            /* the chain's records are contiguous: one base, immediate offsets */
            const float4 *rp = rec + (cv * R + cr) * (nb | 1);
            int b = 0;
            for (; b + 8 <= nb; b += 8) {
                float4 r[8];
#pragma unroll
                for (int u = 0; u < 8; u++) r[u] = rp[b + u];
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    acc = __builtin_fmaf(r[u].x, r[u].y, acc);
                    acc = __builtin_fmaf(r[u].z, r[u].w, acc);
                }
            }
            for (; b < nb; b++) {
                const float4 r = rp[b];
                acc = __builtin_fmaf(r.x, r.y, acc);
                acc = __builtin_fmaf(r.z, r.w, acc);
            }
        } else {
        const float2 *pp = lp + (cv * R + cr) * (nb | 1);
        const float *op = lof + cr * (nb | 1);
        const float *fp = afs + cv; /* uniform in a wave (R = 64) */
        int b = 0;
        for (; b + 8 <= nb; b += 8) {
            float2 pv[8];
            float of[8], ff[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                pv[u] = pp[b + u];
                of[u] = op[b + u];
                ff[u] = fp[(b + u) * NV];
            }
#pragma unroll
            for (int u = 0; u < 8; u++) {
                acc = __builtin_fmaf(pv[u].x, pv[u].y, acc);
                acc = __builtin_fmaf(of[u], ff[u], acc);
            }
        }
        for (; b < nb; b++) {
            const float2 pv = pp[b];
            const float ff = fp[b * NV];
            acc = __builtin_fmaf(pv.x, pv.y, acc);
            acc = __builtin_fmaf(op[b], ff, acc);
        }
        }
    }
    if constexpr (!SWI) {
        if (chain) {
            const int row = lg * R + cr;
            if (row < tab.s[si].rows)
                tab.s[si].Y[(size_t)(v0 + cv) * tab.s[si].ystride + row] = acc;
        }
    } else {
        /* SwiGLU (engine/src/forward_ops.c:98-110): y = silu(gate) * up, then its A8 */
        float *res = (float *)(smem + L.res);
        if (chain) res[cv * R + cr] = acc;
        __syncthreads();
        const int H2 = R / 2; /* == 32: one A8 block per vector */
        if (tid < NV * H2) {
            const int v = tid / H2, j = tid - v * H2;
            const int col = lg * H2 + j;
            const float y = nmx_silu(res[v * R + j]) * res[v * R + H2 + j];
            if (tab.s[0].Y) tab.s[0].Y[(size_t)(v0 + v) * tab.s[0].ystride + col] = y;
            const size_t u = (size_t)(col >> 5) * n + v0 + v;
            nmx_a8_store(y, oq + u * 32, od + u, ofs + u);
        }
    }
}

/* Rows per workgroup for a pass of nv vectors, its threads and blocks per dot unit (*bpu).
 * SwiGLU needs R = 64 (32 gate + 32 up rows = one A8 block). The other launches use chain
 * records and R = 4: measured on the verify shapes (1024 .. 3584 columns, 5 vectors) this beat
 * every larger R (8 by about 1 tok/s end to end: twice the workgroups, so every CU streams
 * weights, each with the same short dot and chain phases). Without a norm prologue, each unit thread takes one block
 * when the workgroup's units fit in 1024 threads, else 4 (at most 256 threads): a unit's blocks
 * are one dependent sequence of LDS reads, dots and record stores, so more units shorten the
 * dot phase. */
int pick_rows(int cols, int nv, bool norm, bool swiglu, int total_rows, int count, int *threads,
              int *bpu, bool pair = false) {
    *bpu = 4;
    const int nsb = cols >> 8;
    if (norm && !swiglu) {
        /* every workgroup redoes the norm prologue: the fewest rows per workgroup (a multiple
         * of 4) whose workgroups fit the 256 CUs in one round */
        for (int R = 4 * ((total_rows + 4 * 256 - 1) / (4 * 256)); R <= 64; R += 4) {
            if (R * 256 < total_rows + count * R) continue; /* each segment rounds up */
            if (mt_layout(cols, nv, R, true, false, pair).total > MT_LDS) break;
            /* 1- or 2-block units in up to 1024 threads (2 prologue columns per thread) when
             * they fit, else 4-block units (8 columns per thread, up to 512 threads); PAIR:
             * one-block units, a float4 of each half per thread */
            for (int b = 1; b <= (pair ? 1 : 4); b *= 2) {
                const int units = R * (8 / b) * nsb;
                const int t = 64 * (((units > R * nv ? units : R * nv) + 63) / 64);
                const int cpt = pair ? 8 : b < 4 ? 2 : MT_NORM_CPT;
                int tt = t * cpt < cols ? 64 * ((cols / cpt + 63) / 64) : t;
                /* the norm's four chains and tail of each of its (PAIR: 2 nv) rows take one
                 * thread each */
                const int tmin = 64 * ((5 * (pair ? 2 : 1) * nv + 63) / 64);
                tt = tt < tmin ? tmin : tt;
                if (tt > (b < 4 ? MT_REC_THREADS : MT_NORM_THREADS)) continue;
                *threads = tt;
                *bpu = b;
                return R;
            }
            break;
        }
        return 0;
    }
    for (int R = swiglu ? 64 : 4; R >= 4; R >>= 1) {
        if (swiglu && R != 64) break;
        if (!swiglu && !norm) *bpu = R * 8 * nsb <= MT_REC_THREADS ? 1 : 4;
        if (swiglu) *bpu = R * 4 * nsb <= MT_REC_THREADS ? 2 : 4;
        const int units = R * (8 / *bpu) * nsb;
        const int t = 64 * (((units > R * nv ? units : R * nv) + 63) / 64);
        if (t > (*bpu < 4 ? MT_REC_THREADS : norm ? MT_NORM_THREADS : swiglu ? MT_MAX_THREADS : MT_REC4_THREADS))
            continue;
        if (mt_layout(cols, nv, R, norm, swiglu).total > MT_LDS) continue;
        if (norm && cols > t * (*bpu < 4 ? 2 : MT_NORM_CPT)) continue;
        *threads = t;
        return R;
    }
    return 0;
}

/* Launch bound of q4k_mt_k<NV, NORM, SWI, BPU, PAIR> (its __launch_bounds__). */
constexpr int mt_bound(bool norm, bool swi, int bpu) {
    return bpu < 4 ? MT_REC_THREADS : norm ? MT_NORM_THREADS : swi ? MT_MAX_THREADS : MT_REC4_THREADS;
}

/* Whether T threads give every phase of q4k_mt_k<nv, norm, swi, bpu, pair> at R rows per
 * workgroup and cols columns the threads that phase assumes; NULL if so, else the first need
 * that fails. A phase whose work items outnumber its threads would leave LDS that a later
 * phase reads unwritten, so the launch refuses such a geometry.
 *   - the weight units: one thread per (row, BPU-block unit), R (8 / bpu) (cols / 256);
 *   - the chains: one thread per (row, vector), R nv;
 *   - the plain norm prologue: T columns per step, CPT steps (2 for 1- and 2-block units,
 *     else MT_NORM_CPT), so T CPT >= cols;
 *   - the norm's chains and tails: 4 + 1 threads per normed row (nv rows; PAIR 2 nv);
 *   - PAIR: one float4 of each h row per thread (cols / 8) and one embedding block of each
 *     row per thread (nv cols / 64);
 *   - SwiGLU: R = 64 and one thread per (vector, output column), nv R / 2.
 * Loops that stride by T (the activation staging, the A8 of the normed rows) need only T to
 * be a multiple of 64 (lane pairs stay in one wave). */
const char *mt_geometry_error(int cols, int nv, int R, int T, int bpu, bool norm, bool swi,
                              bool pair) {
    const int nsb = cols >> 8;
    if (cols <= 0 || cols % 256) return "cols not a multiple of 256";
    if (nv < 1 || nv > MT_MAX_NV) return "vectors per pass";
    if (bpu != 1 && bpu != 2 && bpu != 4) return "blocks per unit";
    if (R < 4 || R % 4) return "rows per workgroup";
    if (T < 64 || T % 64) return "threads not a multiple of 64";
    if (T > mt_bound(norm, swi, bpu)) return "threads above the launch bound";
    if (T < R * (8 / bpu) * nsb) return "threads for the weight units";
    if (T < R * nv) return "threads for the chains";
    if (pair && (!norm || swi || bpu != 1 || cols % 512)) return "PAIR variant";
    if (norm && !pair && T * (bpu < 4 ? 2 : MT_NORM_CPT) < cols) return "threads for the norm columns";
    if (norm && T < 5 * (pair ? 2 : 1) * nv) return "threads for the norm chains";
    if (pair && T < cols / 8) return "threads for the h float4s";
    if (pair && T < nv * (cols / 64)) return "threads for the embedding blocks";
    if (swi && (R != 64 || T < nv * (R / 2))) return "SwiGLU rows or epilogue threads";
    if (mt_layout(cols, nv, R, norm, swi, pair).total > MT_LDS) return "LDS";
    return nullptr;
}

template <int NV, bool NORM, bool SWI, int BPU, bool PAIR = false>
int launch_one(nmx_ctx *ctx, const MtTab &tab, int groups, int cols, int n, int v0, int R, int T,
               const int8_t *q, const float *d, const float *fs, const nmx_norm_in &nm,
               nmx_a8 out, const nmx_mt_pair *pair = nullptr) {
    static bool ready = false; /* idempotent: a racing second call sets the same value */
    if (!ready) {
        NMX_HIP(ctx, hipFuncSetAttribute((const void *)q4k_mt_k<NV, NORM, SWI, BPU, PAIR>,
                                         hipFuncAttributeMaxDynamicSharedMemorySize, MT_LDS));
        ready = true;
    }
    if (const char *why = mt_geometry_error(cols, NV, R, T, BPU, NORM, SWI, PAIR))
        return nmx_fail(ctx, "q4k_mt: geometry cols=%d nv=%d R=%d T=%d bpu=%d: %s", cols, NV, R,
                        T, BPU, why);
    const size_t lds = (size_t)mt_layout(cols, NV, R, NORM, SWI, PAIR).total;
    const void *in0 = NORM ? (const void *)nm.x : (const void *)q;
    const void *in1 = NORM ? (const void *)nm.add : (const void *)d;
    uint64_t aux = NORM ? ((uint64_t)(uint32_t)nm.add_stride << 32) | (uint32_t)nm.x_stride
                        : (uint64_t)(uintptr_t)fs;
    MtPair pr{nullptr, nullptr, nullptr, 0};
    if (PAIR) {
        in0 = pair->h;
        in1 = pair->tok;
        aux = (uint32_t)pair->h_stride;
        pr = MtPair{pair->E, pair->w_emb, pair->keys, pair->nkeys};
    }
    q4k_mt_k<NV, NORM, SWI, BPU, PAIR><<<dim3((unsigned)groups), dim3((unsigned)T), lds, ctx->stream>>>(
        in0, in1, aux, (const uint8_t *)tab.s[0].W, cols, n, v0, R, T, tab.s[0].rows, tab, nm,
        out.q, out.d, out.fs, pr);
    NMX_LAUNCHED(ctx, "q4k_mt");
    return 0;
}

template <int NV>
int launch_nv(nmx_ctx *ctx, const MtTab &tab, int groups, int cols, int n, int v0, int R, int T,
              int bpu, const int8_t *q, const float *d, const float *fs, const nmx_norm_in *nm,
              bool swiglu, nmx_a8 out, const nmx_mt_pair *pair) {
    const nmx_norm_in none{};
    if (pair) return launch_one<NV, true, false, 1, true>(ctx, tab, groups, cols, n, v0, R, T, q, d, fs, *nm, out, pair);
    if (nm && swiglu && bpu == 2) return launch_one<NV, true, true, 2>(ctx, tab, groups, cols, n, v0, R, T, q, d, fs, *nm, out);
    if (nm && swiglu) return launch_one<NV, true, true, 4>(ctx, tab, groups, cols, n, v0, R, T, q, d, fs, *nm, out);
    if (nm && bpu == 1) return launch_one<NV, true, false, 1>(ctx, tab, groups, cols, n, v0, R, T, q, d, fs, *nm, out);
    if (nm && bpu == 2) return launch_one<NV, true, false, 2>(ctx, tab, groups, cols, n, v0, R, T, q, d, fs, *nm, out);
    if (nm) return launch_one<NV, true, false, 4>(ctx, tab, groups, cols, n, v0, R, T, q, d, fs, *nm, out);
    if (swiglu && bpu == 2) return launch_one<NV, false, true, 2>(ctx, tab, groups, cols, n, v0, R, T, q, d, fs, none, out);
    if (swiglu) return launch_one<NV, false, true, 4>(ctx, tab, groups, cols, n, v0, R, T, q, d, fs, none, out);
    if (bpu == 1) return launch_one<NV, false, false, 1>(ctx, tab, groups, cols, n, v0, R, T, q, d, fs, none, out);
    return launch_one<NV, false, false, 4>(ctx, tab, groups, cols, n, v0, R, T, q, d, fs, none, out);
}

/* The geometry of an n-vector product over count matrices (rows[s] rows each): 0 and the
 * plan when q4k_mt_k takes the shape, 1 when the shape belongs to the other kernels. The
 * passes are equal-size groups of at most MT_MAX_NV vectors, larger first (every pass performs
 * the same per-vector operations, so the split does not change any result); the first pass's
 * thread count covers every pass. */
struct MtPlan {
    int R, T, bpu, nv_max;
};

int mt_plan(int count, const int *rows, int cols, int n, bool norm, bool swiglu, bool pair,
            MtPlan *pl) {
    if (count < 1 || count > NMX_MAX_SEGS || cols <= 0 || cols % 256 || n < 1 || n > MT_MAX_NV)
        return 1;
    if (swiglu && (count != 2 || rows[0] != rows[1] || rows[0] % 32)) return 1;
    if (pair && (!norm || swiglu || cols % 512)) return 1;
    const int passes = (n + MT_MAX_NV - 1) / MT_MAX_NV;
    pl->nv_max = (n + passes - 1) / passes;
    int total_rows = 0;
    for (int s = 0; s < count; s++) total_rows += rows[s];
    pl->T = 0;
    pl->bpu = 4;
    pl->R = pick_rows(cols, pl->nv_max, norm, swiglu, total_rows, count, &pl->T, &pl->bpu, pair);
    return pl->R ? 0 : 1;
}

/* Vectors of each pass: the largest-first equal split of n into passes of <= MT_MAX_NV. */
int mt_pass_nv(int left) {
    const int np = (left + MT_MAX_NV - 1) / MT_MAX_NV;
    return (left + np - 1) / np;
}

} // namespace

int nmx_mt_matmul(nmx_ctx *ctx, int count, const nmx_mt_seg *segs, int cols, int n,
                  const int8_t *q, const float *d, const float *fs, const nmx_norm_in *norm,
                  bool swiglu, nmx_a8 out, const nmx_mt_pair *pair) {
    /* more rows than one pass: the row-per-lane / K-split kernels read the weights once for
     * all of them (prefill chunks) */
    if (count < 1 || count > NMX_MAX_SEGS) return 1;
    if (pair && ((uintptr_t)pair->w_emb & 15 || (uintptr_t)pair->h & 15 || pair->h_stride % 4 ||
                 (pair->keys && n != 1)))
        return 1;
    /* the fused norm reads its weight as float4 */
    if (norm && ((uintptr_t)norm->w & 15)) return 1;
    int rows[NMX_MAX_SEGS];
    for (int s = 0; s < count; s++) rows[s] = segs[s].rows;
    MtPlan pl;
    if (mt_plan(count, rows, cols, n, norm != nullptr, swiglu, pair != nullptr, &pl)) return 1;
    const int R = pl.R, T = pl.T, bpu = pl.bpu;
    MtTab tab{};
    tab.count = count;
    int groups = 0;
    for (int s = 0; s < count; s++) {
        tab.s[s] = segs[s];
        tab.g0[s] = groups;
        if (!swiglu) groups += (segs[s].rows + R - 1) / R;
    }
    if (swiglu) {
        groups = segs[0].rows / (R / 2);
        tab.g0[1] = groups; /* never selected: both halves are addressed from segment 0 */
    }
    for (int v0 = 0; v0 < n;) {
        const int nv = mt_pass_nv(n - v0);
        const int Tn = T; /* the first (largest) pass's thread count covers every pass */
        int rc;
        switch (nv) {
        case 8: rc = launch_nv<8>(ctx, tab, groups, cols, n, v0, R, Tn, bpu, q, d, fs, norm, swiglu, out, pair); break;
        case 7: rc = launch_nv<7>(ctx, tab, groups, cols, n, v0, R, Tn, bpu, q, d, fs, norm, swiglu, out, pair); break;
        case 6: rc = launch_nv<6>(ctx, tab, groups, cols, n, v0, R, Tn, bpu, q, d, fs, norm, swiglu, out, pair); break;
        case 5: rc = launch_nv<5>(ctx, tab, groups, cols, n, v0, R, Tn, bpu, q, d, fs, norm, swiglu, out, pair); break;
        case 4: rc = launch_nv<4>(ctx, tab, groups, cols, n, v0, R, Tn, bpu, q, d, fs, norm, swiglu, out, pair); break;
        case 3: rc = launch_nv<3>(ctx, tab, groups, cols, n, v0, R, Tn, bpu, q, d, fs, norm, swiglu, out, pair); break;
        case 2: rc = launch_nv<2>(ctx, tab, groups, cols, n, v0, R, Tn, bpu, q, d, fs, norm, swiglu, out, pair); break;
        default: rc = launch_nv<1>(ctx, tab, groups, cols, n, v0, R, Tn, bpu, q, d, fs, norm, swiglu, out, pair); break;
        }
        if (rc) return rc;
        v0 += nv;
    }
    return 0;
}

extern "C" {

int nmx_mt_plan(int count, const int *rows, int cols, int n, int norm, int swiglu, int pair,
                nmx_mt_geometry *g) {
    if (!rows || !g || count < 1 || count > NMX_MAX_SEGS) return 0;
    for (int s = 0; s < count; s++)
        if (rows[s] <= 0 || rows[s] % 4) return 0;
    MtPlan pl;
    if (mt_plan(count, rows, cols, n, norm != 0, swiglu != 0, pair != 0, &pl)) return 0;
    *g = nmx_mt_geometry{};
    g->rows_per_wg = pl.R;
    g->threads = pl.T;
    g->blocks_per_unit = pl.bpu;
    int groups = 0;
    for (int s = 0; s < count; s++) groups += (rows[s] + pl.R - 1) / pl.R;
    g->workgroups = swiglu ? rows[0] / (pl.R / 2) : groups;
    int rc = 1;
    for (int v0 = 0; v0 < n;) {
        const int nv = mt_pass_nv(n - v0);
        g->nv[g->passes] = nv;
        g->lds_bytes[g->passes] = mt_layout(cols, nv, pl.R, norm != 0, swiglu != 0, pair != 0).total;
        g->passes++;
        if (mt_geometry_error(cols, nv, pl.R, pl.T, pl.bpu, norm != 0, swiglu != 0, pair != 0))
            rc = -1;
        v0 += nv;
    }
    return rc;
}

int nmx_q4k_matmul_norm(nmx_ctx *ctx, int count, const void *const *W, const int *rows,
                        float *const *Y, const int *y_stride, int cols, int n,
                        const nmx_norm_in *in, nmx_a8 a8_tmp) {
    if (!ctx) return -1;
    if (!in || !in->x || !in->w || count < 1 || count > NMX_MAX_SEGS || !W || !rows || !Y ||
        !y_stride || cols <= 0 || cols % 256 || cols > 65536 || n < 1 || n > 64 ||
        in->x_stride < cols || (in->add && in->add_stride < cols) ||
        (in->x_out && in->xo_stride < cols))
        return nmx_fail(ctx, "nmx_q4k_matmul_norm: bad arguments");
    const size_t xb = ((size_t)(n - 1) * in->x_stride + cols) * 4;
    if (in->x_out) {
        const size_t ob = ((size_t)(n - 1) * in->xo_stride + cols) * 4;
        if (nmx_overlap(in->x_out, ob, in->x, xb) ||
            (in->add && nmx_overlap(in->x_out, ob, in->add, ((size_t)(n - 1) * in->add_stride + cols) * 4)))
            return nmx_fail(ctx, "nmx_q4k_matmul_norm: x_out aliases x or add");
    }
    nmx_mt_seg segs[NMX_MAX_SEGS];
    int total = 0;
    for (int s = 0; s < count; s++) {
        if (!W[s] || !Y[s] || rows[s] <= 0 || rows[s] % 4 || y_stride[s] < rows[s])
            return nmx_fail(ctx, "nmx_q4k_matmul_norm: bad matrix %d", s);
        const size_t yb = ((size_t)(n - 1) * y_stride[s] + rows[s]) * 4;
        if (nmx_overlap(Y[s], yb, in->x, xb) ||
            (in->add && nmx_overlap(Y[s], yb, in->add, ((size_t)(n - 1) * in->add_stride + cols) * 4)))
            return nmx_fail(ctx, "nmx_q4k_matmul_norm: output %d aliases the norm input", s);
        segs[s] = nmx_mt_seg{(const uint8_t *)W[s], Y[s], rows[s], y_stride[s]};
        total += rows[s];
    }
    if (total < 32768) {
        const int rc = nmx_mt_matmul(ctx, count, segs, cols, n, nullptr, nullptr, nullptr, in,
                                     false, nmx_a8{});
        if (rc <= 0) return rc;
    }
    if (!a8_tmp.q || !a8_tmp.d || !a8_tmp.fs)
        return nmx_fail(ctx, "nmx_q4k_matmul_norm: shape needs the a8_tmp buffers");
    if (nmx_rmsnorm_xo(ctx, in->x, in->x_stride, in->add, in->add_stride, in->x_out,
                       in->xo_stride, in->w, n, cols, in->eps, nullptr, 0, a8_tmp))
        return -1;
    return nmx_q4k_matmul_multi(ctx, count, W, rows, Y, y_stride, cols, n, a8_tmp.q, a8_tmp.d,
                                a8_tmp.fs);
}

int nmx_q4k_matmul_embed_norm(nmx_ctx *ctx, const void *W, int rows, float *Y, int y_stride,
                              int n, int H, const void *E, int vocab, int32_t *tok,
                              const float *w_emb, const float *h, int h_stride,
                              const float *w_hid, float eps, nmx_a8 a8_tmp,
                              const void *tok_keys, int nkeys) {
    if (!ctx) return -1;
    if (!W || !Y || !E || !tok || !w_emb || !h || !w_hid || rows <= 0 || rows % 4 ||
        y_stride < rows || H < 256 || H % 256 || H > 32768 || vocab <= 0 || vocab % 4 ||
        n < 1 || n > 4096 || h_stride < H ||
        (tok_keys && (n != 1 || nkeys < 1 || (uintptr_t)tok_keys % 8)))
        return nmx_fail(ctx, "nmx_q4k_matmul_embed_norm: bad arguments");
    if (nmx_overlap(Y, ((size_t)(n - 1) * y_stride + rows) * 4, h,
                    ((size_t)(n - 1) * h_stride + H) * 4))
        return nmx_fail(ctx, "nmx_q4k_matmul_embed_norm: Y aliases h");
    if (n <= MT_MAX_NV && rows < 32768) {
        const nmx_norm_in nm{nullptr, 0, nullptr, 0, nullptr, 0, w_hid, eps};
        const nmx_mt_pair pr{(const uint8_t *)E, tok, w_emb, h, h_stride,
                             (const unsigned long long *)tok_keys, nkeys};
        const nmx_mt_seg seg{(const uint8_t *)W, Y, rows, y_stride};
        const int rc = nmx_mt_matmul(ctx, 1, &seg, 2 * H, n, nullptr, nullptr, nullptr, &nm, false,
                                     nmx_a8{}, &pr);
        if (rc <= 0) return rc;
    }
    /* the two calls: both halves' A8 blocks into a8_tmp ([block][n][32], the embedding's
     * blocks first), then the matmul */
    if (tok_keys) return nmx_fail(ctx, "nmx_q4k_matmul_embed_norm: keys need the fused shape");
    if (!a8_tmp.q || !a8_tmp.d || !a8_tmp.fs)
        return nmx_fail(ctx, "nmx_q4k_matmul_embed_norm: shape needs the a8_tmp buffers");
    const size_t hb = (size_t)(H / 32) * n;
    const nmx_a8 a1 = {a8_tmp.q + hb * 32, a8_tmp.d + hb, a8_tmp.fs + hb};
    if (nmx_embed_norm(ctx, E, vocab, tok, n, H, eps, w_emb, nullptr, 0, nullptr, 0, a8_tmp, h,
                       h_stride, w_hid, nullptr, 0, a1))
        return -1;
    return nmx_q4k_matmul(ctx, W, rows, 2 * H, n, a8_tmp.q, a8_tmp.d, a8_tmp.fs, Y, y_stride,
                          nullptr);
}

int nmx_q4k_swiglu(nmx_ctx *ctx, const void *Wg, const void *Wu, int ffn, int cols, int n,
                   const int8_t *q, const float *d, const float *fsum, const nmx_norm_in *in,
                   float *y, nmx_a8 out, nmx_a8 a8_tmp, float *gate_tmp, float *up_tmp) {
    if (!ctx) return -1;
    if (!Wg || !Wu || ffn <= 0 || ffn % 32 || cols <= 0 || cols % 256 || cols > 65536 || n < 1 ||
        n > 64 || !out.q || !out.d || !out.fs || (!in && (!q || !d || !fsum)) ||
        (in && (!in->x || !in->w || in->x_stride < cols || (in->add && in->add_stride < cols) ||
                (in->x_out && in->xo_stride < cols))))
        return nmx_fail(ctx, "nmx_q4k_swiglu: bad arguments");
    if (in && in->x_out && nmx_overlap(in->x_out, ((size_t)(n - 1) * in->xo_stride + cols) * 4,
                                       in->x, ((size_t)(n - 1) * in->x_stride + cols) * 4))
        return nmx_fail(ctx, "nmx_q4k_swiglu: x_out aliases x");
    const nmx_mt_seg segs[2] = {{(const uint8_t *)Wg, y, ffn, ffn}, {(const uint8_t *)Wu, nullptr, ffn, ffn}};
    if (2 * ffn < 65536) {
        const int rc = nmx_mt_matmul(ctx, 2, segs, cols, n, q, d, fsum, in, true, out);
        if (rc <= 0) return rc;
    }
    if (!gate_tmp || !up_tmp || (in && (!a8_tmp.q || !a8_tmp.d || !a8_tmp.fs)))
        return nmx_fail(ctx, "nmx_q4k_swiglu: shape needs the temporary buffers");
    if (in) {
        if (nmx_rmsnorm_xo(ctx, in->x, in->x_stride, in->add, in->add_stride, in->x_out,
                           in->xo_stride, in->w, n, cols, in->eps, nullptr, 0, a8_tmp))
            return -1;
        q = a8_tmp.q, d = a8_tmp.d, fsum = a8_tmp.fs;
    }
    const void *W[2] = {Wg, Wu};
    const int R[2] = {ffn, ffn};
    float *Y[2] = {gate_tmp, up_tmp};
    if (nmx_q4k_matmul_multi(ctx, 2, W, R, Y, R, cols, n, q, d, fsum)) return -1;
    return nmx_silu_mul(ctx, gate_tmp, up_tmp, ffn, n, ffn, y, out);
}

} /* extern "C" */
