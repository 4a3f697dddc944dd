/* Verify-step glue kernels for gfx950: embedding rows, RMSNorm (+ residual add, + A8 of the
 * result), Gated DeltaNet pre (causal conv + SiLU, q/k L2 norm, beta / decay gates) and post
 * (gated RMSNorm), SwiGLU, gated full attention (q/k norm, partial RoPE, KV store, causal GQA
 * softmax attention, sigmoid gate), the rollback commit, and the control block.
 *
 * Every reduction keeps the reference's fixed order (engine/src/forward_ops.c: 4 interleaved
 * partial sums combined (c0+c1)+(c2+c3) then a sequential tail; pf_dot's 16 partial sums;
 * row-order P.V), no fused multiply-add anywhere (compiled with -ffp-contract=off), IEEE
 * divide and sqrt, and the reference's exp (pf_expf, a Cephes-style polynomial) for every
 * SiLU / sigmoid / softmax. The DeltaNet gates use the binary64-evaluated exp / log1p of
 * nmx_math.h in place of glibc's expf / log1pf. */
#include "nmx_internal.h"
#include "nmx_math.h"
#include "nmx_a8.h"
#include "nmx_lanes.h"
#include "nmx_rms.h"

namespace {

/* ---- A8 of one 32-value block held by a 32-lane half-wave (lane = column within block),
 * written as the block-major element (b, v) of an [nb][n] layout (nmx_a8.h). */
__device__ __forceinline__ void a8_block(float x, int b, int v, int n, int8_t *q, float *d,
                                         float *fs) {
    const size_t u = (size_t)b * n + v;
    nmx_a8_store(x, q + u * 32, d + u, fs + u);
}

/* Sum in the reference's order (sumsq forward_ops.c:168-189, pf_softmax_exp :333-353):
 * partial l accumulates v[4m + l] for m ascending over the first cols/4*4 elements;
 * s = (c0 + c1) + (c2 + c3); the tail sequentially into t; result s + t. v[] is in LDS in
 * element order; four lanes run the four chains, reading 16 values per batch so the LDS
 * latency overlaps the dependent adds. Every thread of the block gets the result. */
__device__ float ordered_sum4(const float *sq, int cols, float *red) {
    const int tid = threadIdx.x, m4 = cols >> 2;
    if (tid < 4) {
        float c = 0.0f;
        int m = 0;
        for (; m + 16 <= m4; m += 16) {
            float b[16];
#pragma unroll
            for (int u = 0; u < 16; u++) b[u] = sq[4 * (m + u) + tid];
#pragma unroll
            for (int u = 0; u < 16; u++) c = c + b[u];
        }
        for (; m < m4; m++) c = c + sq[4 * m + tid];
        red[tid] = c;
    } else if (tid == 4) {
        float t = 0.0f;
        for (int i = m4 * 4; i < cols; i++) t = t + sq[i];
        red[4] = t;
    }
    __syncthreads();
    const float s = (red[0] + red[1]) + (red[2] + red[3]);
    const float r = s + red[4];
    __syncthreads();
    return r;
}

/* ---- embedding rows of a Q4K matrix (engine/src/kern_act.c:53-88) ---- */
__global__ __launch_bounds__(256) void embed_k(const uint8_t *__restrict__ W, int cols,
                                               const int32_t *__restrict__ tok,
                                               float *__restrict__ X, int x_stride) {
    const int t = blockIdx.y;
    const int row = tok[t], i = row & 3, nsb = cols >> 8;
    for (int c = blockIdx.x * 256 + threadIdx.x; c < cols; c += gridDim.x * 256) {
        const int sb = c >> 8, k = (c & 255) >> 5, j = c & 31;
        const uint8_t *p = W + ((size_t)(row >> 2) * nsb + sb) * 576;
        const float D = nmx_half(p + 2 * i), M = nmx_half(p + 8 + 2 * i);
        const float dd = D * (float)nmx_get6(p + 16, 4 * k + i);
        const float mm = M * (float)nmx_get6(p + 40, 4 * k + i);
        const uint8_t byte = p[64 + 64 * k + 16 * i + (j & 15)];
        const int u = j < 16 ? (byte & 15) : (byte >> 4);
        X[(size_t)t * x_stride + c] = dd * (float)u - mm;
    }
}

/* ---- RMSNorm of rows (engine/src/forward_ops.c:191-200): optional residual add first
 * (x += add, written back, forward.c pf_add_rows), r = 1 / sqrtf(sumsq / cols + eps),
 * y = (x * r) * w; optional A8 of y for the next matmul. One workgroup per row; every global
 * load of the row (x, add, w) is issued before the first use, PER values per thread. */
template <int PER>
__global__ __launch_bounds__(256) void rmsnorm_k(const float *x, int x_stride,
                                                 const float *add, int add_stride,
                                                 float *xo, int xo_stride,
                                                 const float *__restrict__ w, int cols, float eps,
                                                 float *__restrict__ y, int y_stride,
                                                 int8_t *__restrict__ q, float *__restrict__ d,
                                                 float *__restrict__ fs, int n) {
    extern __shared__ float sq[]; /* chain-major squares */
    __shared__ float red[8];
    const int row = blockIdx.x, tid = threadIdx.x;
    const int m4 = cols >> 2, s4 = cm_stride(cols);
    const float *xr = x + (size_t)row * x_stride;
    float v[PER], wv[PER];
    /* clamped (always in-bounds, branch-free) loads; values past cols are masked below */
#pragma unroll
    for (int u = 0; u < PER; u++) {
        const int i = tid + 256 * u;
        v[u] = xr[i < cols ? i : cols - 1];
        wv[u] = w[i < cols ? i : cols - 1];
    }
    if (add) {
        float av[PER];
#pragma unroll
        for (int u = 0; u < PER; u++) {
            const int i = tid + 256 * u;
            av[u] = add[(size_t)row * add_stride + (i < cols ? i : cols - 1)];
        }
#pragma unroll
        for (int u = 0; u < PER; u++) v[u] = v[u] + av[u];
    }
    if (xo) {
#pragma unroll
        for (int u = 0; u < PER; u++) {
            const int i = tid + 256 * u;
            if (i < cols) xo[(size_t)row * xo_stride + i] = v[u];
        }
    }
#pragma unroll
    for (int u = 0; u < PER; u++) {
        const int i = tid + 256 * u;
        if (i < cols) sq[i < 4 * m4 ? (i & 3) * s4 + (i >> 2) : 4 * s4 + (i - 4 * m4)] = v[u] * v[u];
    }
    __syncthreads();
    const float ss = ordered_sum4_cm(sq, cols, s4, red);
    const float r = 1.0f / sqrtf(ss / (float)cols + eps);
#pragma unroll
    for (int u = 0; u < PER; u++) {
        const int i = tid + 256 * u;
        const bool live = i < cols;
        const float o = live ? (v[u] * r) * wv[u] : 0.0f;
        if (live && y) y[(size_t)row * y_stride + i] = o;
        if (q && 256 * u + (tid & ~31) < cols) a8_block(o, i >> 5, row, n, q, d, fs);
    }
}

template <int P4>
__global__ __launch_bounds__(256) void rmsnorm4_k(const float *x, int x_stride,
                                                  const float *add, int add_stride,
                                                  float *xo, int xo_stride,
                                                  const float *__restrict__ w, int cols, float eps,
                                                  float *__restrict__ y, int y_stride,
                                                  int8_t *__restrict__ q, float *__restrict__ d,
                                                  float *__restrict__ fs, int n) {
    extern __shared__ float sq[]; /* chain-major squares */
    __shared__ float red[8];
    rms4_row<P4>(x, x_stride, add, add_stride, xo, xo_stride, w, cols, eps, y, y_stride, q, d, fs,
                 n, blockIdx.x, sq, red);
}

/* One row chosen on the device (row *idx + off of x, + add, clamped to [0, nrows)) into
 * row 0 of y and of a one-vector A8 layout. */
template <int P4>
__global__ __launch_bounds__(256) void rmsnorm4_row_k(const float *x, int x_stride,
                                                      const float *add, int add_stride,
                                                      const float *__restrict__ w, int cols,
                                                      float eps, const int32_t *idx, int off,
                                                      int nrows, float *__restrict__ y,
                                                      int8_t *__restrict__ q,
                                                      float *__restrict__ d,
                                                      float *__restrict__ fs) {
    extern __shared__ float sq[];
    __shared__ float red[8];
    const int ri = *idx + off;
    const size_t r = (size_t)(ri < 0 ? 0 : ri >= nrows ? nrows - 1 : ri);
    rms4_row<P4>(x + r * x_stride, 0, add ? add + r * add_stride : nullptr, 0, nullptr, 0, w, cols,
                 eps, y, 0, q, d, fs, 1, 0, sq, red);
}

/* Two independent norms of n rows each in one launch (blockIdx.y picks the set). */
struct RmsSet {
    const float *x;
    int x_stride;
    const float *w;
    float *y;
    int y_stride;
    int8_t *q;
    float *d, *fs;
    const uint8_t *E;     /* optional: rows from the Q4K embedding E (rows tok[]) instead of x */
    const int32_t *tok;
    float *xo;            /* optional: the rows (as read or decoded) written here */
    int xo_stride;
    const unsigned long long *keys; /* optional, with E: row n - 1's token is the argmax of */
    int nkeys;                      /* these partial keys, written to tok_w[n - 1] */
    int32_t *tok_w;
};

template <int P4>
__global__ __launch_bounds__(256) void rmsnorm4_pair_k(RmsSet s0, RmsSet s1, int cols, float eps,
                                                       int n) {
    extern __shared__ float sq[];
    __shared__ float red[8];
    const RmsSet &s = blockIdx.y ? s1 : s0;
    const int row = blockIdx.x;
    if (s.keys && row == n - 1) { /* uniform: the token from the keys, by every wave */
        float4 v[P4], a[P4], wv[P4];
        rms4_load_w<P4>(s.w, cols, wv); /* before the keys the row waits for */
        const int tk = nmx_keys_token(s.keys, s.nkeys);
        if (threadIdx.x == 0) s.tok_w[row] = tk;
        rms4_load<P4, true>(nullptr, nullptr, s.w, cols, v, a, wv, s.E, tk);
        rms4_finish<P4>(v, a, wv, false, s.xo ? s.xo + (size_t)row * s.xo_stride : nullptr, cols,
                        eps, s.y ? s.y + (size_t)row * s.y_stride : nullptr, s.q, s.d, s.fs, n,
                        row, sq, red);
        return;
    }
    rms4_row<P4>(s.x, s.x_stride, nullptr, 0, s.xo, s.xo_stride, s.w, cols, eps, s.y, s.y_stride,
                 s.q, s.d, s.fs, n, row, sq, red, s.E, s.tok);
}

/* ---- Gated DeltaNet pre (engine/src/forward_lin.c:36-67): per channel the causal conv over
 * [state rows, tokens] in tap order, SiLU (forward_ops.c:237-260); q / k heads L2-normalised
 * (eps 1e-6) with q scaled by 1/sqrt(dk) (forward_ops.c:204-212). Logged pass: the live
 * state advances by token 0 only and the raw inputs of tokens 1.. go to xin. One workgroup
 * per group of dk channels (a q or k head, or a slice of v); the last workgroup computes the
 * gates beta = sigmoid(b), decay = exp(A softplus(a + dt_bias)) with A = -exp(A_log). */
struct LinPre {
    int n, C, K, dk, kd;     /* tokens, conv channels, conv taps, head dim, q (= k) width */
    const float *raw;        /* [n][raw_stride] in_proj_qkv output */
    int raw_stride;
    float *out;              /* [n][C] conv + SiLU (+ L2 norm) */
    float *state;            /* [K-1][C] */
    const float *conv_w;     /* [C][K] */
    float *xin;              /* [n][C] raw inputs of tokens 1.. (logged) or NULL */
    float qscale, l2eps;
    const float *b_in, *a_in;/* [n][g_stride] */
    int g_stride, heads;
    const float *A_log, *A, *dt_bias;
    float *beta, *decay;     /* [n][heads] */
};

constexpr int PRE_TB = 8; /* tokens per batch: their loads issued together, norms in parallel */

__global__ __launch_bounds__(256) void lin_pre_k(LinPre a) {
    extern __shared__ float sq[]; /* [PRE_TB][dk] squares */
    __shared__ float red[4 * PRE_TB];
    const int ngroups = (a.C + a.dk - 1) / a.dk;
    const int tid = threadIdx.x;
    if ((int)blockIdx.x == ngroups) { /* gates */
        for (int u = tid; u < a.n * a.heads; u += blockDim.x) {
            const int t = u / a.heads, h = u - t * a.heads;
            const float b = a.b_in[(size_t)t * a.g_stride + h];
            const float av = a.a_in[(size_t)t * a.g_stride + h];
            a.beta[u] = 1.0f / (1.0f + nmx_gate_expf(-b));
            const float A = a.A ? a.A[h] : -nmx_gate_expf(a.A_log[h]);
            float sp = av + a.dt_bias[h];
            sp = sp > 20.0f ? sp : nmx_gate_log1pf(nmx_gate_expf(sp));
            a.decay[u] = nmx_gate_expf(A * sp);
        }
        return;
    }
    const int ch = blockIdx.x * a.dk + tid;
    const bool live = tid < a.dk && ch < a.C;
    const int S = a.K - 1;
    const int cc = live ? ch : 0;
    float win[8], wc[8];
#pragma unroll
    for (int r = 0; r < 8; r++) {
        win[r] = (r < S) ? a.state[(size_t)r * a.C + cc] : 0.0f;
        wc[r] = (r < a.K) ? a.conv_w[(size_t)cc * a.K + r] : 0.0f;
    }
    const bool norm = blockIdx.x * a.dk < 2 * a.kd;  /* a q or k head */
    const float scale = blockIdx.x * a.dk < a.kd ? a.qscale : 1.0f;
    const int m4 = a.dk >> 2;
    for (int t0 = 0; t0 < a.n; t0 += PRE_TB) {
        const int nb = a.n - t0 < PRE_TB ? a.n - t0 : PRE_TB;
        float xt[PRE_TB], yv[PRE_TB];
#pragma unroll
        for (int u = 0; u < PRE_TB; u++)
            xt[u] = u < nb ? a.raw[(size_t)(t0 + u) * a.raw_stride + cc] : 0.0f;
#pragma unroll
        for (int u = 0; u < PRE_TB; u++) {
            yv[u] = 0.0f;
            if (u >= nb) continue;
            const int t = t0 + u;
            /* taps in order over [state rows (oldest first), x_t] */
            float acc = wc[0] * (S > 0 ? win[0] : xt[u]);
#pragma unroll
            for (int j = 1; j < 8; j++)
                if (j < a.K) acc = acc + wc[j] * (j < S ? win[j] : xt[u]);
            /* shift the window: it now ends with x_t */
#pragma unroll
            for (int j = 0; j < 7; j++)
                if (j + 1 < S) win[j] = win[j + 1];
#pragma unroll
            for (int j = 0; j < 8; j++)
                if (j == S - 1) win[j] = xt[u];
            if (t == 0 && a.xin && live) {  /* logged pass: token 0 is committed in place */
#pragma unroll
                for (int j = 0; j < 8; j++)
                    if (j < S) a.state[(size_t)j * a.C + ch] = win[j];
            }
            if (t > 0 && a.xin && live) a.xin[(size_t)t * a.C + ch] = xt[u];
            yv[u] = nmx_silu(acc);
        }
        if (norm) { /* L2 norm per token (forward_ops.c:204-212): chains of 4 per token */
            __syncthreads(); /* the previous batch's reads of sq are done */
#pragma unroll
            for (int u = 0; u < PRE_TB; u++)
                if (u < nb && tid < a.dk) sq[u * a.dk + tid] = live ? yv[u] * yv[u] : 0.0f;
            __syncthreads();
            if (tid < 4 * nb) {
                const float *v = sq + (tid >> 2) * a.dk + (tid & 3);
                float c = 0.0f;
                int m = 0;
                for (; m + 16 <= m4; m += 16) {
                    float b[16];
#pragma unroll
                    for (int k = 0; k < 16; k++) b[k] = v[4 * (m + k)];
#pragma unroll
                    for (int k = 0; k < 16; k++) c = c + b[k];
                }
                for (; m < m4; m++) c = c + v[4 * m];
                red[tid] = c;
            }
            __syncthreads();
#pragma unroll
            for (int u = 0; u < PRE_TB; u++) {
                if (u >= nb) continue;
                const float ss = ((red[4 * u] + red[4 * u + 1]) + (red[4 * u + 2] + red[4 * u + 3])) + 0.0f;
                const float r = 1.0f / sqrtf(ss + a.l2eps);
                yv[u] = (yv[u] * r) * scale;
            }
        }
#pragma unroll
        for (int u = 0; u < PRE_TB; u++)
            if (u < nb && live) a.out[(size_t)(t0 + u) * a.C + ch] = yv[u];
    }
    if (!a.xin && live) {
#pragma unroll
        for (int j = 0; j < 8; j++)
            if (j < S) a.state[(size_t)j * a.C + ch] = win[j];
    }
}

/* ---- Gated RMSNorm (engine/src/forward_lin.c:70-81): per (token, head) y = rmsnorm(o) * w,
 * then y *= silu(z); optional A8 of the row for out_proj. One workgroup of dv threads. */
__global__ __launch_bounds__(512) void lin_post_k(const float *__restrict__ o, int o_stride,
                                                  const float *__restrict__ z, int z_stride,
                                                  const float *__restrict__ w, int dv, float eps,
                                                  float *__restrict__ y, int y_stride,
                                                  int8_t *__restrict__ q, float *__restrict__ d,
                                                  float *__restrict__ fs, int n) {
    extern __shared__ float sq[];
    __shared__ float red[8];
    const int t = blockIdx.y, h = blockIdx.x, j = threadIdx.x;
    const float ov = o[(size_t)t * o_stride + h * dv + j];
    sq[j] = ov * ov;
    __syncthreads();
    const float ss = ordered_sum4(sq, dv, red);
    const float r = 1.0f / sqrtf(ss / (float)dv + eps);
    float v = (ov * r) * w[j];
    v = v * nmx_silu(z[(size_t)t * z_stride + h * dv + j]);
    const int col = h * dv + j;
    if (y) y[(size_t)t * y_stride + col] = v;
    if (q) a8_block(v, col >> 5, t, n, q, d, fs);
}

/* ---- SwiGLU activation (engine/src/forward_ops.c:98-110): g = silu(gate) * up, + A8. */
__global__ __launch_bounds__(256) void silu_mul_k(const float *__restrict__ gate,
                                                  const float *__restrict__ up, int stride,
                                                  int cols, float *__restrict__ y,
                                                  int8_t *__restrict__ q, float *__restrict__ d,
                                                  float *__restrict__ fs, int n) {
    const int t = blockIdx.y, c = blockIdx.x * 256 + threadIdx.x;
    const bool live = c < cols;
    const size_t i = (size_t)t * stride + (live ? c : 0);
    const float v = live ? nmx_silu(gate[i]) * up[i] : 0.0f;
    if (y && live) y[(size_t)t * cols + c] = v;
    if (q && blockIdx.x * 256 + (threadIdx.x & ~31) < cols) a8_block(v, c >> 5, t, n, q, d, fs);
}

/* ---- gated full attention ---------------------------------------------------------------
 * attn_prep (engine/src/forward_attn.c:246-260): per token, every KV group: k row RMSNorm +
 * RoPE, K and V rows stored at position pos + t; every query head: RMSNorm + RoPE in place.
 * RoPE (forward_ops.c:149-165): pairs (i, i + rot/2), v_i = a c - b s, v_{i+h} = b c + a s. */
struct Attn {
    int n, nh, nkv, hd, rot, max_ctx;
    float *q;            /* [n][nh][2 hd]: query | gate per head */
    const float *k_in, *v_in; /* [n][nkv hd] */
    const float *q_norm, *k_norm;
    float eps, scale;
    const float *rcos, *rsin;  /* [max_ctx][rot/2] */
    void *kc, *vc;       /* KV caches of the launch's format (nmx_kv_bytes each) */
    const int32_t *pos;  /* device: position of token 0 is *pos + pos_off */
    int pos_off;
    float *o;            /* [n][nh hd] */
    int8_t *aq;
    float *ad, *afs;
};

/* ---- KV cache formats (engine/src/forward_kv.c:28-188): row R = g max_ctx + p of a cache
 * holds hd values as fp32, binary16, or int8 with an fp32 scale in a [nkv][max_ctx] array
 * after the rows. */
enum { KV_F32 = 0, KV_F16 = 1, KV_I8 = 2 };

/* binary16 bits of x rounded to nearest even, subnormals kept (v_cvt_f16_f32); a NaN becomes
 * the quiet NaN with x's sign and top 10 payload bits (forward_kv.c:28-48 f32_to_f16) */
__device__ __forceinline__ uint32_t kv_half_bits(float x) {
    const uint32_t u = __float_as_uint(x);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu))
        return ((u >> 16) & 0x8000u) | 0x7e00u | ((u & 0x7fffffu) >> 13);
    const _Float16 h = (_Float16)x;
    unsigned short b;
    __builtin_memcpy(&b, &h, 2);
    return b;
}

__device__ __forceinline__ float kv_half_value(uint32_t bits16) { /* exact widening */
    const unsigned short b = (unsigned short)bits16;
    _Float16 h;
    __builtin_memcpy(&h, &b, 2);
    return (float)h;
}

/* the int8 code of x at inv = 127 / amax (or 0): round half even, clamped to +-127, NaN to 0
 * (forward_kv.c:101-124) */
__device__ __forceinline__ uint32_t kv_i8_code(float x, float inv) {
    const float y = rintf(x * inv);
    const int q = y > 127.0f ? 127 : y < -127.0f ? -127 : y == y ? (int)y : 0;
    return (uint32_t)(uint8_t)(int8_t)q;
}

/* fp32 values of columns col .. col + 3 of cache row R (col % 4 == 0) */
template <int KVT>
__device__ __forceinline__ float4 kv_load4(const void *cache, size_t R, int hd, int col,
                                           const float *scales) {
    if constexpr (KVT == KV_F32) {
        return *(const float4 *)((const float *)cache + R * hd + col);
    } else if constexpr (KVT == KV_F16) {
        const uint2 h = *(const uint2 *)((const unsigned short *)cache + R * hd + col);
        return make_float4(kv_half_value(h.x), kv_half_value(h.x >> 16), kv_half_value(h.y),
                           kv_half_value(h.y >> 16));
    } else {
        const uint32_t w = *(const uint32_t *)((const int8_t *)cache + R * hd + col);
        const float sc = scales[R];
        return make_float4((float)(int8_t)w * sc, (float)(int8_t)(w >> 8) * sc,
                           (float)(int8_t)(w >> 16) * sc, (float)(int8_t)(w >> 24) * sc);
    }
}

template <int KVT>
__device__ __forceinline__ const float *kv_scales(const void *cache, const Attn &a) {
    return KVT == KV_I8 ? (const float *)((const int8_t *)cache + (size_t)a.nkv * a.max_ctx * a.hd)
                        : nullptr;
}

/* Store one row element per thread (thread i of the row's hd); the int8 format first reduces
 * the row's max |x| over the workgroup (hd threads, exact in any order). */
template <int KVT>
__device__ __forceinline__ void kv_store(void *cache, const Attn &a, size_t R, int i, float x,
                                         float *red) {
    const int hd = a.hd;
    if constexpr (KVT == KV_F32) {
        ((float *)cache)[R * hd + i] = x;
    } else if constexpr (KVT == KV_F16) {
        ((unsigned short *)cache)[R * hd + i] = (unsigned short)kv_half_bits(x);
    } else {
        float m = fabsf(x);
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
        __syncthreads(); /* red free */
        if ((i & 63) == 0) red[i >> 6] = m;
        __syncthreads();
        float amax = 0.0f;
        for (int w = 0; w < (hd >> 6); w++) amax = fmaxf(amax, red[w]);
        /* inv stays finite: a row of subnormals codes to zeros like a zero row */
        const float inv = amax > 127.0f / 3.40282347e+38f ? 127.0f / amax : 0.0f;
        ((int8_t *)cache)[R * hd + i] = (int8_t)kv_i8_code(x, inv);
        if (i == 0) ((float *)((int8_t *)cache + (size_t)a.nkv * a.max_ctx * hd))[R] = amax / 127.0f;
    }
}

template <int KVT>
__global__ __launch_bounds__(512) void attn_prep_k(Attn a) {
    extern __shared__ float sq[];
    __shared__ float buf[1024];
    __shared__ float red[8];
    const int t = blockIdx.y, u = blockIdx.x, i = threadIdx.x, hd = a.hd, h2 = a.rot / 2;
    const int p = *a.pos + a.pos_off + t;
    const bool is_k = u < a.nkv;
    float v;
    if (is_k) v = a.k_in[(size_t)t * a.nkv * hd + u * hd + i];
    else v = a.q[((size_t)t * a.nh + (u - a.nkv)) * 2 * hd + i];
    sq[i] = v * v;
    __syncthreads();
    const float ss = ordered_sum4(sq, hd, red);
    const float r = 1.0f / sqrtf(ss / (float)hd + a.eps);
    v = (v * r) * (is_k ? a.k_norm[i] : a.q_norm[i]);
    buf[i] = v;
    __syncthreads();
    if (i < h2) {
        const float c = a.rcos[(size_t)p * h2 + i], s = a.rsin[(size_t)p * h2 + i];
        const float x0 = buf[i], x1 = buf[i + h2];
        v = x0 * c - x1 * s;
    } else if (i < 2 * h2) {
        const float c = a.rcos[(size_t)p * h2 + i - h2], s = a.rsin[(size_t)p * h2 + i - h2];
        const float x0 = buf[i - h2], x1 = buf[i];
        v = x1 * c + x0 * s;
    }
    if (is_k) { /* uniform per workgroup */
        const size_t R = (size_t)u * a.max_ctx + p;
        kv_store<KVT>(a.kc, a, R, i, v, red);
        kv_store<KVT>(a.vc, a, R, i, a.v_in[(size_t)t * a.nkv * hd + u * hd + i], red);
    } else {
        a.q[((size_t)t * a.nh + (u - a.nkv)) * 2 * hd + i] = v;
    }
}

/* Scores (engine/src/forward_kv.c:281-303, pf_dot forward_ops.c:265-287): for every query
 * head h of KV group g and position p <= pos(t), s = (pf_dot(q_h, k_p) + 0) * scale, where
 * pf_dot keeps 16 interleaved partial sums c_l over elements i = l (mod 16) in i order and
 * combines h_k = (c_4k + c_4k+1) + (c_4k+2 + c_4k+3), s = (h_0 + h_1) + (h_2 + h_3) (hd is a
 * multiple of 16: no tail). Workgroup = (chunk of CP positions, token t, group g): the K rows
 * of the chunk are staged in LDS (row stride hd + 4 floats, so lanes reading different rows
 * hit different banks); lane = position (lane % CP) x part (lane / CP) of the 16 partial
 * sums, the parts combined in the tree order by two cross-lane exchanges; wave w takes the
 * group's query heads w, w + 4, ... */
template <int CP, int KVT>
__global__ __launch_bounds__(256) void attn_score_k(Attn a, float *__restrict__ sc) {
    constexpr int LP = 64 / CP, CPL = 16 / LP; /* lanes per position, partial sums per lane */
    extern __shared__ float4 smem4[];
    const int hd = a.hd, rep = a.nh / a.nkv, rs = hd + 4;
    const int t = blockIdx.y, g = blockIdx.z, p0 = blockIdx.x * CP;
    const int f4 = hd >> 2;
    /* the first 4 query heads of the group, requested before the position is known (the K
     * rows' addresses wait for it); staged into LDS once the K rows are */
    float4 qa[2];
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int f = u * 256 + threadIdx.x, hh = f / f4, c4 = f - hh * f4;
        qa[u] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (f < 4 * f4 && hh < rep)
            qa[u] = ((const float4 *)(a.q + ((size_t)t * a.nh + g * rep + hh) * 2 * hd))[c4];
    }
    const int np = *a.pos + a.pos_off + t + 1;
    if (p0 >= np) return;
    const int rows = np - p0 < CP ? np - p0 : CP;
    float *ks = (float *)smem4;   /* [CP][rs] */
    float *qs = ks + CP * rs;     /* [4][hd] */
    const size_t R0 = (size_t)g * a.max_ctx + p0;
    const float *ksc = kv_scales<KVT>(a.kc, a);
    for (int f0 = 0; f0 < rows * f4; f0 += 4 * 256) {
        float4 b[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int f = f0 + u * 256 + threadIdx.x;
            b[u] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (f < rows * f4) b[u] = kv_load4<KVT>(a.kc, R0 + f / f4, hd, 4 * (f % f4), ksc);
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int f = f0 + u * 256 + threadIdx.x;
            if (f < rows * f4) {
                const int r = f / f4, c4 = f - r * f4;
                *(float4 *)(ks + r * rs + 4 * c4) = b[u];
            }
        }
    }
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int pl = lane % CP, lp = lane / CP;
    const bool live = pl < rows;
    const float *kr = ks + (live ? pl : 0) * rs + CPL * lp;
    for (int hb = 0; hb < rep; hb += 4) {
        __syncthreads(); /* K staged; previous heads' qs reads done */
        if (hb == 0) {
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const int f = u * 256 + threadIdx.x, hh = f / f4, c4 = f - hh * f4;
                if (f < 4 * f4 && hh < rep) *(float4 *)(qs + hh * hd + 4 * c4) = qa[u];
            }
        } else {
            for (int f = threadIdx.x; f < 4 * f4; f += 256) {
                const int hh = f / f4, c4 = f - hh * f4;
                if (hb + hh < rep)
                    *(float4 *)(qs + hh * hd + 4 * c4) =
                        ((const float4 *)(a.q + ((size_t)t * a.nh + g * rep + hb + hh) * 2 * hd))[c4];
            }
        }
        __syncthreads();
        const int h = hb + w;
        if (h >= rep) continue; /* uniform per wave */
        const float *qr = qs + w * hd + CPL * lp;
        float c[CPL];
#pragma unroll
        for (int j = 0; j < CPL; j++) c[j] = 0.0f;
        for (int i = 0; i < hd; i += 16) {
#pragma unroll
            for (int j = 0; j < CPL; j += 4) {
                const float4 kv = *(const float4 *)(kr + i + j);
                const float4 qv = *(const float4 *)(qr + i + j);
                c[j] = c[j] + qv.x * kv.x;
                c[j + 1] = c[j + 1] + qv.y * kv.y;
                c[j + 2] = c[j + 2] + qv.z * kv.z;
                c[j + 3] = c[j + 3] + qv.w * kv.w;
            }
        }
        float x;
        if constexpr (LP == 2) { /* chains 8 lp .. 8 lp + 7: x = h_2lp + h_2lp+1 */
            x = ((c[0] + c[1]) + (c[2] + c[3])) + ((c[4] + c[5]) + (c[6] + c[7]));
        } else {                 /* chains 4 lp .. 4 lp + 3: x = h_lp, then (h0 + h1), (h2 + h3) */
            x = (c[0] + c[1]) + (c[2] + c[3]);
            x = x + __shfl_xor(x, 16);
        }
        const float s = x + __shfl_xor(x, 32);
        if (lp == 0 && live)
            sc[((size_t)t * a.nh + g * rep + h) * a.max_ctx + p0 + pl] = (s + 0.0f) * a.scale;
    }
}

/* acc += x[0] + ... + x[n-1] in order, x[i] = p[i * stride] in LDS, with the reads of 3
 * batches of 8 in flight ahead of the adds (at most 16 LDS reads outstanding). Each batch is
 * four register pairs: two reads of one pair merge into one ds_read2 that lands in the pair
 * itself, so the loop-carried batches need no register copies (with scalar batches the
 * merged reads landed in fresh registers and were copied at the loop's end, which waited for
 * every read in flight). The scheduling barriers keep each batch's reads where they are
 * issued: left alone, the scheduler sinks them to just before their adds. */
__device__ __forceinline__ void pv_load8(float2 (&X)[4], const float *p, int stride, int r) {
#pragma unroll
    for (int u = 0; u < 4; u++) X[u] = make_float2(p[(r + 2 * u) * stride], p[(r + 2 * u + 1) * stride]);
}

__device__ __forceinline__ float pv_add8(float acc, const float2 (&X)[4]) {
#pragma unroll
    for (int u = 0; u < 4; u++) {
        acc = acc + X[u].x;
        acc = acc + X[u].y;
    }
    return acc;
}

__device__ __forceinline__ float pv_chain(float acc, const float *p, int stride, int n) {
    int r = 0;
    if (n >= 32) {
        float2 A[4], B[4], C[4], D[4];
        pv_load8(A, p, stride, 0);
        pv_load8(B, p, stride, 8);
        pv_load8(C, p, stride, 16);
        for (; r + 32 <= n; r += 32) {
            /* A, B, C = rows r .. r+23 loaded; reads past n are clamped (not used) */
            const int d0 = r + 24, a0 = r + 40 <= n ? r + 32 : r, b0 = r + 48 <= n ? r + 40 : r,
                      c0 = r + 56 <= n ? r + 48 : r;
            pv_load8(D, p, stride, d0);
            __builtin_amdgcn_sched_barrier(0);
            acc = pv_add8(acc, A);
            pv_load8(A, p, stride, a0);
            __builtin_amdgcn_sched_barrier(0);
            acc = pv_add8(acc, B);
            pv_load8(B, p, stride, b0);
            __builtin_amdgcn_sched_barrier(0);
            acc = pv_add8(acc, C);
            pv_load8(C, p, stride, c0);
            __builtin_amdgcn_sched_barrier(0);
            acc = pv_add8(acc, D);
        }
        /* A, B, C hold r .. r+23 when those are in range */
        if (r + 8 <= n) {
            acc = pv_add8(acc, A);
            r += 8;
            if (r + 8 <= n) {
                acc = pv_add8(acc, B);
                r += 8;
                if (r + 8 <= n) {
                    acc = pv_add8(acc, C);
                    r += 8;
                }
            }
        }
    }
    for (; r < n; r++) acc = acc + p[r * stride];
    return acc;
}

/* acc += x[0] + ... + x[n-1] in order, x contiguous in LDS and 16-byte aligned: the terms
 * arrive four per ds_read_b128 with immediate offsets, two sets of 32 taking turns (the next
 * set requested before the current one is added), so the chain's wave issues about 0.3 other
 * instructions per dependent add (pv_chain, strided, about 1.3). */
__device__ __forceinline__ float pv_chain4(float acc, const float *x, int n) {
    auto fetch = [&](float4 (&b)[8], int r0) {
#pragma unroll
        for (int u = 0; u < 8; u++) b[u] = *(const float4 *)(x + r0 + 4 * u);
    };
    auto add = [&](const float4 (&b)[8]) {
#pragma unroll
        for (int u = 0; u < 8; u++) {
            acc = acc + b[u].x;
            acc = acc + b[u].y;
            acc = acc + b[u].z;
            acc = acc + b[u].w;
        }
    };
    int r = 0;
    if (n >= 32) {
        float4 ba[8], bb[8];
        fetch(ba, 0);
        for (; r + 64 <= n; r += 64) {
            __builtin_amdgcn_sched_barrier(0);
            fetch(bb, r + 32);
            __builtin_amdgcn_sched_barrier(0);
            add(ba);
            __builtin_amdgcn_sched_barrier(0);
            fetch(ba, r + 96 <= n ? r + 64 : r); /* clamped: not used past n */
            __builtin_amdgcn_sched_barrier(0);
            add(bb);
        }
        __builtin_amdgcn_sched_barrier(0);
        if (r + 32 <= n) { /* ba holds terms r .. r + 31 */
            add(ba);
            r += 32;
        }
    }
    for (; r + 4 <= n; r += 4) {
        const float4 v = *(const float4 *)(x + r);
        acc = acc + v.x;
        acc = acc + v.y;
        acc = acc + v.z;
        acc = acc + v.w;
    }
    for (; r < n; r++) acc = acc + x[r];
    return acc;
}

/* attn_prep_k and attn_score_k in one launch (nmx_attn_fused), for hd = 256 (a thread per
 * element of a row) and at most 4 query heads per KV group. Each workgroup (chunk of CP
 * positions, token t, group g) normalises and rotates the group's query heads of token t
 * itself, and the keys of the pass's new positions in its chunk (tokens t' <= t), with the
 * operations of attn_prep_k; the keys are rounded to the cache format and back, so each score
 * equals the one read from the cache. The workgroup whose chunk holds token t's own position
 * stores that K row and the V row (each (token, group) once; later passes and the P.V launch
 * read them). The rotated queries are not written back: only the scores use them.
 * Every global read of a workgroup (the queries, the chunk's cache rows, the new keys, the
 * value row, both norm weights and the RoPE coefficients) is issued at entry, so they share
 * one memory latency; the threads that hold an element write its square to LDS, and each row's
 * four chains of the norm only add (pv_chain: reads batched ahead of the adds). */
constexpr int QK_HD = 256;
constexpr int QK_NMAX = 8; /* tokens per pass: new key rows of a chunk */

/* max |x| of a row of QK_HD values, one per thread, exact in any order */
__device__ __forceinline__ float qk_row_amax(float x, float *amx, int slot) {
    float m = fabsf(x);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    if ((threadIdx.x & 63) == 0) amx[slot * 4 + (threadIdx.x >> 6)] = m;
    return m;
}

template <int CP, int KVT>
__global__ __launch_bounds__(256) void attn_qk_k(const float *__restrict__ q_in,
                                                 const int32_t *__restrict__ posp,
                                                 const float *__restrict__ k_in,
                                                 const float *__restrict__ v_in, void *kc,
                                                 int nh, int nkv, int pos_off, int max_ctx,
                                                 Attn a, float *__restrict__ sc) {
    constexpr int HD = QK_HD, LP = 64 / CP, CPL = 16 / LP, RS = HD + 4, F4 = HD / 4,
                  OLD4 = CP * F4 / 256; /* float4 reads of cache rows per thread */
    static_assert(CP * F4 % 256 == 0 && HD / 4 <= 256, "attn_qk_k tiling");
    extern __shared__ float4 smem4[];
    __shared__ float part[(4 + QK_NMAX) * 4]; /* partial sums of squares, 4 per row */
    __shared__ float rn[4 + QK_NMAX];         /* 1 / rms of each row */
    __shared__ float amx[(CP + 1) * 4];       /* int8 cache: per (row, wave) max |x| */
    const int i = threadIdx.x, lane = i & 63, w = i >> 6;
    const int rep = nh / nkv, h2 = a.rot / 2;
    const int t = blockIdx.y, g = blockIdx.z, p0 = blockIdx.x * CP;
    float *ks = (float *)smem4; /* [CP][RS] key rows of the chunk, as the cache gives them */
    float *qs = ks + CP * RS;   /* [4][HD] rotated queries */
    float *qw = qs + 4 * HD;    /* [4][HD] squares, then normalised queries */
    float *kw = qw + 4 * HD;    /* [QK_NMAX][HD] squares, then normalised new keys */
    /* the queries and norm weights first (their addresses do not wait for the position) */
    float qv[4];
#pragma unroll
    for (int hh = 0; hh < 4; hh++)
        qv[hh] = hh < rep ? q_in[((size_t)t * nh + g * rep + hh) * 2 * HD + i] : 0.0f;
    const float qn = a.q_norm[i], kn = a.k_norm[i];
    const int pos0 = *posp + pos_off; /* position of token 0 */
    const int np = pos0 + t + 1;
    if (p0 >= np) return;
    const int rows = np - p0 < CP ? np - p0 : CP;
    const int nold = pos0 - p0 <= 0 ? 0 : pos0 - p0 < rows ? pos0 - p0 : rows;
    const int nnew = rows - nold; /* <= t + 1 <= QK_NMAX (the launch's limit) */
    const bool own = np - p0 <= CP; /* token t's own position is row rows - 1 of the chunk */
    const size_t R0 = (size_t)g * max_ctx + p0;
    const float *ksc = kv_scales<KVT>(kc, a);
    /* new keys (row nold + u of the chunk is token p0 + nold + u - pos0) and, for the own
     * row, the values: raw inputs */
    float knw[QK_NMAX];
#pragma unroll
    for (int u = 0; u < QK_NMAX; u++)
        knw[u] = u < nnew ? k_in[(size_t)(p0 + nold + u - pos0) * nkv * HD + g * HD + i] : 0.0f;
    const float vv = own ? v_in[(size_t)t * nkv * HD + g * HD + i] : 0.0f;
    /* the old rows from the cache (element f: float4 f % F4 of row f / F4) */
    float4 b[OLD4];
#pragma unroll
    for (int u = 0; u < OLD4; u++) {
        const int f = u * 256 + i;
        b[u] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (f < nold * F4) b[u] = kv_load4<KVT>(kc, R0 + f / F4, HD, 4 * (f % F4), ksc);
    }
    /* RoPE coefficients of element i at the query's and each new key's position: element
     * i < h2 pairs with i + h2, element h2 <= i < 2 h2 with i - h2; both use index i mod h2 */
    const bool rot = i < 2 * h2;
    const int ri = i < h2 ? i : i - h2;
    float qc = 0.0f, qsn = 0.0f, kcs[QK_NMAX], ksn[QK_NMAX];
    if (rot) {
        qc = a.rcos[(size_t)(pos0 + t) * h2 + ri];
        qsn = a.rsin[(size_t)(pos0 + t) * h2 + ri];
    }
#pragma unroll
    for (int u = 0; u < QK_NMAX; u++) {
        kcs[u] = 0.0f, ksn[u] = 0.0f;
        if (rot && u < nnew) {
            kcs[u] = a.rcos[(size_t)(p0 + nold + u) * h2 + ri];
            ksn[u] = a.rsin[(size_t)(p0 + nold + u) * h2 + ri];
        }
    }
#pragma unroll
    for (int u = 0; u < OLD4; u++) {
        const int f = u * 256 + i;
        if (f < nold * F4) {
            const int r = f / F4, c4 = f - r * F4;
            *(float4 *)(ks + r * RS + 4 * c4) = b[u];
        }
    }
#pragma unroll
    for (int hh = 0; hh < 4; hh++) qw[hh * HD + i] = qv[hh] * qv[hh];
#pragma unroll
    for (int u = 0; u < QK_NMAX; u++)
        if (u < nnew) kw[u * HD + i] = knw[u] * knw[u];
    __syncthreads();
    /* RMSNorm of every row (attn_prep_k: 4 partial sums of squares over i = l (mod 4) in i
     * order, combined (c0 + c1) + (c2 + c3), empty tail), rows 0-3 the queries, then the new
     * keys; at most 48 chains, all in wave 0 */
    if (i < (4 + nnew) * 4) {
        const int j = i >> 2, l = i & 3;
        part[i] = pv_chain(0.0f, (j < 4 ? qw + j * HD : kw + (j - 4) * HD) + l, 4, HD / 4);
    }
    __syncthreads();
    if (i < 4 + nnew) {
        const float *r4 = part + 4 * i;
        const float ss = ((r4[0] + r4[1]) + (r4[2] + r4[3])) + 0.0f;
        rn[i] = 1.0f / sqrtf(ss / (float)HD + a.eps);
    }
    __syncthreads();
#pragma unroll
    for (int hh = 0; hh < 4; hh++) qw[hh * HD + i] = (qv[hh] * rn[hh]) * qn;
#pragma unroll
    for (int u = 0; u < QK_NMAX; u++)
        if (u < nnew) kw[u * HD + i] = (knw[u] * rn[4 + u]) * kn;
    __syncthreads();
    /* RoPE over the first rot elements */
    auto rope = [&](const float *row, float c, float s) {
        if (i < h2) return row[i] * c - row[i + h2] * s;
        if (i < 2 * h2) return row[i] * c + row[i - h2] * s;
        return row[i];
    };
#pragma unroll
    for (int hh = 0; hh < 4; hh++) qs[hh * HD + i] = rope(qw + hh * HD, qc, qsn);
#pragma unroll
    for (int u = 0; u < QK_NMAX; u++)
        if (u < nnew) ks[(nold + u) * RS + i] = rope(kw + u * HD, kcs[u], ksn[u]);
    if constexpr (KVT == KV_I8) {
        /* row maxima of the new keys (and of the own row's values) for their int8 codes */
        __syncthreads(); /* the rotated keys are in ks */
        for (int r = nold; r < rows; r++) (void)qk_row_amax(ks[r * RS + i], amx, r);
        if (own) (void)qk_row_amax(vv, amx, CP);
        __syncthreads();
    }
    const size_t Rown = (size_t)g * max_ctx + (np - 1);
    for (int r = nold; r < rows; r++) {
        const float x = ks[r * RS + i];
        const bool st = own && r == rows - 1;
        if constexpr (KVT == KV_F32) {
            if (st) ((float *)kc)[Rown * HD + i] = x;
        } else if constexpr (KVT == KV_F16) {
            const uint32_t b = kv_half_bits(x);
            ks[r * RS + i] = kv_half_value(b);
            if (st) ((unsigned short *)kc)[Rown * HD + i] = (unsigned short)b;
        } else {
            float amax = 0.0f; /* kv_store's order */
#pragma unroll
            for (int ww = 0; ww < HD / 64; ww++) amax = fmaxf(amax, amx[4 * r + ww]);
            const float inv = amax > 127.0f / 3.40282347e+38f ? 127.0f / amax : 0.0f;
            const uint32_t q = kv_i8_code(x, inv);
            const float scl = amax / 127.0f;
            ks[r * RS + i] = (float)(int8_t)q * scl;
            if (st) {
                ((int8_t *)kc)[Rown * HD + i] = (int8_t)q;
                if (i == 0) ((float *)((int8_t *)kc + (size_t)nkv * max_ctx * HD))[Rown] = scl;
            }
        }
    }
    if (own) { /* the value row: stored as attn_prep_k stores it */
        if constexpr (KVT == KV_F32) {
            ((float *)a.vc)[Rown * HD + i] = vv;
        } else if constexpr (KVT == KV_F16) {
            ((unsigned short *)a.vc)[Rown * HD + i] = (unsigned short)kv_half_bits(vv);
        } else {
            float amax = 0.0f;
#pragma unroll
            for (int ww = 0; ww < HD / 64; ww++) amax = fmaxf(amax, amx[4 * CP + ww]);
            const float inv = amax > 127.0f / 3.40282347e+38f ? 127.0f / amax : 0.0f;
            ((int8_t *)a.vc)[Rown * HD + i] = (int8_t)kv_i8_code(vv, inv);
            if (i == 0) ((float *)((int8_t *)a.vc + (size_t)nkv * max_ctx * HD))[Rown] = amax / 127.0f;
        }
    }
    __syncthreads(); /* ks and qs complete */
    /* the scores, as attn_score_k (wave w takes query head w) */
    const int pl = lane % CP, lp = lane / CP;
    const bool live = pl < rows;
    const float *kr = ks + (live ? pl : 0) * RS + CPL * lp;
    if (w >= rep) return; /* uniform per wave; no barrier follows */
    const float *qr = qs + w * HD + CPL * lp;
    float c[CPL];
#pragma unroll
    for (int j = 0; j < CPL; j++) c[j] = 0.0f;
    for (int e = 0; e < HD; e += 16) {
#pragma unroll
        for (int j = 0; j < CPL; j += 4) {
            const float4 kv = *(const float4 *)(kr + e + j);
            const float4 qv4 = *(const float4 *)(qr + e + j);
            c[j] = c[j] + qv4.x * kv.x;
            c[j + 1] = c[j + 1] + qv4.y * kv.y;
            c[j + 2] = c[j + 2] + qv4.z * kv.z;
            c[j + 3] = c[j + 3] + qv4.w * kv.w;
        }
    }
    float x;
    if constexpr (LP == 2) {
        x = ((c[0] + c[1]) + (c[2] + c[3])) + ((c[4] + c[5]) + (c[6] + c[7]));
    } else {
        x = (c[0] + c[1]) + (c[2] + c[3]);
        x = x + __shfl_xor(x, 16);
    }
    const float s = x + __shfl_xor(x, 32);
    if (lp == 0 && live)
        sc[((size_t)t * nh + g * rep + w) * max_ctx + p0 + pl] = (s + 0.0f) * a.scale;
}

/* Softmax and P.V (forward_attn.c:171-181, forward_ops.c:294-382, :360-382): max (exact in
 * any order: only its value is used, and exp(x - (+-0)) agrees), e_p = exp(s_p - max) with
 * 4 partial sums + tail, w_p = e_p * (1 / sum); o[d] = sum_p w_p v_p[d] accumulated in p
 * order from zero; o *= sigmoid(gate) (forward_attn.c:217-220); + A8 of o for o_proj.
 * Workgroup = (PV_DS output dims, head h, token t). Linear workgroup i takes value slice
 * (dims, KV group) i mod S and (query head of the group, token) i / S, S = hd / PV_DS x nkv:
 * consecutive workgroups go to different XCDs (round-robin), so the workgroups reading one
 * slice share one XCD's L2. The scores row and the first PV_PT value rows are requested at
 * entry; the scores and then the exponentials sit in LDS chain-major (each partial sum's
 * terms contiguous), and each tile lands in LDS as w_p v_p[d] (the products the chain adds),
 * one row per dimension. Wave 0's lanes run the chains (one per dimension), four terms per
 * 16-byte read, the next 32 requested ahead of the adds; while wave 0 runs a tile's chains,
 * waves 1-3 load the next PV_PT2 rows. The dependent fp32 adds bound the kernel; 32 dims per
 * workgroup give twice the workgroups of 64, and a first tile of PV_PT positions keeps a
 * workgroup's LDS under half of the CU's for contexts up to 1024 positions, so two workgroups
 * share a CU and a 5-token verify pass (320 workgroups) runs in one round. */
constexpr int PV_DS = 32;           /* output dims per workgroup: one A8 block */
constexpr int PV_PT = 576;          /* positions of the first tile */
constexpr int PV_PT2 = 384;         /* positions of each later tile (loaded by waves 1-3) */
constexpr int PV_PER = PV_PT * (PV_DS / 4) / 256;    /* float4 loads per thread, first tile */
constexpr int PV_PER2 = PV_PT2 * (PV_DS / 4) / 192;  /* per thread of waves 1-3, later tiles */
/* attn_pv_k keeps a tile's products w_p v_p[d] one row per output dim (PV_DS rows of PV_RS,
 * positions contiguous): 16-byte aligned rows 4 words apart modulo 64 banks, so the chain
 * lanes' 16-byte reads are conflict-free */
constexpr int PV_RS = PV_PT + 4;

/* Chain-major index of position p of an np-position row, m4 = np / 4, s4 the row stride:
 * the terms of partial sum l = p % 4 of the ordered softmax sum contiguous, the tail after the
 * four rows. */
__device__ __forceinline__ int pv_cm(int p, int m4, int s4) {
    return p < 4 * m4 ? (p & 3) * s4 + (p >> 2) : 4 * s4 + (p - 4 * m4);
}

template <int KVT>
__global__ __launch_bounds__(256) void attn_pv_k(const float *__restrict__ sc,
                                                 const int32_t *__restrict__ posp,
                                                 const void *vc, int pos_off, int max_ctx,
                                                 int nh, int nkv, int hd_, Attn a) {
    extern __shared__ float4 smem4[];
    __shared__ float red[8];
    constexpr int F4 = PV_DS / 4;
    const int hd = hd_, rep = nh / nkv, S = (hd / PV_DS) * nkv;
    const int tid = threadIdx.x, sl = blockIdx.x % S, k = blockIdx.x / S;
    const int d0 = (sl % (hd / PV_DS)) * PV_DS, g = sl / (hd / PV_DS);
    const int h = g * rep + k % rep, t = k / rep;
    const int np = *posp + pos_off + t + 1;
    const int m4 = np >> 2, s4 = cm_stride(max_ctx);
    float *ecm = (float *)smem4; /* [4 s4 + 4] scores, then exponentials, chain-major */
    float *vt = ecm + 4 * s4 + 4; /* [PV_DS][PV_RS] products of a tile, one row per dim */
    const float *srow = sc + ((size_t)t * nh + h) * max_ctx;
    const size_t R0 = (size_t)g * max_ctx;
    const float *vsc = kv_scales<KVT>(vc, a);
    /* the output gate of lane tid < PV_DS (read here so its latency overlaps the tile's) */
    const float gate = tid < PV_DS ? a.q[((size_t)t * nh + h) * 2 * hd + hd + d0 + tid] : 0.0f;
    /* the scores row, then the first tile's values (element f = u 256 + tid: float4 f % F4 of
     * row f / F4) */
    float bs[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int p = u * 256 + tid;
        bs[u] = p < np ? srow[p] : 0.0f;
    }
    const int rows0 = np < PV_PT ? np : PV_PT;
    /* the first tile in two halves of PV_HA rows: the first half's values in every thread
     * (element f = u 256 + tid), the second half's in waves 1-3 only (f = u 192 + tid - 64),
     * which store its products while wave 0 runs the first half's chains */
    constexpr int PV_UA = PV_PER / 2, PV_HA = PV_UA * 256 / F4, PV_UB = PV_UA * 256 / 192;
    static_assert(PV_PER % 2 == 0 && PV_UA * 256 % 192 == 0 && PV_HA % 4 == 0,
                  "halves of whole rows, the second 16-byte aligned in LDS");
    float4 va[PV_UA], vbh[PV_UB];
#pragma unroll
    for (int u = 0; u < PV_UA; u++) {
        const int f = u * 256 + tid, r = f / F4, c4 = f - r * F4;
        va[u] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (r < rows0) va[u] = kv_load4<KVT>(vc, R0 + r, hd, d0 + 4 * c4, vsc);
    }
    if (tid >= 64) {
#pragma unroll
        for (int u = 0; u < PV_UB; u++) {
            const int f = u * 192 + tid - 64, r = PV_HA + f / F4, c4 = f % F4;
            vbh[u] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (r < rows0) vbh[u] = kv_load4<KVT>(vc, R0 + r, hd, d0 + 4 * c4, vsc);
        }
    }
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int p = u * 256 + tid;
        if (p < np) ecm[pv_cm(p, m4, s4)] = bs[u];
    }
    for (int p0 = 4 * 256; p0 < np; p0 += 256) { /* contexts beyond 1024 positions */
        const int p = p0 + tid;
        if (p < np) ecm[pv_cm(p, m4, s4)] = srow[p];
    }
    __syncthreads();
    float mx = -INFINITY;
    for (int p = tid; p < np; p += 256) mx = fmaxf(mx, ecm[pv_cm(p, m4, s4)]);
    mx = nmx_max_f32_wave(mx);
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    for (int p = tid; p < np; p += 256) {
        const int i = pv_cm(p, m4, s4);
        ecm[i] = nmx_expf_cephes(ecm[i] - mx);
    }
    __syncthreads();
    /* 4 partial sums over e[4m + l] (m ascending) + the tail, in the reference's order */
    if (tid < 4) {
        red[tid] = pv_chain4(0.0f, ecm + tid * s4, m4);
    } else if (tid == 4) {
        float tl = 0.0f;
        for (int i = 0; i < np - 4 * m4; i++) tl = tl + ecm[4 * s4 + i];
        red[4] = tl;
    }
    __syncthreads();
    const float inv = 1.0f / (((red[0] + red[1]) + (red[2] + red[3])) + red[4]);
    /* w_p = e_p * (1 / sum); the tile's rows of dims 4 c4 .. 4 c4 + 3 get w_p v_p[d] */
    auto put = [&](int r, int c4, float w, float4 v) {
        float *q = vt + 4 * c4 * PV_RS + r;
        q[0] = w * v.x;
        q[PV_RS] = w * v.y;
        q[2 * PV_RS] = w * v.z;
        q[3 * PV_RS] = w * v.w;
    };
    float o = 0.0f;
    /* every thread stores the first half's products; then wave 0's chain lanes add them while
     * waves 1-3 store the second half's (whose values may still be arriving); the chains go on
     * over the second half and the later tiles, each adding the positions in order */
    const int hA = rows0 < PV_HA ? rows0 : PV_HA;
#pragma unroll
    for (int u = 0; u < PV_UA; u++) {
        const int f = u * 256 + tid, r = f / F4, c4 = f - r * F4;
        if (r < rows0) put(r, c4, ecm[pv_cm(r, m4, s4)] * inv, va[u]);
    }
    __syncthreads();
    if (tid < PV_DS) {
        o = pv_chain4(o, vt + tid * PV_RS, hA);
    } else if (tid >= 64) {
#pragma unroll
        for (int u = 0; u < PV_UB; u++) {
            const int f = u * 192 + tid - 64, r = PV_HA + f / F4, c4 = f % F4;
            if (r < rows0) put(r, c4, ecm[pv_cm(r, m4, s4)] * inv, vbh[u]);
        }
    }
    __syncthreads();
    for (int base = hA, rows = rows0 - hA, voff = hA; base < np;) {
        const int next = base + rows, rows2 = np - next < PV_PT2 ? np - next : PV_PT2;
        float4 nb[PV_PER2];
        if (tid >= 64 && next < np) { /* waves 1-3: the next tile, during wave 0's chains */
            const int f0 = tid - 64;
#pragma unroll
            for (int u = 0; u < PV_PER2; u++) {
                const int f = u * 192 + f0, r = f / F4, c4 = f - r * F4;
                nb[u] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if (r < rows2) nb[u] = kv_load4<KVT>(vc, R0 + next + r, hd, d0 + 4 * c4, vsc);
            }
        }
        if (tid < PV_DS) o = pv_chain4(o, vt + tid * PV_RS + voff, rows);
        __syncthreads(); /* the chains of this tile are done */
        if (next >= np) break;
        if (tid >= 64) {
            const int f0 = tid - 64;
#pragma unroll
            for (int u = 0; u < PV_PER2; u++) {
                const int f = u * 192 + f0, r = f / F4, c4 = f - r * F4;
                if (r < rows2) put(r, c4, ecm[pv_cm(next + r, m4, s4)] * inv, nb[u]);
            }
        }
        __syncthreads();
        base = next, rows = rows2, voff = 0;
    }
    if (tid < PV_DS) {
        o = o * nmx_sigmoid(gate);
        const int col = h * hd + d0 + tid;
        a.o[(size_t)t * nh * hd + col] = o;
        if (a.aq) a8_block(o, col >> 5, t, a.n, a.aq, a.ad, a.afs);
    }
}

/* The same softmax and P.V for caches longer than the scores row that fits in LDS (max_ctx
 * above PV_ATT_MAX): the max over the row from the scores workspace, then the exponentials
 * segment by segment (SEG positions in LDS) with the four ordered partial sums and the tail
 * carried across segments, then the value rows in tiles, each weight recomputed as
 * e_p * (1 / sum) with e_p = exp(s_p - max) (the same operations as the in-LDS kernel, so the
 * results are identical). */
constexpr int PV_ATT_MAX = 8192; /* scores kept in LDS by attn_pv_k */
constexpr int PV_SEG = 4096;     /* positions per exponential segment of attn_pv_long_k */

template <int KVT>
__global__ __launch_bounds__(256) void attn_pv_long_k(Attn a, const float *__restrict__ sc) {
    extern __shared__ float4 smem4[];
    __shared__ float red[8];
    constexpr int F4 = PV_DS / 4;
    const int hd = a.hd, rep = a.nh / a.nkv, S = (hd / PV_DS) * a.nkv;
    const int tid = threadIdx.x, sl = blockIdx.x % S, k = blockIdx.x / S;
    const int d0 = (sl % (hd / PV_DS)) * PV_DS, g = sl / (hd / PV_DS);
    const int h = g * rep + k % rep, t = k / rep;
    const int np = *a.pos + a.pos_off + t + 1;
    float *seg = (float *)smem4;     /* [PV_SEG] */
    float *vt = seg + PV_SEG;        /* [PV_PT2][PV_DS] */
    const float *srow = sc + ((size_t)t * a.nh + h) * a.max_ctx;
    const size_t R0 = (size_t)g * a.max_ctx;
    const float *vsc = kv_scales<KVT>(a.vc, a);

    float mx = -INFINITY;
    for (int p = tid; p < np; p += 256) mx = fmaxf(mx, srow[p]);
    mx = nmx_max_f32_wave(mx);
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();

    /* partial sum l over e[4m + l], m ascending (m < np / 4), and the tail, in order */
    const int q4 = 4 * (np >> 2);
    float chain = 0.0f; /* lane tid < 4: partial sum tid; lane 4: the tail */
    for (int s0 = 0; s0 < np; s0 += PV_SEG) {
        const int len = np - s0 < PV_SEG ? np - s0 : PV_SEG;
        for (int p = tid; p < len; p += 256) seg[p] = nmx_expf_cephes(srow[s0 + p] - mx);
        __syncthreads();
        const int full = q4 - s0 < len ? (q4 - s0 > 0 ? q4 - s0 : 0) : len; /* in quads' range */
        if (tid < 4) chain = pv_chain(chain, seg + tid, 4, full >> 2);
        else if (tid == 4)
            for (int i = full; i < len; i++) chain = chain + seg[i];
        __syncthreads();
    }
    if (tid < 5) red[tid] = chain;
    __syncthreads();
    const float inv = 1.0f / (((red[0] + red[1]) + (red[2] + red[3])) + red[4]);

    float o = 0.0f;
    for (int base = 0; base < np; base += PV_PT2) {
        const int rows = np - base < PV_PT2 ? np - base : PV_PT2;
        for (int f = tid; f < rows * F4; f += 256) {
            const int r = f / F4, c4 = f - r * F4;
            const float4 v = kv_load4<KVT>(a.vc, R0 + base + r, hd, d0 + 4 * c4, vsc);
            const float w = nmx_expf_cephes(srow[base + r] - mx) * inv;
            *(float4 *)(vt + r * PV_DS + 4 * c4) = make_float4(w * v.x, w * v.y, w * v.z, w * v.w);
        }
        __syncthreads();
        if (tid < PV_DS) o = pv_chain(o, vt + tid, PV_DS, rows);
        __syncthreads();
    }
    if (tid < PV_DS) {
        const int d = d0 + tid;
        const float *qrow = a.q + ((size_t)t * a.nh + h) * 2 * hd;
        o = o * nmx_sigmoid(qrow[hd + d]);
        const int col = h * hd + d;
        a.o[(size_t)t * a.nh * hd + col] = o;
        if (a.aq) a8_block(o, col >> 5, t, a.n, a.aq, a.ad, a.afs);
    }
}

/* ---- confidence gate of a draft (engine/src/spec.c:93-97, forward_ops.c:294-353) -------
 * p = 1 / s, s = sum of e_i = pf_expf(l_i - max) in the reference's order; flag = p >= tau.
 * The e_i are summed in fp64 first (error ~ n 2^-53, negligible); the ordered fp32 sum differs
 * from the exact one by at most (n / 4 + n % 4 + 3) 2^-24 relative (positive terms), so unless
 * 1 / s64 is within twice n 2^-24 of tau the comparison is decided. Otherwise the fp32 sum is
 * formed as the reference forms it, the exponentials PV_SEG at a time in LDS, the four partial
 * sums and the tail carried across segments. */
__global__ __launch_bounds__(1024) void top1_gate_k(const float *__restrict__ l, int n, float tau,
                                                    int32_t *__restrict__ flag) {
    __shared__ float seg[PV_SEG];
    __shared__ float redf[16];
    __shared__ double redd[16];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    float mx = -INFINITY;
    for (int i = tid; i < n; i += 1024) mx = fmaxf(mx, l[i]);
    mx = nmx_max_f32_wave(mx);
    if (lane == 0) redf[w] = mx;
    __syncthreads();
    mx = redf[0];
    for (int j = 1; j < 16; j++) mx = fmaxf(mx, redf[j]);
    double s64 = 0.0;
    for (int i = tid; i < n; i += 1024) s64 += (double)nmx_expf_cephes(l[i] - mx);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) s64 += __shfl_xor(s64, off);
    if (lane == 0) redd[w] = s64;
    __syncthreads();
    s64 = 0.0;
    for (int j = 0; j < 16; j++) s64 += redd[j];
    const double p64 = s64 > 0.0 ? 1.0 / s64 : 0.0, m = 2.0 * (double)(n + 16) * 0x1p-24;
    if (p64 * (1.0 - m) >= (double)tau || p64 * (1.0 + m) < (double)tau) {
        if (tid == 0) flag[0] = p64 >= (double)tau;
        return; /* uniform: every thread took the same branch */
    }
    const int q4 = 4 * (n >> 2);
    float chain = 0.0f; /* lane tid < 4: partial sum tid; lane 4: the tail */
    for (int s0 = 0; s0 < n; s0 += PV_SEG) {
        const int len = n - s0 < PV_SEG ? n - s0 : PV_SEG;
        __syncthreads(); /* the previous segment is consumed */
        for (int i = tid; i < len; i += 1024) seg[i] = nmx_expf_cephes(l[s0 + i] - mx);
        __syncthreads();
        const int full = q4 - s0 < len ? (q4 - s0 > 0 ? q4 - s0 : 0) : len;
        if (tid < 4) chain = pv_chain(chain, seg + tid, 4, full >> 2);
        else if (tid == 4)
            for (int i = full; i < len; i++) chain = chain + seg[i];
    }
    __syncthreads();
    if (tid < 5) redf[tid] = chain;
    __syncthreads();
    if (tid == 0) {
        const float sum = ((redf[0] + redf[1]) + (redf[2] + redf[3])) + redf[4];
        const float p = sum > 0.0f ? 1.0f / sum : 0.0f;
        flag[0] = p >= tau;
    }
}

/* ---- rollback commit over every linear layer (engine/src/forward_lin.c:185-204): with
 * E = e - 1 (e = ctl[1]), conv state <- last K-1 rows of [state after token 0, raw inputs
 * 1..E]; pending replay rows <- log rows 1..E; ctl[2] = E (keep). With bak, the rows of the
 * state after token 0 are kept there; redo computes the commit from them instead (a second
 * commit of a smaller e after the first, when the host stops inside the accepted run). */
struct Commit {
    int layers, C, S;            /* linear layers, conv channels, K - 1 */
    float *state;                /* [layers][S][C] */
    const float *xin;            /* [layers][cap][C] */
    const float *log;            /* [layers][cap][row] */
    float *pend;                 /* [layers][cap][row] */
    int cap, row;                /* rows per log, floats per log row (heads (dk + dv + 1)) */
    int32_t *ctl;
    int32_t *vt;                 /* optional: vt[0] = vt[ctl[1]] */
    float *bak;                  /* optional: [layers][S][C] state after token 0 */
    int redo;                    /* commit from bak (which the first commit filled) */
    /* the acceptance from the head's partial keys (keys NULL: e = ctl[1] from the head's own
     * reduction): n rows of nkeys keys, drafts d1..d(n-1) from the head launch's copy */
    const unsigned long long *keys;
    int nkeys, n;
    const int32_t *drafts;
    int32_t *out;                /* [2 + n]: a, bonus, argmax of each row */
    int32_t *mb;                 /* optional host mailbox of nvt tokens */
    int nvt;
};

constexpr int ACC_MAX_N = 16; /* rows of an acceptance resolved from keys */

/* The verify's argmax per row from the head's partial keys, then the acceptance loop
 * (engine/src/spec.c:340-345): a = 0; g = argmax(row 0); while a < n - 1 and drafts[a] == g:
 * a++, g = argmax(row a). Every workgroup of the commit resolves it itself (the same keys, the
 * same result); workgroup (0, 0) also writes what head_finish_k writes with a commit: out, vt[a
 * + 1] = g, ctl[1] = e = a + 1, the mailbox [a, g, vt[0..nvt) after that update] and its flag
 * (system-scope release), and cur: vt[0] = g. The drafts come from the head launch's copy, so
 * that no workgroup reads a vt entry that workgroup (0, 0) writes. Returns a. */
__device__ int accept_from_keys(const Commit &a, bool lead) {
    __shared__ unsigned long long red[4][ACC_MAX_N];
    __shared__ int am[ACC_MAX_N], s_dr[ACC_MAX_N], s_vt[64], s_a;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    unsigned long long k[ACC_MAX_N];
#pragma unroll
    for (int v = 0; v < ACC_MAX_N; v++) k[v] = 0ull;
    for (int b = tid; b < a.nkeys; b += 256) {
        unsigned long long o[ACC_MAX_N]; /* every row's load issued before the first compare */
#pragma unroll
        for (int v = 0; v < ACC_MAX_N; v++)
            if (v < a.n) o[v] = a.keys[(size_t)v * a.nkeys + b];
#pragma unroll
        for (int v = 0; v < ACC_MAX_N; v++)
            if (v < a.n) k[v] = o[v] > k[v] ? o[v] : k[v];
    }
    /* the drafts and vt after the keys: loads complete in order, so their LDS stores cannot
     * hold back the key requests */
    const int dr = tid < a.n - 1 ? a.drafts[tid] : 0;
    const int vv = lead && a.mb && tid < a.nvt ? a.vt[tid] : 0;
    if (tid < a.n - 1) s_dr[tid] = dr;
    if (lead && a.mb && tid < a.nvt) s_vt[tid] = vv;
#pragma unroll
    for (int v = 0; v < ACC_MAX_N; v++) {
        if (v < a.n) { /* uniform */
            const unsigned long long m = nmx_max_u64_wave(k[v]);
            if (lane == 0) red[wv][v] = m;
        }
    }
    __syncthreads();
    if (tid < a.n) {
        unsigned long long m = red[0][tid];
        for (int w = 1; w < 4; w++) m = red[w][tid] > m ? red[w][tid] : m;
        am[tid] = (int)(0xffffffffu - (unsigned)(m & 0xffffffffull));
    }
    __syncthreads();
    if (tid == 0) {
        int acc = 0, g = am[0];
        while (acc < a.n - 1 && s_dr[acc] == g) {
            acc++;
            g = am[acc];
        }
        s_a = acc;
        if (lead) {
            a.out[0] = acc;
            a.out[1] = g;
            for (int t = 0; t < a.n; t++) a.out[2 + t] = am[t];
            a.vt[acc + 1] = g;
            a.ctl[1] = acc + 1;
            if (a.mb) {
                a.mb[0] = acc;
                a.mb[1] = g;
                for (int i = 0; i < a.nvt; i++) a.mb[2 + i] = i == acc + 1 ? g : s_vt[i];
                __hip_atomic_store(a.mb + 2 + a.nvt, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
            }
            a.vt[0] = g; /* cur <- vt[e] */
        }
    }
    __syncthreads();
    return s_a;
}

/* The commit of e = E + 1 tokens per linear layer (one conv channel per thread: the grid
 * covers C): the conv state rows become rows E .. E + S - 1 of [state after token 0; xin rows
 * 1 ..], and log rows 1 .. E become the pending rows. Every row a commit can take is requested
 * before E is known (E <= n - 1 with keys, read from ctl otherwise), so the acceptance's round
 * trip and these loads overlap, and the commit itself only selects and stores. */
__global__ __launch_bounds__(256) void commit_k(Commit a) {
    constexpr int XR = ACC_MAX_N - 1, LR = 4; /* xin rows, log values per thread, in registers */
    const int l = blockIdx.y;
    const bool lead = blockIdx.x == 0 && l == 0;
    const int tid = blockIdx.x * 256 + threadIdx.x, stride = gridDim.x * 256, c = tid;
    float *st = a.state + (size_t)l * a.S * a.C;
    float *bk = a.bak ? a.bak + (size_t)l * a.S * a.C : nullptr;
    const float *src0 = a.redo ? bk : st; /* rows of the state after token 0 */
    const float *xi = a.xin + (size_t)l * a.cap * a.C;
    const float *lg = a.log + (size_t)l * a.cap * a.row;
    float *pd = a.pend + (size_t)l * a.cap * a.row;
    const int E0 = a.keys ? 0 : a.ctl[1] - 1;
    const int emax = a.keys ? a.n - 1 : E0; /* the largest E */
    const bool ch = c < a.C;
    float old[8], xr[XR], lv[LR];
#pragma unroll
    for (int j = 0; j < 8; j++) old[j] = ch && j < a.S ? src0[(size_t)j * a.C + c] : 0.0f;
#pragma unroll
    for (int u = 0; u < XR; u++) xr[u] = ch && u < emax ? xi[(size_t)(u + 1) * a.C + c] : 0.0f;
#pragma unroll
    for (int u = 0; u < LR; u++) {
        const int i = tid + u * stride;
        lv[u] = i < emax * a.row ? lg[a.row + i] : 0.0f;
    }
    const int E = a.keys ? accept_from_keys(a, lead) : E0;
    if (E == 0 && !a.redo) { /* e = 1: the state after token 0 is the committed one, no replay
                              * rows, and no later commit of a smaller e can need the kept rows */
        if (l == 0 && tid == 0) {
            a.ctl[2] = 0;
            if (a.vt && !a.keys) a.vt[0] = a.vt[1];
        }
        return;
    }
    if (ch) {
        float nv[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int src = j + E; /* row src of [state after token 0 (S rows); xin rows 1 ..] */
            float x = 0.0f;
            if (src < a.S) {
#pragma unroll
                for (int r = 0; r < 8; r++) x = r == src ? old[r] : x;
            } else if (src - a.S < XR) {
#pragma unroll
                for (int u = 0; u < XR; u++) x = u == src - a.S ? xr[u] : x;
            } else {
                x = xi[(size_t)(src - a.S + 1) * a.C + c];
            }
            nv[j] = j < a.S ? x : 0.0f;
        }
        if (bk && !a.redo) {
#pragma unroll
            for (int j = 0; j < 8; j++)
                if (j < a.S) bk[(size_t)j * a.C + c] = old[j];
        }
#pragma unroll
        for (int j = 0; j < 8; j++)
            if (j < a.S) st[(size_t)j * a.C + c] = nv[j];
    }
#pragma unroll
    for (int u = 0; u < LR; u++) {
        const int i = tid + u * stride;
        if (i < E * a.row) pd[i] = lv[u]; /* E <= emax */
    }
    for (int i = tid + LR * stride; i < E * a.row; i += stride) pd[i] = lg[a.row + i];
    if (l == 0 && tid == 0) {
        a.ctl[2] = E;
        if (a.vt && !a.keys) a.vt[0] = a.vt[E + 1]; /* cur <- vt[e] */
    }
}

/* a = out[0], g = out[1] of nmx_head_accept: vt[a + 1] = g; ctl[1] = e = a + 1. */
/* mb (optional, host memory): [a, bonus, vt[0..nvt) after the update], then mb[2 + nvt] = 1
 * with a system-scope release, so a host that reads 1 there (acquire) sees the values. One
 * thread writes everything, in that order. */
__global__ void accept_commit_k(const int32_t *out, int32_t *vt, int32_t *ctl, int32_t *mb, int nvt) {
    const int a = out[0], bonus = out[1];
    vt[a + 1] = bonus;
    ctl[1] = a + 1;
    if (mb) {
        mb[0] = a;
        mb[1] = bonus;
        for (int i = 0; i < nvt; i++) mb[2 + i] = i == a + 1 ? bonus : vt[i];
        __hip_atomic_store(mb + 2 + nvt, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

/* y[i] = gate (0: nmx_gate_expf, 1: nmx_gate_log1pf) of the binary32 input with bit pattern
 * first + i */
__global__ __launch_bounds__(256) void gate_eval_k(int which, uint32_t first, long n,
                                                   float *__restrict__ y) {
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256) {
        const float x = __uint_as_float(first + (uint32_t)i);
        y[i] = which ? nmx_gate_log1pf(x) : nmx_gate_expf(x);
    }
}

__global__ void ctl_k(int32_t *ctl, int op, int idx, int value) {
    if (op == 0) ctl[idx] = value;          /* set */
    else ctl[0] = ctl[0] + ctl[1];          /* advance n_past by e */
}

__global__ void copy_token_k(int32_t *vt, const int32_t *ctl) { vt[0] = vt[ctl[1]]; }

/* dst[c] = src[(*idx + off) * stride + c] */
__global__ void select_row_k(const float *src, int stride, const int32_t *idx, int off, int cols,
                             float *dst) {
    const int r = *idx + off;
    for (int c = blockIdx.x * 256 + threadIdx.x; c < cols; c += gridDim.x * 256)
        dst[c] = src[(size_t)r * stride + c];
}

} // namespace

extern "C" {

int nmx_embed_q4k(nmx_ctx *ctx, const void *W, int vocab, int cols, const int32_t *tok, int n,
                  float *X, int x_stride) {
    if (!ctx) return -1;
    if (!W || !tok || !X || vocab <= 0 || vocab % 4 || cols <= 0 || cols % 256 || n < 1 ||
        n > 4096 || x_stride < cols)
        return nmx_fail(ctx, "nmx_embed_q4k: bad arguments");
    dim3 grid((unsigned)((cols + 255) / 256), (unsigned)n);
    embed_k<<<grid, 256, 0, ctx->stream>>>((const uint8_t *)W, cols, tok, X, x_stride);
    NMX_LAUNCHED(ctx, "embed");
    return 0;
}

int nmx_rmsnorm_xo(nmx_ctx *ctx, const float *x, int x_stride, const float *add, int add_stride,
                   float *xo, int xo_stride, const float *w, int n, int cols, float eps, float *y,
                   int y_stride, nmx_a8 a8) {
    if (!ctx) return -1;
    if (!x || !w || n < 1 || n > 4096 || cols < 1 || cols > 16384 || x_stride < cols ||
        (add && add_stride < cols) || (y && y_stride < cols) || (xo && xo_stride < cols))
        return nmx_fail(ctx, "nmx_rmsnorm: bad arguments n=%d cols=%d", n, cols);
    if (a8.q && (cols % 32 || !a8.d || !a8.fs)) return nmx_fail(ctx, "nmx_rmsnorm: bad A8 output");
    const size_t lds = ((size_t)4 * cm_stride(cols) + 4) * 4;
    auto al16 = [](const void *p) { return ((uintptr_t)p & 15) == 0; };
    if (cols % 32 == 0 && cols <= 4096 && x_stride % 4 == 0 && al16(x) && al16(w) &&
        (!add || (add_stride % 4 == 0 && al16(add))) && (!xo || (xo_stride % 4 == 0 && al16(xo))) &&
        (!y || (y_stride % 4 == 0 && al16(y)))) {
#define NMX_RMS4(P)                                                                             \
    rmsnorm4_k<P><<<(unsigned)n, 256, lds, ctx->stream>>>(x, x_stride, add, add_stride, xo,     \
                                                          xo_stride, w, cols, eps, y, y_stride, \
                                                          a8.q, a8.d, a8.fs, n)
        if (cols <= 1024) NMX_RMS4(1);
        else if (cols <= 2048) NMX_RMS4(2);
        else NMX_RMS4(4);
#undef NMX_RMS4
        NMX_LAUNCHED(ctx, "rmsnorm");
        return 0;
    }
#define NMX_RMS(P)                                                                              \
    rmsnorm_k<P><<<(unsigned)n, 256, lds, ctx->stream>>>(x, x_stride, add, add_stride, xo,      \
                                                         xo_stride, w, cols, eps, y, y_stride,  \
                                                         a8.q, a8.d, a8.fs, n)
    if (cols <= 1024) NMX_RMS(4);
    else if (cols <= 2048) NMX_RMS(8);
    else if (cols <= 4096) NMX_RMS(16);
    else NMX_RMS(64);
#undef NMX_RMS
    NMX_LAUNCHED(ctx, "rmsnorm");
    return 0;
}

int nmx_rmsnorm_pair(nmx_ctx *ctx, int n, int cols, float eps, const float *x0, int x0_stride,
                     const float *w0, float *y0, int y0_stride, nmx_a8 a0, const float *x1,
                     int x1_stride, const float *w1, float *y1, int y1_stride, nmx_a8 a1) {
    if (!ctx) return -1;
    auto al16 = [](const void *p) { return ((uintptr_t)p & 15) == 0; };
    const bool fast = cols % 32 == 0 && cols <= 1024 && x0 && x1 && w0 && w1 && al16(x0) &&
                      al16(x1) && al16(w0) && al16(w1) && x0_stride % 4 == 0 && x1_stride % 4 == 0 &&
                      (!y0 || (al16(y0) && y0_stride % 4 == 0 && y0_stride >= cols)) &&
                      (!y1 || (al16(y1) && y1_stride % 4 == 0 && y1_stride >= cols)) &&
                      x0_stride >= cols && x1_stride >= cols && n >= 1 && n <= 4096 &&
                      (!a0.q || (a0.d && a0.fs)) && (!a1.q || (a1.d && a1.fs));
    if (!fast) /* the general kernel, one launch per set */
        return nmx_rmsnorm_xo(ctx, x0, x0_stride, nullptr, 0, nullptr, 0, w0, n, cols, eps, y0,
                              y0_stride, a0) ||
               nmx_rmsnorm_xo(ctx, x1, x1_stride, nullptr, 0, nullptr, 0, w1, n, cols, eps, y1,
                              y1_stride, a1);
    const RmsSet s0{x0, x0_stride, w0, y0, y0_stride, a0.q, a0.d, a0.fs, nullptr, nullptr, nullptr, 0};
    const RmsSet s1{x1, x1_stride, w1, y1, y1_stride, a1.q, a1.d, a1.fs, nullptr, nullptr, nullptr, 0};
    const size_t lds = ((size_t)4 * cm_stride(cols) + 4) * 4;
    rmsnorm4_pair_k<1><<<dim3((unsigned)n, 2), 256, lds, ctx->stream>>>(s0, s1, cols, eps, n);
    NMX_LAUNCHED(ctx, "rmsnorm_pair");
    return 0;
}

int nmx_rmsnorm_row(nmx_ctx *ctx, const float *x, int x_stride, const float *add,
                    int add_stride, const float *w, int cols, float eps, const int32_t *idx,
                    int off, int nrows, float *y, nmx_a8 a8) {
    if (!ctx) return -1;
    auto al16 = [](const void *p) { return ((uintptr_t)p & 15) == 0; };
    if (!x || !w || !idx || nrows < 1 || cols % 32 || cols < 32 || cols > 1024 || x_stride < cols ||
        x_stride % 4 || !al16(x) || !al16(w) || (add && (add_stride < cols || add_stride % 4 ||
        !al16(add))) || (y && !al16(y)) || (a8.q && (!a8.d || !a8.fs)))
        return nmx_fail(ctx, "nmx_rmsnorm_row: bad arguments cols=%d", cols);
    const size_t lds = ((size_t)4 * cm_stride(cols) + 4) * 4;
    rmsnorm4_row_k<1><<<1, 256, lds, ctx->stream>>>(x, x_stride, add, add_stride, w, cols, eps, idx,
                                                    off, nrows, y, a8.q, a8.d, a8.fs);
    NMX_LAUNCHED(ctx, "rmsnorm_row");
    return 0;
}

int nmx_embed_norm(nmx_ctx *ctx, const void *E, int vocab, const int32_t *tok, int n, int cols,
                   float eps, const float *w0, float *xo0, int xo0_stride, float *y0, int y0_stride,
                   nmx_a8 a0, const float *x1, int x1_stride, const float *w1, float *y1,
                   int y1_stride, nmx_a8 a1) {
    if (!ctx) return -1;
    if (!E || !tok || !w0 || vocab <= 0 || vocab % 4 || cols % 256 || cols < 256 || n < 1 ||
        n > 4096 || (xo0 && xo0_stride < cols) || (y0 && y0_stride < cols) ||
        (x1 && (!w1 || x1_stride < cols || (y1 && y1_stride < cols))))
        return nmx_fail(ctx, "nmx_embed_norm: bad arguments");
    auto al16 = [](const void *p) { return ((uintptr_t)p & 15) == 0; };
    const bool fast = cols <= 1024 && al16(w0) && (!xo0 || (al16(xo0) && xo0_stride % 4 == 0)) &&
                      (!y0 || (al16(y0) && y0_stride % 4 == 0)) && (!a0.q || (a0.d && a0.fs)) &&
                      (!x1 || (al16(x1) && al16(w1) && x1_stride % 4 == 0 &&
                               (!y1 || (al16(y1) && y1_stride % 4 == 0)) && (!a1.q || (a1.d && a1.fs))));
    if (!fast) { /* the embedding into xo0 (required then), then the norms */
        if (!xo0) return nmx_fail(ctx, "nmx_embed_norm: unaligned rows need xo0");
        if (nmx_embed_q4k(ctx, E, vocab, cols, tok, n, xo0, xo0_stride)) return -1;
        if (nmx_rmsnorm_xo(ctx, xo0, xo0_stride, nullptr, 0, nullptr, 0, w0, n, cols, eps, y0,
                           y0_stride, a0))
            return -1;
        return x1 ? nmx_rmsnorm_xo(ctx, x1, x1_stride, nullptr, 0, nullptr, 0, w1, n, cols, eps, y1,
                                   y1_stride, a1)
                  : 0;
    }
    const RmsSet s0{nullptr, 0, w0, y0, y0_stride, a0.q, a0.d, a0.fs,
                    (const uint8_t *)E, tok, xo0, xo0_stride};
    const RmsSet s1{x1, x1_stride, w1, y1, y1_stride, a1.q, a1.d, a1.fs, nullptr, nullptr, nullptr, 0};
    const size_t lds = ((size_t)4 * cm_stride(cols) + 4) * 4;
    rmsnorm4_pair_k<1><<<dim3((unsigned)n, x1 ? 2 : 1), 256, lds, ctx->stream>>>(s0, s1, cols, eps, n);
    NMX_LAUNCHED(ctx, "embed_norm");
    return 0;
}

int nmx_embed_norm_keys(nmx_ctx *ctx, const void *E, int vocab, int32_t *tok, int n, int cols,
                        float eps, const float *w, float *xo, int xo_stride, nmx_a8 a8,
                        const void *keys, int nkeys) {
    if (!ctx) return -1;
    auto al16 = [](const void *p) { return ((uintptr_t)p & 15) == 0; };
    if (!E || !tok || !w || !keys || nkeys < 1 || (uintptr_t)keys % 8 || vocab <= 0 ||
        vocab % 4 || cols % 256 || cols < 256 || cols > 1024 || n < 1 || n > 4096 || !al16(w) ||
        (xo && (xo_stride < cols || !al16(xo) || xo_stride % 4)) || (a8.q && (!a8.d || !a8.fs)))
        return nmx_fail(ctx, "nmx_embed_norm_keys: bad arguments");
    const RmsSet s0{nullptr, 0, w, nullptr, 0, a8.q, a8.d, a8.fs, (const uint8_t *)E, tok, xo,
                    xo_stride, (const unsigned long long *)keys, nkeys, tok};
    const RmsSet s1{};
    const size_t lds = ((size_t)4 * cm_stride(cols) + 4) * 4;
    rmsnorm4_pair_k<1><<<dim3((unsigned)n, 1), 256, lds, ctx->stream>>>(s0, s1, cols, eps, n);
    NMX_LAUNCHED(ctx, "embed_norm");
    return 0;
}

int nmx_rmsnorm(nmx_ctx *ctx, float *x, int x_stride, const float *add, int add_stride,
                const float *w, int n, int cols, float eps, float *y, int y_stride,
                nmx_a8 a8) {
    return nmx_rmsnorm_xo(ctx, x, x_stride, add, add_stride, add ? x : nullptr, x_stride, w, n,
                          cols, eps, y, y_stride, a8);
}

int nmx_lin_pre(nmx_ctx *ctx, const nmx_lin_pre_args *p) {
    if (!ctx) return -1;
    if (!p || p->n < 1 || p->n > 64 || p->conv_k < 1 || p->conv_k > 8 || p->dk < 32 ||
        p->dk > 256 || p->dk % 32 || p->C < 2 * p->kd || p->C % 32 || !p->raw || !p->out ||
        !p->state || !p->conv_w || !p->b_in || !p->a_in || !p->beta || !p->decay ||
        !p->dt_bias || (!p->A_log && !p->A) || p->heads < 1 || p->n * p->heads > 4096 ||
        p->raw_stride < p->C || p->g_stride < p->heads || p->kd % p->dk)
        return nmx_fail(ctx, "nmx_lin_pre: bad arguments");
    LinPre a{p->n, p->C, p->conv_k, p->dk, p->kd, p->raw, p->raw_stride, p->out, p->state,
             p->conv_w, p->xin, p->qscale, p->l2eps, p->b_in, p->a_in, p->g_stride, p->heads,
             p->A_log, p->A, p->dt_bias, p->beta, p->decay};
    const int groups = (p->C + p->dk - 1) / p->dk;
    const unsigned threads = p->dk < 64 ? 64 : (unsigned)p->dk;
    lin_pre_k<<<(unsigned)(groups + 1), threads, (size_t)PRE_TB * p->dk * 4, ctx->stream>>>(a);
    NMX_LAUNCHED(ctx, "lin_pre");
    return 0;
}

int nmx_lin_post(nmx_ctx *ctx, const float *o, int o_stride, const float *z, int z_stride,
                 const float *w, int n, int heads, int dv, float eps, float *y, int y_stride,
                 nmx_a8 a8) {
    if (!ctx) return -1;
    if (!o || !z || !w || n < 1 || n > 4096 || heads < 1 || dv < 32 || dv > 512 || dv % 32 ||
        o_stride < heads * dv || z_stride < heads * dv || (y && y_stride < heads * dv))
        return nmx_fail(ctx, "nmx_lin_post: bad arguments");
    dim3 grid((unsigned)heads, (unsigned)n);
    lin_post_k<<<grid, (unsigned)dv, (size_t)dv * 4, ctx->stream>>>(o, o_stride, z, z_stride, w, dv,
                                                                   eps, y, y_stride, a8.q, a8.d,
                                                                   a8.fs, n);
    NMX_LAUNCHED(ctx, "lin_post");
    return 0;
}

int nmx_silu_mul(nmx_ctx *ctx, const float *gate, const float *up, int stride, int n, int cols,
                 float *y, nmx_a8 a8) {
    if (!ctx) return -1;
    if (!gate || !up || n < 1 || n > 4096 || cols < 32 || cols % 32 || stride < cols)
        return nmx_fail(ctx, "nmx_silu_mul: bad arguments");
    dim3 grid((unsigned)((cols + 255) / 256), (unsigned)n);
    silu_mul_k<<<grid, 256, 0, ctx->stream>>>(gate, up, stride, cols, y, a8.q, a8.d, a8.fs, n);
    NMX_LAUNCHED(ctx, "silu_mul");
    return 0;
}

static int attn_args(nmx_ctx *ctx, const nmx_attn_args *p, Attn *a) {
    if (!p || p->n < 1 || p->n > 64 || p->nkv < 1 || p->nh < p->nkv || p->nh % p->nkv ||
        p->hd < 64 || p->hd > 512 || p->hd % 64 || p->rot % 2 || p->rot > p->hd ||
        p->max_ctx < 1 || p->max_ctx > (1 << 20) || !p->q || !p->k_in || !p->v_in || !p->q_norm ||
        !p->k_norm || !p->rope_cos || !p->rope_sin || !p->kc || !p->vc || !p->pos || !p->o)
        return nmx_fail(ctx, "nmx_attn: bad arguments");
    if (p->kv_dtype < KV_F32 || p->kv_dtype > KV_I8)
        return nmx_fail(ctx, "nmx_attn: kv_dtype %d", p->kv_dtype);
    *a = Attn{p->n, p->nh, p->nkv, p->hd, p->rot, p->max_ctx, p->q, p->k_in, p->v_in, p->q_norm,
              p->k_norm, p->eps, p->scale, p->rope_cos, p->rope_sin, p->kc, p->vc, p->pos,
              p->pos_off, p->o, p->a8.q, p->a8.d, p->a8.fs};
    return 0;
}

} /* extern "C" */

namespace {

template <int KVT>
void launch_attn_prep(nmx_ctx *ctx, const nmx_attn_args *p, const Attn &a) {
    dim3 grid((unsigned)(p->nkv + p->nh), (unsigned)p->n);
    attn_prep_k<KVT><<<grid, (unsigned)p->hd, (size_t)p->hd * 4, ctx->stream>>>(a);
}

template <int KVT>
int launch_pv(nmx_ctx *ctx, const nmx_attn_args *p, const Attn &a);

template <int KVT>
int launch_attn(nmx_ctx *ctx, const nmx_attn_args *p, const Attn &a) {
    const int cp = p->hd <= 256 ? 32 : 16;
    dim3 sgrid((unsigned)((p->max_ctx + cp - 1) / cp), (unsigned)p->n, (unsigned)p->nkv);
    const size_t slds = ((size_t)cp * (p->hd + 4) + 4 * (size_t)p->hd) * 4;
    if (cp == 32) attn_score_k<32, KVT><<<sgrid, 256, slds, ctx->stream>>>(a, p->scores);
    else attn_score_k<16, KVT><<<sgrid, 256, slds, ctx->stream>>>(a, p->scores);
    NMX_LAUNCHED(ctx, "attn_score");
    return launch_pv<KVT>(ctx, p, a);
}

template <int KVT>
int launch_pv(nmx_ctx *ctx, const nmx_attn_args *p, const Attn &a) {
    const unsigned pgrid = (unsigned)((p->hd / PV_DS) * p->nh * p->n);
    const size_t plds = ((size_t)4 * cm_stride(p->max_ctx) + 4 + (size_t)PV_DS * PV_RS) * 4;
    static bool pv_ready = false; /* idempotent */
    if (!pv_ready) {
        NMX_HIP(ctx, hipFuncSetAttribute((const void *)attn_pv_k<KVT>,
                                         hipFuncAttributeMaxDynamicSharedMemorySize,
                                         (int)((4 * (size_t)cm_stride(PV_ATT_MAX) + 4 +
                                                (size_t)PV_DS * PV_RS) * 4)));
        pv_ready = true;
    }
    if (p->max_ctx > PV_ATT_MAX) {
        const size_t llds = ((size_t)PV_SEG + (size_t)PV_PT2 * PV_DS) * 4;
        attn_pv_long_k<KVT><<<pgrid, 256, llds, ctx->stream>>>(a, p->scores);
    } else {
        attn_pv_k<KVT><<<pgrid, 256, plds, ctx->stream>>>(p->scores, a.pos, a.vc, a.pos_off, a.max_ctx,
                                                           a.nh, a.nkv, a.hd, a);
    }
    NMX_LAUNCHED(ctx, "attn_pv");
    return 0;
}

/* attn_qk_k + the P.V launch of launch_attn; outside attn_qk_k's limits, and for passes of
 * more than 8 tokens (prefill chunks: each of their workgroups would redo up to 32 key rows'
 * norms, measured slower than the separate launch), the three launches */
template <int KVT>
int launch_attn_fused(nmx_ctx *ctx, const nmx_attn_args *p, const Attn &a) {
    if (p->hd != QK_HD || p->nh / p->nkv > 4 || p->n > QK_NMAX) {
        launch_attn_prep<KVT>(ctx, p, a);
        NMX_LAUNCHED(ctx, "attn_prep");
        return launch_attn<KVT>(ctx, p, a);
    }
    constexpr int CP = 32;
    const size_t lds = ((size_t)CP * (QK_HD + 4) + (8 + (size_t)QK_NMAX) * QK_HD) * 4;
    static bool ready = false; /* idempotent */
    if (!ready) {
        NMX_HIP(ctx, hipFuncSetAttribute((const void *)attn_qk_k<CP, KVT>,
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        ready = true;
    }
    dim3 grid((unsigned)((p->max_ctx + CP - 1) / CP), (unsigned)p->n, (unsigned)p->nkv);
    attn_qk_k<CP, KVT><<<grid, 256, lds, ctx->stream>>>(a.q, a.pos, a.k_in, a.v_in, a.kc, a.nh, a.nkv,
                                                        a.pos_off, a.max_ctx, a, p->scores);
    NMX_LAUNCHED(ctx, "attn_qk");
    return launch_pv<KVT>(ctx, p, a);
}

} // namespace

extern "C" {

int nmx_attn_fused(nmx_ctx *ctx, const nmx_attn_args *p) {
    if (!ctx) return -1;
    Attn a;
    if (attn_args(ctx, p, &a)) return -1;
    if (!p->scores) return nmx_fail(ctx, "nmx_attn_fused: NULL scores workspace");
    if (p->kv_dtype == KV_F16) return launch_attn_fused<KV_F16>(ctx, p, a);
    if (p->kv_dtype == KV_I8) return launch_attn_fused<KV_I8>(ctx, p, a);
    return launch_attn_fused<KV_F32>(ctx, p, a);
}

int nmx_attn_prep(nmx_ctx *ctx, const nmx_attn_args *p) {
    if (!ctx) return -1;
    Attn a;
    if (attn_args(ctx, p, &a)) return -1;
    if (p->kv_dtype == KV_F16) launch_attn_prep<KV_F16>(ctx, p, a);
    else if (p->kv_dtype == KV_I8) launch_attn_prep<KV_I8>(ctx, p, a);
    else launch_attn_prep<KV_F32>(ctx, p, a);
    NMX_LAUNCHED(ctx, "attn_prep");
    return 0;
}

int nmx_attn(nmx_ctx *ctx, const nmx_attn_args *p) {
    if (!ctx) return -1;
    Attn a;
    if (attn_args(ctx, p, &a)) return -1;
    if (!p->scores) return nmx_fail(ctx, "nmx_attn: NULL scores workspace");
    if (p->kv_dtype == KV_F16) return launch_attn<KV_F16>(ctx, p, a);
    if (p->kv_dtype == KV_I8) return launch_attn<KV_I8>(ctx, p, a);
    return launch_attn<KV_F32>(ctx, p, a);
}

int nmx_top1_gate(nmx_ctx *ctx, const float *logits, int n, float tau, int32_t *flag) {
    if (!ctx) return -1;
    if (!logits || !flag || n < 1 || n > (1 << 24))
        return nmx_fail(ctx, "nmx_top1_gate: bad arguments");
    top1_gate_k<<<1, 1024, 0, ctx->stream>>>(logits, n, tau, flag);
    NMX_LAUNCHED(ctx, "top1_gate");
    return 0;
}

size_t nmx_kv_bytes(int kv_dtype, int nkv, int max_ctx, int hd) {
    if (kv_dtype < KV_F32 || kv_dtype > KV_I8 || nkv < 1 || max_ctx < 1 || hd < 1) return 0;
    const size_t rows = (size_t)nkv * (size_t)max_ctx;
    const size_t es = kv_dtype == KV_F32 ? 4 : kv_dtype == KV_F16 ? 2 : 1;
    return rows * hd * es + (kv_dtype == KV_I8 ? rows * 4 : 0);
}

static int lin_commit(nmx_ctx *ctx, const nmx_commit_args *p, const nmx_accept_keys *k) {
    if (!ctx) return -1;
    if (!p || p->layers < 1 || p->conv_k < 2 || p->conv_k > 8 || p->C < 1 || p->cap < 1 ||
        p->row < 1 || !p->state || !p->xin || !p->log || !p->pend || !p->ctl)
        return nmx_fail(ctx, "nmx_lin_commit: bad arguments");
    if (p->redo && !p->state_bak) return nmx_fail(ctx, "nmx_lin_commit: redo needs state_bak");
    Commit a{p->layers, p->C, p->conv_k - 1, p->state, p->xin, p->log, p->pend, p->cap, p->row,
             p->ctl, p->vt, p->state_bak, p->redo, nullptr, 0, 0, nullptr, nullptr, nullptr, 0};
    if (k) {
        if (p->redo || !p->vt || !k->keys || !k->out || k->nkeys < 1 || k->n < 1 ||
            k->n > ACC_MAX_N || (k->n > 1 && !k->drafts) || (uintptr_t)k->keys % 8 ||
            k->n > p->cap || (k->mailbox && (k->nvt < k->n + 1 || k->nvt > 64)))
            return nmx_fail(ctx, "nmx_lin_commit_keys: bad arguments (n=%d nkeys=%d)", k->n,
                            k->nkeys);
        a.keys = (const unsigned long long *)k->keys;
        a.nkeys = k->nkeys;
        a.n = k->n;
        a.drafts = k->drafts;
        a.out = k->out;
        a.mb = k->mailbox;
        a.nvt = k->mailbox ? k->nvt : 0;
    }
    dim3 grid((unsigned)((p->C + 255) / 256), (unsigned)p->layers);
    commit_k<<<grid, 256, 0, ctx->stream>>>(a);
    NMX_LAUNCHED(ctx, "lin_commit");
    return 0;
}

int nmx_lin_commit(nmx_ctx *ctx, const nmx_commit_args *p) { return lin_commit(ctx, p, nullptr); }

int nmx_lin_commit_keys(nmx_ctx *ctx, const nmx_commit_args *p, const nmx_accept_keys *k) {
    if (!k) return ctx ? nmx_fail(ctx, "nmx_lin_commit_keys: NULL keys") : -1;
    return lin_commit(ctx, p, k);
}

int nmx_accept_commit(nmx_ctx *ctx, const int32_t *out, int32_t *vt, int32_t *ctl) {
    if (!ctx) return -1;
    if (!out || !vt || !ctl) return nmx_fail(ctx, "nmx_accept_commit: NULL pointer");
    accept_commit_k<<<1, 1, 0, ctx->stream>>>(out, vt, ctl, nullptr, 0);
    NMX_LAUNCHED(ctx, "accept_commit");
    return 0;
}

int nmx_accept_commit_mb(nmx_ctx *ctx, const int32_t *out, int32_t *vt, int32_t *ctl,
                         int32_t *mailbox, int nvt) {
    if (!ctx) return -1;
    if (!out || !vt || !ctl || !mailbox || nvt < 1 || nvt > 1024)
        return nmx_fail(ctx, "nmx_accept_commit_mb: bad arguments");
    accept_commit_k<<<1, 1, 0, ctx->stream>>>(out, vt, ctl, mailbox, nvt);
    NMX_LAUNCHED(ctx, "accept_commit");
    return 0;
}

int nmx_gate_eval(nmx_ctx *ctx, int which, uint32_t first, long n, float *y) {
    if (!ctx) return -1;
    if ((which != 0 && which != 1) || n < 1 || !y || (uint64_t)first + (uint64_t)n > (1ull << 32))
        return nmx_fail(ctx, "nmx_gate_eval: bad arguments");
    gate_eval_k<<<2048, 256, 0, ctx->stream>>>(which, first, n, y);
    NMX_LAUNCHED(ctx, "gate_eval");
    return 0;
}

int nmx_ctl_set(nmx_ctx *ctx, int32_t *ctl, int idx, int value) {
    if (!ctx) return -1;
    if (!ctl || idx < 0 || idx > 15) return nmx_fail(ctx, "nmx_ctl_set: bad arguments");
    ctl_k<<<1, 1, 0, ctx->stream>>>(ctl, 0, idx, value);
    NMX_LAUNCHED(ctx, "ctl_set");
    return 0;
}

int nmx_ctl_advance(nmx_ctx *ctx, int32_t *ctl) {
    if (!ctx) return -1;
    if (!ctl) return nmx_fail(ctx, "nmx_ctl_advance: NULL pointer");
    ctl_k<<<1, 1, 0, ctx->stream>>>(ctl, 1, 0, 0);
    NMX_LAUNCHED(ctx, "ctl_advance");
    return 0;
}

int nmx_copy_token(nmx_ctx *ctx, int32_t *vt, const int32_t *ctl) {
    if (!ctx) return -1;
    if (!vt || !ctl) return nmx_fail(ctx, "nmx_copy_token: NULL pointer");
    copy_token_k<<<1, 1, 0, ctx->stream>>>(vt, ctl);
    NMX_LAUNCHED(ctx, "copy_token");
    return 0;
}

int nmx_select_row(nmx_ctx *ctx, const float *src, int stride, const int32_t *idx, int off,
                   int cols, float *dst) {
    if (!ctx) return -1;
    if (!src || !idx || !dst || cols < 1 || stride < cols)
        return nmx_fail(ctx, "nmx_select_row: bad arguments");
    select_row_k<<<(unsigned)((cols + 255) / 256), 256, 0, ctx->stream>>>(src, stride, idx, off, cols,
                                                                         dst);
    NMX_LAUNCHED(ctx, "select_row");
    return 0;
}

} /* extern "C" */
