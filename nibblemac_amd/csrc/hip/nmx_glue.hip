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

namespace {

/* ---- A8 of one 32-value block held by a 32-lane half-wave (lane = column within block) ----
 * engine/src/kern_act.c:14-42: amax, id = 127 / amax, round-half-even codes, d = amax / 127,
 * fsum = d * sum(codes). Writes the block-major element (b, v). */
__device__ __forceinline__ void a8_block(float x, int b, int v, int n, int8_t *q, float *d,
                                         float *fs) {
    const int j = threadIdx.x & 31;
    float amax = fabsf(x);
#pragma unroll
    for (int off = 16; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 32));
    const float id = amax > 0.0f ? 127.0f / amax : 0.0f;
    const int c = (int)rintf(x * id);
    int sum = c;
#pragma unroll
    for (int off = 16; off >= 1; off >>= 1) sum += __shfl_xor(sum, off, 32);
    const size_t u = (size_t)b * n + v;
    q[u * 32 + j] = (int8_t)(c > 127 ? 127 : c < -128 ? -128 : c);
    if (j == 0) {
        const float dd = amax / 127.0f;
        d[u] = dd;
        fs[u] = dd * (float)sum;
    }
}

/* Sum in the reference's order (sumsq forward_ops.c:168-189, pf_softmax_exp :333-353):
 * partial l accumulates v[4m + l] for m ascending over the first cols/4*4 elements;
 * s = (c0 + c1) + (c2 + c3); the tail sequentially into t; result s + t. v[] is in LDS (the
 * squares for a norm); four lanes run the four chains. Every thread of the block gets it. */
__device__ float ordered_sum4(const float *sq, int cols, float *red) {
    const int tid = threadIdx.x, m4 = cols >> 2;
    if (tid < 4) {
        float c = 0.0f;
        for (int m = 0; m < m4; m++) c = c + sq[4 * m + tid];
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
 * y = (x * r) * w; optional A8 of y for the next matmul. One workgroup per row. */
__global__ __launch_bounds__(256) void rmsnorm_k(float *__restrict__ x, int x_stride,
                                                 const float *__restrict__ add, int add_stride,
                                                 const float *__restrict__ w, int cols, float eps,
                                                 float *__restrict__ y, int y_stride,
                                                 int8_t *__restrict__ q, float *__restrict__ d,
                                                 float *__restrict__ fs, int n) {
    extern __shared__ float sq[];
    __shared__ float red[8];
    const int row = blockIdx.x, tid = threadIdx.x;
    float *xr = x + (size_t)row * x_stride;
    for (int i = tid; i < cols; i += 256) {
        float v = xr[i];
        if (add) {
            v = v + add[(size_t)row * add_stride + i];
            xr[i] = v;
        }
        sq[i] = v * v;
    }
    __syncthreads();
    const float ss = ordered_sum4(sq, cols, red);
    const float r = 1.0f / sqrtf(ss / (float)cols + eps);
    for (int base = 0; base < cols; base += 256) {
        const int i = base + tid;
        const bool live = i < cols;
        const float v = live ? (xr[i] * r) * w[i] : 0.0f;
        if (live && y) y[(size_t)row * y_stride + i] = v;
        if (q && base + (tid & ~31) < cols) a8_block(v, i >> 5, row, n, q, d, fs);
    }
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

__global__ __launch_bounds__(256) void lin_pre_k(LinPre a) {
    extern __shared__ float sq[]; /* [dk] squares */
    __shared__ float red[8];
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
    float win[8];
    const int cc = live ? ch : 0;
#pragma unroll
    for (int r = 0; r < 8; r++) win[r] = (r < S) ? a.state[(size_t)r * a.C + cc] : 0.0f;
    const float *wc = a.conv_w + (size_t)cc * a.K;
    const bool norm = blockIdx.x * a.dk < 2 * a.kd;  /* a q or k head */
    const float scale = blockIdx.x * a.dk < a.kd ? a.qscale : 1.0f;
    for (int t = 0; t < a.n; t++) {
        const float xt = a.raw[(size_t)t * a.raw_stride + cc];
        /* taps in order over [state rows (oldest first), x_t] */
        float acc = wc[0] * (S > 0 ? win[0] : xt);
#pragma unroll
        for (int j = 1; j < 8; j++)
            if (j < a.K) acc = acc + wc[j] * (j < S ? win[j] : xt);
        /* shift the window: it now ends with x_t */
#pragma unroll
        for (int j = 0; j < 7; j++)
            if (j + 1 < S) win[j] = win[j + 1];
#pragma unroll
        for (int j = 0; j < 8; j++)
            if (j == S - 1) win[j] = xt;
        if (t == 0 && a.xin && live) {  /* logged pass: token 0 is committed in place */
#pragma unroll
            for (int j = 0; j < 8; j++)
                if (j < S) a.state[(size_t)j * a.C + ch] = win[j];
        }
        if (t > 0 && a.xin && live) a.xin[(size_t)t * a.C + ch] = xt;
        float yv = nmx_silu(acc);
        if (norm) {
            sq[tid] = live ? yv * yv : 0.0f;
            __syncthreads();
            const float ss = ordered_sum4(sq, a.dk, red);
            const float r = 1.0f / sqrtf(ss + a.l2eps);
            yv = (yv * r) * scale;
        }
        if (live) a.out[(size_t)t * a.C + ch] = yv;
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
    float *kc, *vc;      /* [nkv][max_ctx][hd] */
    const int32_t *pos;  /* device: position of token 0 is *pos + pos_off */
    int pos_off;
    float *o;            /* [n][nh hd] */
    int8_t *aq;
    float *ad, *afs;
};

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
    if (is_k) {
        a.kc[((size_t)u * a.max_ctx + p) * hd + i] = v;
        a.vc[((size_t)u * a.max_ctx + p) * hd + i] = a.v_in[(size_t)t * a.nkv * hd + u * hd + i];
    } else {
        a.q[((size_t)t * a.nh + (u - a.nkv)) * 2 * hd + i] = v;
    }
}

/* Scores (pf_dot's 16 interleaved partial sums, then * scale; forward_kv.c:281-303,
 * forward_ops.c:265-287), softmax (max; exp(a - max) with 4 partial sums + tail; * 1/sum;
 * forward_attn.c:171-181, forward_ops.c:294-353), P.V in row order from zero
 * (forward_ops.c:360-382), o *= sigmoid(gate) (forward_attn.c:217-220); + A8 of o for o_proj.
 * One workgroup of hd threads per (token, query head). */
__global__ __launch_bounds__(512) void attn_k(Attn a) {
    extern __shared__ float att[]; /* [np] */
    __shared__ float qs[512];
    __shared__ float red[8];
    const int t = blockIdx.y, h = blockIdx.x, tid = threadIdx.x, hd = a.hd, nt = blockDim.x;
    const int g = h / (a.nh / a.nkv);
    const int np = *a.pos + a.pos_off + t + 1;
    const float *qrow = a.q + ((size_t)t * a.nh + h) * 2 * hd;
    qs[tid] = qrow[tid];
    __syncthreads();
    const float *K = a.kc + (size_t)g * a.max_ctx * hd;
    const int i16 = hd / 16 * 16;
    for (int p = tid; p < np; p += nt) {
        const float *kr = K + (size_t)p * hd;
        float c[16];
#pragma unroll
        for (int l = 0; l < 16; l++) c[l] = 0.0f;
        for (int i = 0; i < i16; i += 16) {
#pragma unroll
            for (int l = 0; l < 16; l++) c[l] = c[l] + qs[i + l] * kr[i + l];
        }
        float hs[4];
#pragma unroll
        for (int k = 0; k < 4; k++) hs[k] = (c[4 * k] + c[4 * k + 1]) + (c[4 * k + 2] + c[4 * k + 3]);
        const float s = (hs[0] + hs[1]) + (hs[2] + hs[3]);
        float tl = 0.0f;
        for (int i = i16; i < hd; i++) tl = tl + qs[i] * kr[i];
        att[p] = (s + tl) * a.scale;
    }
    __syncthreads();
    /* maximum: exact in any order (only its value is used, and exp(x - (+-0)) agrees) */
    float mx = -INFINITY;
    for (int p = tid; p < np; p += nt) mx = fmaxf(mx, att[p]);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = red[0];
    for (int w = 1; w < nt / 64; w++) mx = fmaxf(mx, red[w]);
    __syncthreads();
    for (int p = tid; p < np; p += nt) att[p] = nmx_expf_cephes(att[p] - mx);
    __syncthreads();
    const float sum = ordered_sum4(att, np, red);
    const float inv = 1.0f / sum;
    for (int p = tid; p < np; p += nt) att[p] = att[p] * inv;
    __syncthreads();
    const float *V = a.vc + (size_t)g * a.max_ctx * hd;
    float o = 0.0f;
    for (int p = 0; p < np; p++) o = o + att[p] * V[(size_t)p * hd + tid];
    o = o * nmx_sigmoid(qrow[hd + tid]);
    const int col = h * hd + tid;
    a.o[(size_t)t * a.nh * hd + col] = o;
    if (a.aq) a8_block(o, col >> 5, t, a.n, a.aq, a.ad, a.afs);
}

/* ---- rollback commit over every linear layer (engine/src/forward_lin.c:185-204): with
 * E = e - 1 (e = ctl[1]), conv state <- last K-1 rows of [state after token 0, raw inputs
 * 1..E]; pending replay rows <- log rows 1..E; ctl[2] = E (keep). */
struct Commit {
    int layers, C, S;            /* linear layers, conv channels, K - 1 */
    float *state;                /* [layers][S][C] */
    const float *xin;            /* [layers][cap][C] */
    const float *log;            /* [layers][cap][row] */
    float *pend;                 /* [layers][cap][row] */
    int cap, row;                /* rows per log, floats per log row (heads (dk + dv + 1)) */
    int32_t *ctl;
};

__global__ __launch_bounds__(256) void commit_k(Commit a) {
    const int l = blockIdx.y;
    const int E = a.ctl[1] - 1;
    const int tid = blockIdx.x * 256 + threadIdx.x, stride = gridDim.x * 256;
    float *st = a.state + (size_t)l * a.S * a.C;
    const float *xi = a.xin + (size_t)l * a.cap * a.C;
    for (int c = tid; c < a.C; c += stride) {
        float nv[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int src = j + E;
            nv[j] = j >= a.S ? 0.0f
                  : src < a.S ? st[(size_t)src * a.C + c] : xi[(size_t)(src - a.S + 1) * a.C + c];
        }
#pragma unroll
        for (int j = 0; j < 8; j++)
            if (j < a.S) st[(size_t)j * a.C + c] = nv[j];
    }
    const float *lg = a.log + (size_t)l * a.cap * a.row;
    float *pd = a.pend + (size_t)l * a.cap * a.row;
    for (int i = tid; i < E * a.row; i += stride) pd[i] = lg[a.row + i];
    if (l == 0 && tid == 0) a.ctl[2] = E;
}

/* a = out[0], g = out[1] of nmx_head_accept: vt[a + 1] = g; ctl[1] = e = a + 1. */
__global__ void accept_commit_k(const int32_t *out, int32_t *vt, int32_t *ctl) {
    const int a = out[0];
    vt[a + 1] = out[1];
    ctl[1] = a + 1;
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

int nmx_rmsnorm(nmx_ctx *ctx, float *x, int x_stride, const float *add, int add_stride,
                const float *w, int n, int cols, float eps, float *y, int y_stride,
                nmx_a8 a8) {
    if (!ctx) return -1;
    if (!x || !w || n < 1 || n > 4096 || cols < 1 || cols > 16384 || x_stride < cols ||
        (add && add_stride < cols) || (y && y_stride < cols))
        return nmx_fail(ctx, "nmx_rmsnorm: bad arguments n=%d cols=%d", n, cols);
    if (a8.q && (cols % 32 || !a8.d || !a8.fs)) return nmx_fail(ctx, "nmx_rmsnorm: bad A8 output");
    rmsnorm_k<<<(unsigned)n, 256, (size_t)cols * 4, ctx->stream>>>(
        x, x_stride, add, add_stride, w, cols, eps, y, y_stride, a8.q, a8.d, a8.fs, n);
    NMX_LAUNCHED(ctx, "rmsnorm");
    return 0;
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
    lin_pre_k<<<(unsigned)(groups + 1), threads, (size_t)threads * 4, ctx->stream>>>(a);
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
        p->max_ctx < 1 || p->max_ctx > 8192 || !p->q || !p->k_in || !p->v_in || !p->q_norm ||
        !p->k_norm || !p->rope_cos || !p->rope_sin || !p->kc || !p->vc || !p->pos || !p->o)
        return nmx_fail(ctx, "nmx_attn: bad arguments");
    *a = Attn{p->n, p->nh, p->nkv, p->hd, p->rot, p->max_ctx, p->q, p->k_in, p->v_in, p->q_norm,
              p->k_norm, p->eps, p->scale, p->rope_cos, p->rope_sin, p->kc, p->vc, p->pos,
              p->pos_off, p->o, p->a8.q, p->a8.d, p->a8.fs};
    return 0;
}

int nmx_attn_prep(nmx_ctx *ctx, const nmx_attn_args *p) {
    if (!ctx) return -1;
    Attn a;
    if (attn_args(ctx, p, &a)) return -1;
    dim3 grid((unsigned)(p->nkv + p->nh), (unsigned)p->n);
    attn_prep_k<<<grid, (unsigned)p->hd, (size_t)p->hd * 4, ctx->stream>>>(a);
    NMX_LAUNCHED(ctx, "attn_prep");
    return 0;
}

int nmx_attn(nmx_ctx *ctx, const nmx_attn_args *p) {
    if (!ctx) return -1;
    Attn a;
    if (attn_args(ctx, p, &a)) return -1;
    dim3 grid((unsigned)p->nh, (unsigned)p->n);
    attn_k<<<grid, (unsigned)p->hd, (size_t)p->max_ctx * 4, ctx->stream>>>(a);
    NMX_LAUNCHED(ctx, "attn");
    return 0;
}

int nmx_lin_commit(nmx_ctx *ctx, const nmx_commit_args *p) {
    if (!ctx) return -1;
    if (!p || p->layers < 1 || p->conv_k < 2 || p->conv_k > 8 || p->C < 1 || p->cap < 1 ||
        p->row < 1 || !p->state || !p->xin || !p->log || !p->pend || !p->ctl)
        return nmx_fail(ctx, "nmx_lin_commit: bad arguments");
    Commit a{p->layers, p->C, p->conv_k - 1, p->state, p->xin, p->log, p->pend, p->cap, p->row,
             p->ctl};
    dim3 grid((unsigned)((p->C + 255) / 256), (unsigned)p->layers);
    commit_k<<<grid, 256, 0, ctx->stream>>>(a);
    NMX_LAUNCHED(ctx, "lin_commit");
    return 0;
}

int nmx_accept_commit(nmx_ctx *ctx, const int32_t *out, int32_t *vt, int32_t *ctl) {
    if (!ctx) return -1;
    if (!out || !vt || !ctl) return nmx_fail(ctx, "nmx_accept_commit: NULL pointer");
    accept_commit_k<<<1, 1, 0, ctx->stream>>>(out, vt, ctl);
    NMX_LAUNCHED(ctx, "accept_commit");
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
