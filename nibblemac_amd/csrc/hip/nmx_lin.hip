/* Gated DeltaNet recurrence for gfx950 with the speculative rollback log (include/nmx.h
 * nmx_lin_rule / nmx_lin_apply).
 *
 * Exactness contract (engine/src/matvec_ref.c:114-188): per v-head h, token t and value column
 * j, with S[i][j] the state,
 *   pass 1, i ascending:  S = S * decay;  kv = kv + S * k_i
 *   delta = (v_j - kv) * beta
 *   pass 2, i ascending:  S = S + k_i * delta;  o = o + S * q_i
 * every operation rounded separately. Columns are independent; the two sums over i are not.
 *
 * Mapping: a quad of 4 lanes owns one column j; lane c of the quad keeps the keys
 * i in [c dk/4, (c+1) dk/4) of that column in VGPRs for the whole pass (all tokens, the
 * pending replays, the log), so the state is read from HBM once and written once. The
 * multiplies of both passes run on the 4 lanes in parallel; each ordered sum is carried lane
 * 0 -> 1 -> 2 -> 3 of the quad by DPP (the same left-to-right sequence of fp32 adds as the
 * reference).
 * q and k of the token are staged in LDS (broadcast reads, padded against bank conflicts).
 *
 * State layout in HBM (private to this contract, engine/src/ops.h:74-75; nmx_state_index):
 * per head, the value columns in groups of 16 (one wave's quads), and within a group the
 * float4 slot k of every lane contiguous, so each 128-bit load or store of a wave covers one
 * contiguous 1 KB run (a lane's dk/4 keys contiguous instead put 64 lanes on 64 lines per
 * instruction, and issuing them took about 2 us per workgroup in the mixer).
 * Log rows keep the reference layout [n][heads][dk + dv + 1] = k | delta | decay. */
#include "nmx_internal.h"
#include "nmx_a8.h"

namespace {

/* Tokens (or pending rows) staged per batch: their k / q rows in LDS, gates and v_j in
 * registers, every load of a batch issued before the first is used. */
constexpr int TB = 8;

template <int DK4>
__global__ __launch_bounds__(256) void lin_rule_k(nmx_lin_args a) {
    extern __shared__ float sm[]; /* [TB][4][PAD] k, [TB][4][PAD] q, [TB] decay, [TB] beta */
    constexpr int DK = DK4 * 4, PAD = DK4 + 4, ROW = 4 * PAD;
    float *sk = sm, *sq = sm + TB * ROW, *sdec = sq + TB * ROW, *sbet = sdec + TB;
    const int h = blockIdx.x, tid = threadIdx.x, c = tid & 3;
    const int JW = blockDim.x >> 2;
    const int j = blockIdx.y * JW + (tid >> 2);
    const int dv = a.dv, heads = a.heads;
    const bool live = j < dv;
    const int jj = live ? j : dv - 1;
    const int kh = h / a.rep, kd = (heads / a.rep) * DK;
    const size_t logw = (size_t)DK + dv + 1;
    const bool logged = a.log != nullptr;

    float *Sp = a.S + state_lane(h, jj, c, DK, dv);
    const int SS = state_slot(jj, dv);
    float s[DK4];
#pragma unroll
    for (int r = 0; r < DK4; r += 4) {
        const float4 x = *(const float4 *)(Sp + (r >> 2) * SS);
        s[r] = x.x, s[r + 1] = x.y, s[r + 2] = x.z, s[r + 3] = x.w;
    }

    /* deferred commit of the previous pass (matvec_ref.c:169-188 arithmetic) */
    int keep = a.keep;
    if (a.keep_dev) {
        const int kd_ = *a.keep_dev;
        keep = kd_ < keep ? kd_ : keep;
    }
    for (int u0 = 0; u0 < keep; u0 += TB) {
        const int nb = keep - u0 < TB ? keep - u0 : TB;
        float pdel[TB];
#pragma unroll
        for (int u = 0; u < TB; u++)
            pdel[u] = u < nb ? a.pend[((size_t)(u0 + u) * heads + h) * logw + DK + jj] : 0.0f;
        __syncthreads();
        for (int x0 = 0; x0 < nb * DK; x0 += 8 * (int)blockDim.x) {
            float kb[8];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int x = x0 + e * (int)blockDim.x + tid;
                const int xc = x < nb * DK ? x : nb * DK - 1;
                const int u = xc / DK, i = xc - u * DK;
                kb[e] = a.pend[((size_t)(u0 + u) * heads + h) * logw + i];
            }
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int x = x0 + e * (int)blockDim.x + tid;
                if (x < nb * DK) {
                    const int u = x / DK, i = x - u * DK;
                    sk[u * ROW + (i / DK4) * PAD + i % DK4] = kb[e];
                }
            }
        }
        if (tid < nb) sdec[tid] = a.pend[((size_t)(u0 + tid) * heads + h) * logw + DK + dv];
        __syncthreads();
#pragma unroll
        for (int u = 0; u < TB; u++) {
            if (u < nb) {
                const float pdec = sdec[u];
                const float *kk = sk + u * ROW + c * PAD;
#pragma unroll
                for (int r = 0; r < DK4; r++) {
                    s[r] = s[r] * pdec;
                    s[r] = s[r] + kk[r] * pdel[u];
                }
            }
        }
    }

    const bool store_now = (a.n == 0) || (a.log0 && keep > 0);
    if (store_now && live) {
#pragma unroll
        for (int r = 0; r < DK4; r += 4) *(float4 *)(Sp + (r >> 2) * SS) = make_float4(s[r], s[r + 1], s[r + 2], s[r + 3]);
    }

    for (int t0 = 0; t0 < a.n; t0 += TB) {
        const int nb = a.n - t0 < TB ? a.n - t0 : TB;
        float vj[TB];
#pragma unroll
        for (int u = 0; u < TB; u++)
            vj[u] = u < nb ? a.qkv[(size_t)(t0 + u) * a.qkv_stride + 2 * kd + h * dv + jj] : 0.0f;
        __syncthreads(); /* the previous batch's LDS reads are done */
        /* q / k rows of the batch: 8 elements per thread per round, loads issued first */
        for (int x0 = 0; x0 < nb * DK; x0 += 8 * (int)blockDim.x) {
            float qb[8], kb[8];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int x = x0 + e * (int)blockDim.x + tid;
                const int xc = x < nb * DK ? x : nb * DK - 1;
                const int u = xc / DK, i = xc - u * DK;
                const float *row = a.qkv + (size_t)(t0 + u) * a.qkv_stride;
                qb[e] = row[kh * DK + i];
                kb[e] = row[kd + kh * DK + i];
            }
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int x = x0 + e * (int)blockDim.x + tid;
                if (x < nb * DK) {
                    const int u = x / DK, i = x - u * DK;
                    sq[u * ROW + (i / DK4) * PAD + i % DK4] = qb[e];
                    sk[u * ROW + (i / DK4) * PAD + i % DK4] = kb[e];
                }
            }
        }
        if (tid < nb) {
            sdec[tid] = a.decay[(size_t)(t0 + tid) * heads + h];
            sbet[tid] = a.beta[(size_t)(t0 + tid) * heads + h];
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < TB; u++) {
            if (u >= nb) break;
            const int t = t0 + u;
            const float *kk = sk + u * ROW + c * PAD, *qq = sq + u * ROW + c * PAD;
            const float dec = sdec[u], bet = sbet[u];
            float p[DK4];
#pragma unroll
            for (int r = 0; r < DK4; r++) {
                s[r] = s[r] * dec;
                p[r] = s[r] * kk[r];
            }
            const float kv = nmx_quad_chain<DK4>(p);
            const float del = (vj[u] - kv) * bet;

#pragma unroll
            for (int r = 0; r < DK4; r++) {
                s[r] = s[r] + kk[r] * del;
                p[r] = s[r] * qq[r];
            }
            const float ov = nmx_quad_chain<DK4>(p);
            if (live && c == 0) a.o[(size_t)t * a.o_stride + h * dv + j] = ov;

            if (logged && (t > 0 || a.log0)) {
                float *lr = a.log + ((size_t)t * heads + h) * logw;
                if (live && c == 0) lr[DK + j] = del;
                if (blockIdx.y == 0) {
                    for (int x = tid; x < DK; x += blockDim.x) lr[x] = sk[u * ROW + (x / DK4) * PAD + x % DK4];
                    if (tid == 0) lr[DK + dv] = dec;
                }
            }
            /* the committed state: after token 0 of a reference-mode logged pass, after the
             * last token of a plain pass */
            const bool commit = logged ? (!a.log0 && t == 0) : (t == a.n - 1);
            if (commit && live) {
#pragma unroll
                for (int r = 0; r < DK4; r += 4)
                    *(float4 *)(Sp + (r >> 2) * SS) = make_float4(s[r], s[r + 1], s[r + 2], s[r + 3]);
            }
        }
    }
}

template <int DK4>
int launch_rule(nmx_ctx *ctx, const nmx_lin_args &a) {
    /* 32 value columns (128 threads) per workgroup: several workgroups per head, each with
     * its state slice in VGPRs */
    const int jw = a.dv < 32 ? a.dv : 32;
    dim3 grid((unsigned)a.heads, (unsigned)((a.dv + jw - 1) / jw));
    dim3 block((unsigned)(4 * jw));
    const size_t lds = (2 * TB * 4 * (DK4 + 4) + 2 * TB) * sizeof(float);
    lin_rule_k<DK4><<<grid, block, lds, ctx->stream>>>(a);
    NMX_LAUNCHED(ctx, "lin_rule");
    return 0;
}

int validate(nmx_ctx *ctx, const nmx_lin_args *a, const char *what) {
    if (!a) return nmx_fail(ctx, "%s: NULL args", what);
    if (a->heads < 1 || a->heads > 256 || a->rep < 1 || a->heads % a->rep || a->dv < 1 ||
        a->dv > 1024 || a->n < 0 || a->n > 64 || a->keep < 0 || a->keep > 64)
        return nmx_fail(ctx, "%s: bad shape n=%d heads=%d rep=%d dk=%d dv=%d keep=%d", what, a->n,
                        a->heads, a->rep, a->dk, a->dv, a->keep);
    if (a->dk != 32 && a->dk != 64 && a->dk != 128 && a->dk != 256)
        return nmx_fail(ctx, "%s: dk=%d not supported (32, 64, 128, 256)", what, a->dk);
    if (!a->S) return nmx_fail(ctx, "%s: NULL state", what);
    if (a->keep > 0 && !a->pend) return nmx_fail(ctx, "%s: keep=%d without pend", what, a->keep);
    const size_t sb = (size_t)a->heads * a->dk * a->dv * 4;
    const size_t logw = (size_t)a->dk + a->dv + 1;
    if (a->keep > 0 && nmx_overlap(a->S, sb, a->pend, (size_t)a->keep * a->heads * logw * 4))
        return nmx_fail(ctx, "%s: state aliases pend", what);
    if (a->n > 0) {
        const int kd = (a->heads / a->rep) * a->dk;
        if (!a->qkv || !a->decay || !a->beta || !a->o)
            return nmx_fail(ctx, "%s: NULL input/output", what);
        if (a->qkv_stride < 2 * kd + a->heads * a->dv || a->o_stride < a->heads * a->dv)
            return nmx_fail(ctx, "%s: bad strides qkv=%d o=%d", what, a->qkv_stride, a->o_stride);
        const size_t ob = ((size_t)(a->n - 1) * a->o_stride + (size_t)a->heads * a->dv) * 4;
        const size_t qb = ((size_t)(a->n - 1) * a->qkv_stride + 2 * kd + (size_t)a->heads * a->dv) * 4;
        if (nmx_overlap(a->o, ob, a->S, sb) || nmx_overlap(a->o, ob, a->qkv, qb))
            return nmx_fail(ctx, "%s: output aliases state or input", what);
        if (a->log) {
            const size_t lb = (size_t)a->n * a->heads * logw * 4;
            if (nmx_overlap(a->log, lb, a->S, sb) || nmx_overlap(a->log, lb, a->o, ob) ||
                nmx_overlap(a->log, lb, a->qkv, qb) ||
                (a->keep > 0 && nmx_overlap(a->log, lb, a->pend, (size_t)a->keep * a->heads * logw * 4)))
                return nmx_fail(ctx, "%s: log aliases another buffer", what);
        }
    }
    return 0;
}

int dispatch(nmx_ctx *ctx, const nmx_lin_args &a) {
    switch (a.dk) {
    case 32: return launch_rule<8>(ctx, a);
    case 64: return launch_rule<16>(ctx, a);
    case 128: return launch_rule<32>(ctx, a);
    default: return launch_rule<64>(ctx, a);
    }
}

} // namespace

extern "C" {

int nmx_lin_rule(nmx_ctx *ctx, const nmx_lin_args *a) {
    if (!ctx) return -1;
    if (validate(ctx, a, "nmx_lin_rule")) return -1;
    if (a->n < 1) return nmx_fail(ctx, "nmx_lin_rule: n=%d (>= 1 needed)", a->n);
    return dispatch(ctx, *a);
}

size_t nmx_state_index(int h, int j, int i, int dk, int dv) { return state_index(h, j, i, dk, dv); }

int nmx_lin_apply(nmx_ctx *ctx, float *S, const float *log, int keep, int heads, int dk, int dv) {
    if (!ctx) return -1;
    if (keep == 0) return 0;
    nmx_lin_args a = {};
    a.n = 0;
    a.heads = heads;
    a.rep = 1;
    a.dk = dk;
    a.dv = dv;
    a.S = S;
    a.pend = log;
    a.keep = keep;
    if (validate(ctx, &a, "nmx_lin_apply")) return -1;
    return dispatch(ctx, a);
}

} /* extern "C" */
