/* The Gated DeltaNet mixer of one verify pass in one launch for gfx950 (include/nmx.h
 * nmx_lin_mix): for every value head, the causal conv + SiLU of the head's q / k / v channels
 * with the conv state and the rollback inputs, the q / k L2 norms and the beta / decay gates
 * (engine/src/forward_lin.c:36-67, forward_ops.c:204-260), the recurrence with the pending
 * replays and the per-token log (matvec_ref.c:114-188), and the gated RMSNorm + A8 of the
 * output (forward_lin.c:70-81). Every value is computed with the same operations in the same
 * order as nmx_lin_pre, nmx_lin_rule and nmx_lin_post, so the results are identical; the conv
 * outputs, gates and o stay in LDS between the three stages instead of going through HBM and
 * three kernel boundaries.
 *
 * One workgroup per value head (one value head per key head, so every conv channel belongs to
 * one workgroup), 4 dv threads: the recurrence keeps the quad-per-column mapping
 * of nmx_lin_rule (lane c of the quad holds keys [c dk/4, (c+1) dk/4) of its column in VGPRs);
 * the conv stage has one thread per channel; the norms run as 4-lane ordered chains. */
#include "nmx_internal.h"
#include "nmx_math.h"
#include "nmx_a8.h"

namespace {

constexpr int MIX_TB = 8;          /* tokens per batch of conv-input loads; pending rows per batch */
constexpr int MIX_MAX_THREADS = 512;
constexpr int MIX_LDS = 157 * 1024; /* dynamic LDS: 160 KB less the static reduction array */

struct LinMix {
    /* pre */
    int n, C, K, kd;
    const float *raw;
    int raw_stride;
    float *state;
    const float *conv_w;
    float *xin;
    float qscale, l2eps;
    const float *b_in, *a_in;
    int g_stride;
    const float *A_log, *A, *dt_bias;
    /* rule */
    int heads, rep, dv;
    float *S;
    float *log;
    const float *pend;
    int keep, log0;
    const int32_t *keep_dev;
    /* post */
    const float *z;
    int z_stride;
    const float *w;
    float eps;
    float *y;
    int y_stride;
    int8_t *aq;
    float *ad, *afs;
};

__host__ __device__ constexpr int mix_lds_floats(int n, int dk, int dv) {
    /* q, k (rule layout [n][4][dk/4 + 4]), v, o [n][dv], pending keys [MIX_TB][4][dk/4 + 4],
     * pending deltas [MIX_TB][dv], z of the first tokens [MIX_TB][dv], norm weight [dv],
     * beta, decay [n], norm factors [3 n] (q, k L2; o RMS) */
    return 2 * n * 4 * (dk / 4 + 4) + 2 * n * dv + MIX_TB * 4 * (dk / 4 + 4) + 2 * MIX_TB * dv +
           dv + 5 * n;
}

template <int DK4>
__global__ __launch_bounds__(MIX_MAX_THREADS) void lin_mix_k(
    const float *__restrict__ raw, const float *__restrict__ z_in, const float *__restrict__ a_in,
    const float *__restrict__ b_in, int raw_stride, int z_stride, int g_stride, int kdim, int rep,
    int dv_, int n_, LinMix a) {
    extern __shared__ __align__(16) float sm[];
    __shared__ float red[8 * 64];
    __shared__ float spdec[MIX_TB]; /* decays of the pending batch (red serves the L2 norms) */
    __shared__ uint64_t sx2[32];    /* the gate exp's 2^(i/32) table */
    __shared__ float sgh[2];        /* the head's A (or A_log) and dt_bias */
    constexpr int DK = DK4 * 4, PAD = DK4 + 4, ROW = 4 * PAD;
    const int n = n_, dv = dv_, heads = a.heads;
    const int h = blockIdx.x, tid = threadIdx.x, T = 4 * dv, c = tid & 3; /* the launch's size */
    const int j = tid >> 2; /* value column of the quad (T = 4 dv) */
    const int kh = h / rep, kd = kdim;
    const size_t logw = (size_t)DK + dv + 1;
    const bool logged = a.log != nullptr;
    float *sq = sm, *sk = sq + n * ROW, *sv = sk + n * ROW, *so = sv + n * dv;
    float *sp = so + n * dv, *spd = sp + MIX_TB * ROW, *sz = spd + MIX_TB * dv;
    float *sw = sz + MIX_TB * dv, *sbet = sw + dv, *sdec = sbet + n, *srn = sdec + n;
    auto kidx = [](int i) { return (i / DK4) * PAD + i % DK4; }; /* rule layout of key i */
    const int n0 = n < MIX_TB ? n : MIX_TB; /* tokens whose inputs are requested at entry */

    /* ==== every input of the first batch is requested here, before any of it is used; the
     * recurrence state last, since loads complete in order and the state is needed only by
     * the pending replay, which runs after the conv, gates and L2 norms ==== */
    /* pending rows of the first batch, up to the host's bound on keep: keys (x = e T + tid
     * over [pb0][DK]), deltas (over [pb0][dv]), decays (tid < pb0) */
    const int pb0 = a.keep < MIX_TB ? a.keep : MIX_TB;
    float pkey[2], pdel[2], pdec = 0.0f;
#pragma unroll
    for (int e = 0; e < 2; e++) {
        const int x = e * T + tid, uk = x / DK, ik = x - uk * DK, ud = x / dv, jd = x - ud * dv;
        pkey[e] = 0.0f, pdel[e] = 0.0f;
        if (uk < pb0) pkey[e] = a.pend[((size_t)uk * heads + h) * logw + ik];
        if (ud < pb0) pdel[e] = a.pend[((size_t)ud * heads + h) * logw + DK + jd];
    }
    if (tid < pb0) pdec = a.pend[((size_t)tid * heads + h) * logw + DK + dv];
    /* conv: thread tid < nch owns channel tid (K = 4: 3 state rows, the taps as one float4) */
    const int nch = 2 * DK + dv, ci = tid;
    const bool conv_on = ci < nch;
    const int gc = ci < DK ? kh * DK + ci : ci < 2 * DK ? kd + kh * DK + (ci - DK)
                                                        : 2 * kd + h * dv + (ci - 2 * DK);
    float cwin[3], cx[MIX_TB];
    float4 cw = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int r = 0; r < 3; r++) cwin[r] = 0.0f;
    if (conv_on) {
#pragma unroll
        for (int r = 0; r < 3; r++) cwin[r] = a.state[(size_t)r * a.C + gc];
        cw = *(const float4 *)(a.conv_w + (size_t)gc * 4);
    }
#pragma unroll
    for (int u = 0; u < MIX_TB; u++) {
        cx[u] = 0.0f;
        if (conv_on && u < n0) cx[u] = raw[(size_t)u * raw_stride + gc];
    }
    /* gate items of the last wave, which owns no channel (y = tid - (T - 64)): item y < n is the
     * decay of token y, item n <= y < 2 n the beta of token y - n */
    const int gy = tid - (T - 64);
    float ga = 0.0f, gA = 0.0f, gdt = 0.0f;
    if (gy >= 0 && gy < n) {
        ga = a_in[(size_t)gy * g_stride + h];
        gA = a.A ? a.A[h] : a.A_log[h];
        gdt = a.dt_bias[h];
    } else if (gy >= n && gy < 2 * n) {
        ga = b_in[(size_t)(gy - n) * g_stride + h];
    }
    const uint64_t x2v = tid < 32 ? nmx_exp2_32[tid] : 0ull;
    /* z of the first tokens and the norm weight, as float4 (x4 = tid over [n0][dv / 4]) */
    const bool z_on = 4 * tid < n0 * dv, w_on = 4 * tid < dv;
    float4 zq = make_float4(0.f, 0.f, 0.f, 0.f), wq = zq;
    if (z_on) {
        const int t = (4 * tid) / dv, jj = 4 * tid - t * dv;
        zq = *(const float4 *)(z_in + (size_t)t * z_stride + h * dv + jj);
    }
    if (w_on) wq = *(const float4 *)(a.w + 4 * tid);
    /* recurrence state of the quad's keys */
    float *Sp = a.S + state_lane(h, j, c, DK, dv);
    const int SS = state_slot(j, dv); /* a wave's loads: one contiguous 1 KB run each */
    float s[DK4];
#pragma unroll
    for (int r = 0; r < DK4; r += 4) {
        const float4 x = *(const float4 *)(Sp + (r >> 2) * SS);
        s[r] = x.x, s[r + 1] = x.y, s[r + 2] = x.z, s[r + 3] = x.w;
    }

    /* pending rows to replay: the host's bound, or fewer from the device control block */
    int keep = a.keep;
    if (a.keep_dev) {
        const int kd_ = *a.keep_dev;
        keep = kd_ < keep ? kd_ : keep;
    }

    /* ---- requested values that later phases read from LDS ---- */
#pragma unroll
    for (int e = 0; e < 2; e++) {
        const int x = e * T + tid, uk = x / DK, ik = x - uk * DK, ud = x / dv;
        if (uk < pb0) sp[uk * ROW + kidx(ik)] = pkey[e];
        if (ud < pb0) spd[x] = pdel[e];
    }
    if (tid < pb0) spdec[tid] = pdec;
    if (z_on) *(float4 *)(sz + 4 * tid) = zq;
    if (w_on) *(float4 *)(sw + 4 * tid) = wq;
    if (tid < 32) sx2[tid] = x2v;
    if (gy == 0) sgh[0] = gA, sgh[1] = gdt;
    __syncthreads();

    /* ---- conv + SiLU of the head's channels: q (dk), k (dk), v (dv), one per thread ---- */
    if (conv_on) {
        float win[3];
        const float wc[4] = {cw.x, cw.y, cw.z, cw.w};
#pragma unroll
        for (int r = 0; r < 3; r++) win[r] = cwin[r];
        for (int t0 = 0; t0 < n; t0 += MIX_TB) {
            const int nb = n - t0 < MIX_TB ? n - t0 : MIX_TB;
            float xt[MIX_TB];
#pragma unroll
            for (int u = 0; u < MIX_TB; u++) xt[u] = cx[u];
            if (t0 > 0) {
#pragma unroll
                for (int u = 0; u < MIX_TB; u++)
                    xt[u] = u < nb ? raw[(size_t)(t0 + u) * raw_stride + gc] : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < MIX_TB; u++) {
                if (u >= nb) continue;
                const int t = t0 + u;
                /* taps in order over [state rows (oldest first), x_t] */
                float acc = wc[0] * win[0];
                acc = acc + wc[1] * win[1];
                acc = acc + wc[2] * win[2];
                acc = acc + wc[3] * xt[u];
                win[0] = win[1], win[1] = win[2], win[2] = xt[u];
                if (t == 0 && a.xin) { /* logged pass: token 0 is committed in place */
#pragma unroll
                    for (int q = 0; q < 3; q++) a.state[(size_t)q * a.C + gc] = win[q];
                }
                if (t > 0 && a.xin) a.xin[(size_t)t * a.C + gc] = xt[u];
                const float yv = nmx_silu(acc);
                if (ci < DK) sq[t * ROW + kidx(ci)] = yv;
                else if (ci < 2 * DK) sk[t * ROW + kidx(ci - DK)] = yv;
                else sv[t * dv + (ci - 2 * DK)] = yv;
            }
        }
        if (!a.xin) {
#pragma unroll
            for (int q = 0; q < 3; q++) a.state[(size_t)q * a.C + gc] = win[q];
        }
    }
    /* meanwhile the last wave computes the gates, beta = sigmoid(b) and
     * decay = exp(A softplus(a + dt_bias)) with A = -exp(A_log): each lane's first item from
     * the values requested at entry (the head's A and dt_bias through LDS, since a value
     * the compiler requests again here would be waited for behind the wave's recurrence
     * state), items past the wave (2 n > 64) in a loop of their own, whose loads would
     * otherwise make the first item's waits wait for every request in flight */
    auto gate = [&](int x, float g, float Ai, float dt) {
        if (x < n) {
            const float A = a.A ? Ai : -nmx_gate_expf_t(Ai, sx2);
            float sp_ = g + dt;
            sp_ = sp_ > 20.0f ? sp_ : nmx_gate_log1pf(nmx_gate_expf_t(sp_, sx2));
            sdec[x] = nmx_gate_expf_t(A * sp_, sx2);
        } else {
            sbet[x - n] = 1.0f / (1.0f + nmx_gate_expf_t(-g, sx2));
        }
    };
    if (gy >= 0 && 2 * n <= 63) {
        /* (the whole gate wave) each lane's first exponential in one call: exp(a + dt) in the
         * decay lanes, exp(-b) in the beta lanes and exp(A_log) in lane 63, which has no item;
         * then the betas' divide and the decays' log1p and last exponential. The decay chain
         * is two exponentials long instead of three, and the betas' exponential no longer runs
         * after it */
        const bool dl = gy < n, bl = gy >= n && gy < 2 * n;
        const float spv = ga + sgh[1];
        const float e1 = nmx_gate_expf_t(gy == 63 ? sgh[0] : dl ? spv : -ga, sx2);
        const float A =
            a.A ? sgh[0] : -__int_as_float(__builtin_amdgcn_readlane(__float_as_int(e1), 63));
        if (dl) {
            const float sp_ = spv > 20.0f ? spv : nmx_gate_log1pf(e1);
            sdec[gy] = nmx_gate_expf_t(A * sp_, sx2);
        } else if (bl) {
            sbet[gy - n] = 1.0f / (1.0f + e1);
        }
    } else if (gy >= 0 && gy < 2 * n) {
        gate(gy, ga, sgh[0], sgh[1]);
    }
    if (gy >= 0) {
        for (int x = gy + 64; x < 2 * n; x += 64) {
            const float g =
                x < n ? a_in[(size_t)x * g_stride + h] : b_in[(size_t)(x - n) * g_stride + h];
            gate(x, g, sgh[0], sgh[1]);
        }
    }
    __syncthreads();

    /* ---- q / k L2 norms (4 partial sums of squares + empty tail), q scaled ---- */
    for (int x = tid; x < 8 * n; x += T) {
        const int t = x >> 3, w = (x >> 2) & 1, l = x & 3;
        const float *v = (w ? sk : sq) + t * ROW;
        float cs = 0.0f;
#pragma unroll 8
        for (int m = 0; m < DK4; m++) {
            const float e = v[kidx(4 * m + l)];
            cs = cs + e * e;
        }
        red[x] = cs;
    }
    __syncthreads();
    for (int x = tid; x < 2 * n; x += T) { /* x = 2 t + w */
        const float *r4 = red + 4 * x;
        const float ss = ((r4[0] + r4[1]) + (r4[2] + r4[3])) + 0.0f;
        srn[x] = 1.0f / sqrtf(ss + a.l2eps);
    }
    __syncthreads();
    for (int x = tid; x < n * DK; x += T) {
        const int t = x / DK, i = x - t * DK;
#pragma unroll
        for (int w = 0; w < 2; w++) {
            float *v = (w ? sk : sq) + t * ROW + kidx(i);
            *v = (*v * srn[2 * t + w]) * (w ? 1.0f : a.qscale);
        }
    }
    __syncthreads();

    /* ---- the deferred commit of the previous pass (matvec_ref.c:169-188 arithmetic): the
     * state's rows, requested at entry, have arrived during the conv, gates and L2 norms;
     * the first batch of pending rows is in LDS since the first barrier ---- */
    for (int u0 = 0; u0 < keep; u0 += MIX_TB) {
        const int nb = keep - u0 < MIX_TB ? keep - u0 : MIX_TB;
        if (u0 > 0) { /* later batches (keep > MIX_TB) load here */
            float kb[2], db[2], dc = 0.0f;
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int x = e * T + tid, uk = x / DK, ik = x - uk * DK, ud = x / dv, jd = x - ud * dv;
                kb[e] = uk < nb ? a.pend[((size_t)(u0 + uk) * heads + h) * logw + ik] : 0.0f;
                db[e] = ud < nb ? a.pend[((size_t)(u0 + ud) * heads + h) * logw + DK + jd] : 0.0f;
            }
            if (tid < nb) dc = a.pend[((size_t)(u0 + tid) * heads + h) * logw + DK + dv];
            __syncthreads(); /* the previous batch is applied */
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int x = e * T + tid, uk = x / DK, ik = x - uk * DK, ud = x / dv;
                if (uk < nb) sp[uk * ROW + kidx(ik)] = kb[e];
                if (ud < nb) spd[x] = db[e];
            }
            if (tid < nb) spdec[tid] = dc;
            __syncthreads();
        }
#pragma unroll
        for (int u = 0; u < MIX_TB; u++) {
            if (u < nb) {
                const float pdec_ = spdec[u], pdel_ = spd[u * dv + j];
                const float *kk = sp + u * ROW + c * PAD;
#pragma unroll
                for (int r = 0; r < DK4; r++) {
                    s[r] = s[r] * pdec_;
                    s[r] = s[r] + kk[r] * pdel_;
                }
            }
        }
    }
    const bool store_now = a.log0 && keep > 0;
    if (store_now) {
#pragma unroll
        for (int r = 0; r < DK4; r += 4) *(float4 *)(Sp + (r >> 2) * SS) = make_float4(s[r], s[r + 1], s[r + 2], s[r + 3]);
    }

    /* ---- recurrence over the tokens (nmx_lin_rule arithmetic) ---- */
    for (int t = 0; t < n; t++) {
        const float *kk = sk + t * ROW + c * PAD, *qq = sq + t * ROW + c * PAD;
        const float dec = sdec[t], bet = sbet[t];
        float p[DK4];
#pragma unroll
        for (int r = 0; r < DK4; r++) {
            s[r] = s[r] * dec;
            p[r] = s[r] * kk[r];
        }
        const float kv = nmx_quad_chain<DK4>(p);
        const float del = (sv[t * dv + j] - kv) * bet;
#pragma unroll
        for (int r = 0; r < DK4; r++) {
            s[r] = s[r] + kk[r] * del;
            p[r] = s[r] * qq[r];
        }
        const float ov = nmx_quad_chain<DK4>(p);
        if (c == 0) so[t * dv + j] = ov;
        if (logged && (t > 0 || a.log0)) {
            float *lr = a.log + ((size_t)t * heads + h) * logw;
            if (c == 0) lr[DK + j] = del;
            for (int x = tid; x < DK; x += T) lr[x] = sk[t * ROW + kidx(x)];
            if (tid == 0) lr[DK + dv] = dec;
        }
        /* the committed state: after token 0 of a reference-mode logged pass, after the last
         * token of a plain pass */
        const bool commit = logged ? (!a.log0 && t == 0) : (t == n - 1);
        if (commit) {
#pragma unroll
            for (int r = 0; r < DK4; r += 4)
                *(float4 *)(Sp + (r >> 2) * SS) = make_float4(s[r], s[r + 1], s[r + 2], s[r + 3]);
        }
    }
    __syncthreads();

    /* ---- gated RMSNorm of o per token (4 partial sums of squares), * w * silu(z), A8 ---- */
    const int m4 = dv >> 2;
    for (int x = tid; x < 4 * n; x += T) {
        const int t = x >> 2, l = x & 3;
        const float *v = so + t * dv + l;
        float cs = 0.0f;
#pragma unroll 8
        for (int m = 0; m < m4; m++) cs = cs + v[4 * m] * v[4 * m];
        red[x] = cs;
    }
    __syncthreads();
    for (int t = tid; t < n; t += T) {
        const float *r4 = red + 4 * t;
        const float ss = ((r4[0] + r4[1]) + (r4[2] + r4[3])) + 0.0f;
        srn[2 * n + t] = 1.0f / sqrtf(ss / (float)dv + a.eps);
    }
    __syncthreads();
    auto out = [&](int x, float z) { /* a 32-lane half-wave holds one A8 block */
        const int t = x / dv, jj = x - t * dv;
        const float ov = so[t * dv + jj];
        const float gz = nmx_silu(z);
        float yv = (ov * srn[2 * n + t]) * sw[jj];
        yv = yv * gz;
        const int col = h * dv + jj;
        if (a.y) a.y[(size_t)t * a.y_stride + col] = yv;
        if (a.aq) {
            const size_t u = (size_t)(col >> 5) * n + t;
            nmx_a8_store(yv, a.aq + u * 32, a.ad + u, a.afs + u);
        }
    };
    /* items x and x + T together where both exist (the boundary n0 dv is a multiple of 32,
     * so each half-wave takes one branch): their chains interleave, where the threads with
     * two items ran them one after the other and ended the launch last */
    auto out2 = [&](int x1, float z1, int x2, float z2) {
        const int t1 = x1 / dv, j1 = x1 - t1 * dv, t2 = x2 / dv, j2 = x2 - t2 * dv;
        const float g1 = nmx_silu(z1), g2 = nmx_silu(z2);
        float y1 = (so[t1 * dv + j1] * srn[2 * n + t1]) * sw[j1];
        float y2 = (so[t2 * dv + j2] * srn[2 * n + t2]) * sw[j2];
        y1 = y1 * g1;
        y2 = y2 * g2;
        const int c1 = h * dv + j1, c2 = h * dv + j2;
        if (a.y) {
            a.y[(size_t)t1 * a.y_stride + c1] = y1;
            a.y[(size_t)t2 * a.y_stride + c2] = y2;
        }
        if (a.aq) {
            const size_t u1 = (size_t)(c1 >> 5) * n + t1, u2 = (size_t)(c2 >> 5) * n + t2;
            nmx_a8_store2(y1, a.aq + u1 * 32, a.ad + u1, a.afs + u1, y2, a.aq + u2 * 32,
                          a.ad + u2, a.afs + u2);
        }
    };
    /* z of the first n0 tokens from LDS, of later ones from memory, in two loops: one load
     * through a pointer that may be either is a generic load, and a wait for it waits for every
     * memory operation in flight, the state and log stores included */
    for (int x = tid; x < n0 * dv; x += 2 * T) {
        if (x + T < n0 * dv) out2(x, sz[x], x + T, sz[x + T]);
        else out(x, sz[x]);
    }
    for (int x = n0 * dv + tid; x < n * dv; x += T) {
        const int t = x / dv, jj = x - t * dv;
        out(x, z_in[(size_t)t * z_stride + h * dv + jj]);
    }
}

template <int DK4>
int launch_mix(nmx_ctx *ctx, const LinMix &m, size_t lds) {
    static bool ready = false; /* idempotent */
    if (!ready) {
        NMX_HIP(ctx, hipFuncSetAttribute((const void *)lin_mix_k<DK4>,
                                         hipFuncAttributeMaxDynamicSharedMemorySize, MIX_LDS));
        ready = true;
    }
    lin_mix_k<DK4><<<dim3((unsigned)m.heads), dim3((unsigned)(4 * m.dv)), lds, ctx->stream>>>(
        m.raw, m.z, m.a_in, m.b_in, m.raw_stride, m.z_stride, m.g_stride, m.kd, m.rep, m.dv, m.n, m);
    NMX_LAUNCHED(ctx, "lin_mix");
    return 0;
}

} // namespace

extern "C" {

int nmx_lin_mix(nmx_ctx *ctx, const nmx_lin_mix_args *a) {
    if (!ctx) return -1;
    if (!a) return nmx_fail(ctx, "nmx_lin_mix: NULL args");
    const nmx_lin_pre_args &p = a->pre;
    const nmx_lin_args &r = a->rule;
    const int n = p.n, dk = p.dk, dv = r.dv;
    if (n < 1 || n > 64 || n != r.n || dk != r.dk || p.heads != r.heads || !a->z || !a->norm_w ||
        a->z_stride < r.heads * dv || (a->y && a->y_stride < r.heads * dv) || dv % 32 ||
        p.kd != (r.heads / r.rep) * dk || p.C != 2 * p.kd + r.heads * dv)
        return nmx_fail(ctx, "nmx_lin_mix: inconsistent arguments");
    const size_t lds = (size_t)mix_lds_floats(n, dk, dv) * 4;
    /* one value head per key head: with shared key heads, a workgroup could read a shared
     * q / k channel's conv state after its owner committed token 0 into it */
    /* the fused kernel gives each thread of the first T - 64 one conv channel (the last wave
     * computes the gates: 2 dk + dv <= T - 64), a batch of
     * pending keys two elements per thread (dk <= dv), and reads z / w / the taps as float4:
     * K = 4, 16-byte aligned z, w and taps */
    auto al = [](const void *q, unsigned m) { return ((uintptr_t)q & (m - 1)) == 0; };
    const bool vec_ok = p.conv_k == 4 && a->z_stride % 4 == 0 && al(p.conv_w, 16) &&
                        al(a->z, 16) && al(a->norm_w, 16);
    const bool fused = r.rep == 1 && (dk == 64 || dk == 128) && 4 * dv <= MIX_MAX_THREADS &&
                       dk <= dv && 2 * dk + dv <= 4 * dv - 64 && lds <= MIX_LDS && vec_ok &&
                       !(r.log0 && !r.log);
    if (!fused) { /* the separate kernels, through the intermediate buffers of the structs */
        if (nmx_lin_pre(ctx, &p) || nmx_lin_rule(ctx, &r)) return -1;
        return nmx_lin_post(ctx, r.o, r.o_stride, a->z, a->z_stride, a->norm_w, n, r.heads, dv,
                            a->eps, a->y, a->y_stride, a->a8);
    }
    if (!p.raw || !p.state || !p.conv_w || !p.b_in || !p.a_in || !p.dt_bias ||
        (!p.A_log && !p.A) || !r.S || (r.keep > 0 && !r.pend) || p.raw_stride < p.C ||
        p.g_stride < p.heads || r.heads % r.rep || r.keep < 0 || r.keep > 64)
        return nmx_fail(ctx, "nmx_lin_mix: bad arguments");
    LinMix m{n, p.C, p.conv_k, p.kd, p.raw, p.raw_stride, p.state, p.conv_w, p.xin, p.qscale,
             p.l2eps, p.b_in, p.a_in, p.g_stride, p.A_log, p.A, p.dt_bias, r.heads, r.rep, dv,
             r.S, r.log, r.pend, r.keep, r.log0, r.keep_dev, a->z, a->z_stride, a->norm_w,
             a->eps, a->y, a->y_stride, a->a8.q, a->a8.d, a->a8.fs};
    return dk == 64 ? launch_mix<16>(ctx, m, lds) : launch_mix<32>(ctx, m, lds);
}

} /* extern "C" */
