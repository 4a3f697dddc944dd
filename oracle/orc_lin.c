/* ORACLE — test infrastructure only (see oracle.h). Gated DeltaNet recurrence with the
 * speculative rollback log, restating engine/src/matvec_ref.c:114-188. */
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

/* One head, one token (matvec_ref.c:114-136). S [dk][dv]:
 *   pass 1, i ascending: S_ij = S_ij * decay; kv_j = kv_j + S_ij * k_i
 *   delta_j = (v_j - kv_j) * beta
 *   pass 2, i ascending: S_ij = S_ij + k_i * delta_j; o_j = o_j + S_ij * q_i
 * Every operation rounds separately (no fused multiply-add). delta is left in tmp. */
static void delta_rule(float *S, const float *q, const float *k, const float *v, float decay,
                       float beta, float *o, float *tmp, int dk, int dv) {
    float *kv = tmp;
    for (int j = 0; j < dv; j++) kv[j] = 0.0f;
    for (int i = 0; i < dk; i++) {
        float *row = S + (size_t)i * dv;
        const float ki = k[i];
        for (int j = 0; j < dv; j++) {
            row[j] = row[j] * decay;
            kv[j] = kv[j] + row[j] * ki;
        }
    }
    for (int j = 0; j < dv; j++) kv[j] = (v[j] - kv[j]) * beta;
    for (int j = 0; j < dv; j++) o[j] = 0.0f;
    for (int i = 0; i < dk; i++) {
        float *row = S + (size_t)i * dv;
        const float ki = k[i], qi = q[i];
        for (int j = 0; j < dv; j++) {
            row[j] = row[j] + ki * kv[j];
            o[j] = o[j] + row[j] * qi;
        }
    }
}

/* Commit replay (matvec_ref.c:169-188): per logged row, row = row * decay; row = row + k_i *
 * delta_j — the same two roundings as the direct run, so replay == direct bit for bit. */
void orc_lin_apply(float *S, const float *log, int keep, int heads, int dk, int dv) {
    const size_t logw = (size_t)dk + dv + 1;
    for (int h = 0; h < heads; h++) {
        float *Sh = S + (size_t)h * dk * dv;
        for (int t = 0; t < keep; t++) {
            const float *u = log + ((size_t)t * heads + h) * logw;
            const float *d = u + dk, decay = u[dk + dv];
            for (int i = 0; i < dk; i++) {
                float *row = Sh + (size_t)i * dv;
                const float ki = u[i];
                for (int j = 0; j < dv; j++) {
                    row[j] = row[j] * decay;
                    row[j] = row[j] + ki * d[j];
                }
            }
        }
    }
}

/* Logged pass (matvec_ref.c:140-167 and the contract of engine/src/ops.h:54-93): the pending
 * updates first, then per head the tokens; with a log, token 0 stays in place and tokens
 * 1.. run on a copy of the head, their rows t >= 1 logged as k | delta | decay. log0 (no
 * reference counterpart): every token runs on the copy and row 0 is logged too. */
void orc_lin_rule(const orc_lin_args *a) {
    const int dk = a->dk, dv = a->dv, kd = (a->heads / a->rep) * dk;
    const size_t hs = (size_t)dk * dv, logw = (size_t)dk + dv + 1;
    float *tmp = malloc((size_t)dv * sizeof(float));
    float *work = malloc(hs * sizeof(float));
    if (a->keep > 0) orc_lin_apply(a->S, a->pend, a->keep, a->heads, dk, dv);
    for (int h = 0; h < a->heads; h++) {
        const int kh = h / a->rep;
        float *S = a->S + h * hs;
        for (int t = 0; t < a->n; t++) {
            if (a->log && t == (a->log0 ? 0 : 1)) {
                memcpy(work, S, hs * sizeof(float));
                S = work;
            }
            const float *qkv = a->qkv + (size_t)t * a->qkv_stride;
            const float *k = qkv + kd + kh * dk;
            const float decay = a->decay[(size_t)t * a->heads + h];
            delta_rule(S, qkv + kh * dk, k, qkv + 2 * kd + h * dv, decay,
                       a->beta[(size_t)t * a->heads + h], a->o + (size_t)t * a->o_stride + h * dv,
                       tmp, dk, dv);
            if (a->log && (t > 0 || a->log0)) {
                float *u = a->log + ((size_t)t * a->heads + h) * logw;
                memcpy(u, k, (size_t)dk * sizeof(float));
                memcpy(u + dk, tmp, (size_t)dv * sizeof(float));
                u[dk + dv] = decay;
            }
        }
    }
    free(work);
    free(tmp);
}
