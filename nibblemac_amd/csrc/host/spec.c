/* Speculative greedy decoding with the MTP head on the device (engine/src/spec.c:153-383,
 * restated for a device-resident model). One round with P = n_past and cur the newest token:
 *
 *   verify graph (one submit):  MTP chain d2..dk (d1 is ready from the last round), the
 *       logged main pass over [cur, d1..dk], the LM head fused with argmax + acceptance;
 *   host:  reads a and the tokens, emits them until a stop condition -> e (normally a + 1);
 *   commit graph (one submit):  cur <- vt[e], the rollback commit of every linear layer (conv
 *       state now, the e - 1 recurrent updates deferred to the next pass), the MTP head over
 *       the committed rows (next d1 and its hidden), n_past += e.
 *
 * Both graphs are captured once per draft count and replayed at any position (the kernels read
 * n_past, e and keep from the device control block). Tokens emitted equal plain greedy
 * decoding whatever the drafts are. */
#define _POSIX_C_SOURCE 200809L
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "engine.h"

#define CK(call)                                                                              \
    do {                                                                                      \
        if ((call) != 0) {                                                                    \
            fprintf(stderr, "pinfer: %s: %s\n", #call, nmx_error(c->dev));                    \
            return PINFER_E_ARG;                                                              \
        }                                                                                     \
    } while (0)
#define TRY(expr)                                                                             \
    do {                                                                                      \
        int rc_ = (expr);                                                                     \
        if (rc_ != PINFER_OK) return rc_;                                                     \
    } while (0)

void e_drop_graphs(pinfer_ctx *c) {
    for (int i = 0; i <= E_MAX_K; i++) {
        nmx_graph_destroy(c->g_verify[i]);
        nmx_graph_destroy(c->g_commit[i]);
        c->g_verify[i] = c->g_commit[i] = NULL;
    }
}

static int draft_vocab(const pinfer_ctx *c, const pinfer_spec_params *sp) {
    const int v = sp->draft_vocab; /* engine/src/spec.c:83-86 */
    return v >= 4 && v < c->vocab ? (v & ~3) : c->vocab;
}

/* ---- device sequences (captured into graphs) -------------------------------------------- */
static float *m_cur(pinfer_ctx *c) { return c->mbuf; }
static float *m_ping(pinfer_ctx *c, int i) { return c->mbuf + (size_t)(1 + (i & 1)) * c->H; }

/* MTP chain + verify pass + head/acceptance for ke drafts (engine/src/spec.c:303-345). */
static int seq_verify(pinfer_ctx *c, int ke, int nv) {
    for (int s = 1; s < ke; s++) {
        const float *h = s == 1 ? m_cur(c) : m_ping(c, s - 1);
        TRY(e_mtp_forward(c, h, c->vt + s, 1, s - 1, 0, nv, c->vt + s + 1, m_ping(c, s)));
    }
    TRY(e_forward(c, c->vt, ke + 1, 1));
    e_scratch *sc = &c->s;
    CK(nmx_head_accept(c->dev, c->head.w, c->vocab, c->H, ke + 1, sc->a_h.q, sc->a_h.d, sc->a_h.fs,
                       NULL, c->vt + 1, c->hwork, c->hout));
    CK(nmx_accept_commit(c->dev, c->hout, c->vt, c->ctl));
    return PINFER_OK;
}

/* Commit e = ctl[1] tokens and run the MTP head over them (engine/src/spec.c:346-365). */
static int seq_commit(pinfer_ctx *c, int ke, int nv) {
    CK(nmx_copy_token(c->dev, c->vt, c->ctl)); /* cur <- vt[e] */
    nmx_commit_args a = {c->n_lin, c->conv_dim, c->conv_k, c->conv_state, c->xin, c->log, c->pend,
                         c->cap, c->lv_heads * (c->lk_dim + c->lv_dim + 1), c->ctl};
    if (c->n_lin) CK(nmx_lin_commit(c->dev, &a));
    CK(nmx_copy_d2d(c->dev, c->hbuf, c->s.xn, (size_t)(ke + 1) * c->H * sizeof(float)));
    TRY(e_mtp_forward(c, c->hbuf, c->vt + 1, ke + 1, 0, 1, nv, c->vt + 1, m_cur(c)));
    CK(nmx_ctl_advance(c->dev, c->ctl));
    return PINFER_OK;
}

static int graph_for(pinfer_ctx *c, int ke, int nv, int commit, nmx_graph **out) {
    nmx_graph **slot = commit ? &c->g_commit[ke] : &c->g_verify[ke];
    if (c->graph_nv != nv) {
        e_drop_graphs(c);
        c->graph_nv = nv;
    }
    if (!*slot) {
        CK(nmx_graph_begin(c->dev));
        int rc = commit ? seq_commit(c, ke, nv) : seq_verify(c, ke, nv);
        nmx_graph *g = nmx_graph_end(c->dev);
        if (rc != PINFER_OK) {
            nmx_graph_destroy(g);
            return rc;
        }
        if (!g) {
            fprintf(stderr, "pinfer: graph capture failed: %s\n", nmx_error(c->dev));
            return PINFER_E_ARG;
        }
        *slot = g;
    }
    *out = *slot;
    return PINFER_OK;
}

static int run_seq(pinfer_ctx *c, int ke, int nv, int commit) {
    if (!c->use_graphs) return commit ? seq_commit(c, ke, nv) : seq_verify(c, ke, nv);
    nmx_graph *g;
    TRY(graph_for(c, ke, nv, commit, &g));
    CK(nmx_graph_launch(c->dev, g));
    return PINFER_OK;
}

/* ---- host driver ------------------------------------------------------------------------- */
typedef struct {
    int eos;
    const int32_t *stop_ids;
    int n_stop;
    int (*on_token)(int32_t, void *);
    void *user;
} e_stop;

/* engine/src/spec.c:205-215 */
static int emit(int32_t *out, int *count, int n_max, int32_t tok, const e_stop *sp) {
    out[(*count)++] = tok;
    int stop = *count >= n_max;
    if (sp->on_token && sp->on_token(tok, sp->user)) stop = 1;
    if (tok == sp->eos) stop = 1;
    for (int i = 0; i < sp->n_stop && !stop; i++) stop = tok == sp->stop_ids[i];
    return stop;
}

static int zero_mtp_rows(pinfer_ctx *c, int p0, int p1) {
    if (p1 <= p0) return PINFER_OK;
    for (int g = 0; g < c->n_kv; g++) {
        const size_t off = ((size_t)g * c->max_ctx + p0) * c->hd, len = (size_t)(p1 - p0) * c->hd * 4;
        CK(nmx_fill_zero(c->dev, c->mkc + off, len));
        CK(nmx_fill_zero(c->dev, c->mvc + off, len));
    }
    return PINFER_OK;
}

/* engine/src/spec.c:153-202: the prompt in chunks through the main model (final-normed rows
 * kept), then the MTP head over the same rows when k > 0 (row i pairs h_i with token i + 1, the
 * last row with the first generated token), leaving cur in vt[0], d1 in vt[1], its MTP hidden. */
static int prefill(pinfer_ctx *c, const int32_t *prompt, int n, int use_mtp, int nv) {
    const int base = c->n_past;
    if (use_mtp && c->mtp_rows < base) TRY(zero_mtp_rows(c, c->mtp_rows, base));
    int32_t next[E_MAX_BATCH];
    for (int c0 = 0; c0 < n; c0 += E_MAX_BATCH) {
        const int nb = n - c0 < E_MAX_BATCH ? n - c0 : E_MAX_BATCH, last = c0 + nb == n;
        CK(nmx_upload(c->dev, c->tok, prompt + c0, (size_t)nb * sizeof(int32_t)));
        TRY(e_set_pos(c, c->n_past));
        TRY(e_forward(c, c->tok, nb, 0));
        if (last) TRY(e_head_last(c, nb, c->vt, 0));
        if (use_mtp) {
            CK(nmx_copy_d2d(c->dev, c->hbuf, c->s.xn, (size_t)nb * c->H * sizeof(float)));
            for (int i = 0; i < nb; i++) next[i] = c0 + i + 1 < n ? prompt[c0 + i + 1] : 0;
            CK(nmx_upload(c->dev, c->tok, next, (size_t)nb * sizeof(int32_t)));
            if (last) CK(nmx_copy_d2d(c->dev, c->tok + nb - 1, c->vt, sizeof(int32_t)));
            TRY(e_mtp_forward(c, c->hbuf, c->tok, nb, 0, 0, nv, last ? c->vt + 1 : NULL,
                              last ? m_cur(c) : NULL));
        }
        c->n_past += nb;
    }
    TRY(e_set_pos(c, c->n_past));
    if (use_mtp) c->mtp_rows = c->n_past;
    return PINFER_OK;
}

/* Apply the deferred recurrent updates of the last commit (engine/src/forward_lin.c:207-216). */
static int lin_flush(pinfer_ctx *c) {
    if (c->keep <= 0) return PINFER_OK;
    const int logw = c->lk_dim + c->lv_dim + 1;
    for (int li = 0; li < c->n_lin; li++)
        CK(nmx_lin_apply(c->dev, c->rec + (size_t)li * c->lv_heads * c->lk_dim * c->lv_dim,
                         c->pend + (size_t)li * c->cap * c->lv_heads * logw, c->keep, c->lv_heads,
                         c->lk_dim, c->lv_dim));
    CK(nmx_ctl_set(c->dev, c->ctl, 2, 0));
    c->keep = 0;
    return PINFER_OK;
}

/* One plain step (engine/src/spec.c:238-262): cur through the model at n_past, argmax; with
 * the MTP head the final-normed row is kept for a later MTP pass. */
static int plain_step(pinfer_ctx *c, int use_mtp, int *pend_n, int *pend_pos, int32_t *pend_tok,
                      int32_t *next) {
    const int P = c->n_past;
    TRY(e_set_pos(c, P));
    TRY(e_forward(c, c->vt, 1, 0));
    c->keep = 0;
    TRY(e_head_last(c, 1, c->vt, 0));
    if (use_mtp) {
        if (*pend_n == 0) *pend_pos = P;
        CK(nmx_copy_d2d(c->dev, c->hbuf + (size_t)(E_MAX_BATCH - E_MAX_K - 2 + *pend_n) * c->H,
                        c->s.xn, (size_t)c->H * sizeof(float)));
    }
    CK(nmx_download(c->dev, next, c->vt, sizeof(int32_t)));
    if (use_mtp) pend_tok[(*pend_n)++] = *next;
    c->n_past = P + 1;
    TRY(e_set_pos(c, c->n_past));
    return PINFER_OK;
}

static int flush_pending(pinfer_ctx *c, int *pend_n, int pend_pos, const int32_t *pend_tok, int nv) {
    if (*pend_n == 0) return PINFER_OK;
    CK(nmx_upload(c->dev, c->tok, pend_tok, (size_t)*pend_n * sizeof(int32_t)));
    TRY(e_set_pos(c, pend_pos));
    TRY(e_mtp_forward(c, c->hbuf + (size_t)(E_MAX_BATCH - E_MAX_K - 2) * c->H, c->tok, *pend_n, 0,
                      0, nv, c->vt + 1, m_cur(c)));
    c->mtp_rows = pend_pos + *pend_n;
    *pend_n = 0;
    TRY(e_set_pos(c, c->n_past));
    return PINFER_OK;
}

static double now_sec(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + (double)ts.tv_nsec * 1e-9;
}

int e_generate_timed(pinfer_ctx *c, const int32_t *prompt, int n_prompt, int32_t *out,
                     int n_max, const pinfer_spec_params *sp_in, const pinfer_gen_opts *opts,
                     pinfer_spec_stats *st, int *status, int no_eos, double *t_prefill,
                     double *t_decode) {
    pinfer_spec_params plain = {0, 0, 0, 0};
    const pinfer_spec_params *sp = sp_in ? sp_in : &plain;
    int dummy;
    if (!status) status = &dummy;
    *status = PINFER_OK;
    if (!c || !out || n_max <= 0 || !prompt || n_prompt <= 0 || sp->k < 0 ||
        sp->k > PINFER_SPEC_MAX_K || sp->ngram < 0 || sp->ngram > PINFER_SPEC_MAX_K ||
        (opts && opts->n_stop > 0 && !opts->stop_ids))
        return *status = PINFER_E_ARG;
    if (sp->k > 0 && !c->has_mtp) return *status = PINFER_E_FORMAT;
    for (int i = 0; i < n_prompt; i++)
        if (prompt[i] < 0 || prompt[i] >= c->vocab) return *status = PINFER_E_ARG;
    if (n_prompt > c->max_ctx - c->n_past) return *status = PINFER_E_CTX_FULL;
    const int use_mtp = sp->k > 0, nv = draft_vocab(c, sp);
    e_stop stop = {no_eos ? -1 : c->eos, opts ? opts->stop_ids : NULL, opts ? opts->n_stop : 0,
                   opts ? opts->on_token : NULL, opts ? opts->user : NULL};
    const double t0 = now_sec();
    int rc = prefill(c, prompt, n_prompt, use_mtp, nv);
    if (rc != PINFER_OK) return *status = rc;
    int32_t cur;
    if (nmx_download(c->dev, &cur, c->vt, sizeof cur)) return *status = PINFER_E_ARG;
    const double t1 = now_sec();
    if (t_prefill) *t_prefill = t1 - t0;
    int count = 0, done = emit(out, &count, n_max, cur, &stop);
    int pend_n = 0, pend_pos = 0;
    int32_t pend_tok[E_MAX_K + 2];
    int32_t host[2 + E_MAX_BATCH], vt[E_MAX_K + 2];
    while (!done) {
        const int P = c->n_past;
        int left = n_max - count - 1;
        if (left > c->max_ctx - P - 1) left = c->max_ctx - P - 1;
        if (left < 0) {
            rc = PINFER_E_CTX_FULL;
            break;
        }
        const int ke = sp->k < left ? sp->k : left;
        if (ke == 0) {
            if (st && use_mtp) st->rounds++;
            if ((rc = plain_step(c, use_mtp, &pend_n, &pend_pos, pend_tok, &cur)) != PINFER_OK) break;
            done = emit(out, &count, n_max, cur, &stop);
            continue;
        }
        if ((rc = run_seq(c, ke, nv, 0)) != PINFER_OK) break;
        if (nmx_download(c->dev, host, c->hout, 2 * sizeof(int32_t)) ||
            nmx_download(c->dev, vt, c->vt, (size_t)(ke + 2) * sizeof(int32_t))) {
            rc = PINFER_E_ARG;
            break;
        }
        const int a = host[0];
        int e = 0;
        while (e <= a && !done) done = emit(out, &count, n_max, vt[++e], &stop);
        if (e != a + 1 && nmx_ctl_set(c->dev, c->ctl, 1, e)) {
            rc = PINFER_E_ARG;
            break;
        }
        if ((rc = run_seq(c, ke, nv, 1)) != PINFER_OK) break;
        c->n_past = P + e;
        c->keep = e - 1;
        c->mtp_rows = P + e;
        cur = vt[e];
        if (st) {
            st->rounds++;
            st->drafted += ke;
            st->accepted += a;
        }
    }
    if (rc == PINFER_OK && use_mtp) rc = flush_pending(c, &pend_n, pend_pos, pend_tok, nv);
    int frc = lin_flush(c);
    if (rc == PINFER_OK) rc = frc;
    if (nmx_sync(c->dev) && rc == PINFER_OK) rc = PINFER_E_ARG;
    if (t_decode) *t_decode = now_sec() - t1;
    *status = rc;
    return count;
}

int e_generate(pinfer_ctx *c, const int32_t *prompt, int n_prompt, int32_t *out, int n_max,
               const pinfer_spec_params *sp, const pinfer_gen_opts *opts,
               pinfer_spec_stats *st, int *status) {
    return e_generate_timed(c, prompt, n_prompt, out, n_max, sp, opts, st, status, 0, NULL, NULL);
}
