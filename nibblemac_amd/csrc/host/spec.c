/* Speculative greedy decoding with the MTP head on the device (engine/src/spec.c:153-383,
 * restated for a device-resident model). One round with P = n_past and cur the newest token is
 * ONE graph launch:
 *
 *   MTP chain d2..dk (d1 is ready from the last round); the logged main pass over
 *   [cur, d1..dk]; the LM head fused with argmax + acceptance, which writes (a, tokens) to the
 *   host mailbox; the commit of e = a + 1 tokens (cur <- vt[e], the rollback commit of every
 *   linear layer: conv state now, the e - 1 recurrent updates deferred into the next pass); the
 *   MTP head over the committed rows (next d1 and its hidden); n_past += e.
 *
 * The host reads the mailbox while the graph's commit part still runs, emits the tokens and
 * launches the next round behind it, so the stream never drains between rounds. When a stop
 * condition ends the generation inside the accepted run (e < a + 1), one corrective commit is
 * enqueued after the graph: the linear layers' commit redone for e from the kept conv rows,
 * n_past and e set; the MTP rows past the stop are never read. Graphs are captured once per
 * draft count and replayed at any position (the kernels read n_past, e and keep from the
 * device control block). With pinfer_spec_params.ngram a round may instead draft by prompt
 * lookup (ngram.c, engine/src/spec.c:133-151): its graph has no MTP chain (the host uploads the
 * drafts) and no MTP pass (the committed rows wait, with those of plain steps, for one batched
 * MTP pass before the next MTP round, engine/src/spec.c:110-131). With
 * pinfer_spec_params.adaptive the draft count of each round (0: a plain step) comes from the
 * policy of adapt.c. Tokens emitted equal plain greedy decoding whatever the drafts are. */
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
        nmx_graph_destroy(c->g_round[i]);
        nmx_graph_destroy(c->g_round_ng[i]);
        c->g_round[i] = c->g_round_ng[i] = NULL;
    }
}

static int draft_vocab(const pinfer_ctx *c, const pinfer_spec_params *sp) {
    const int v = sp->draft_vocab; /* engine/src/spec.c:83-86 */
    return v >= 4 && v < c->vocab ? (v & ~3) : c->vocab;
}

/* ---- device sequences (captured into graphs) -------------------------------------------- */
static float *m_cur(pinfer_ctx *c) { return c->mbuf; }
static float *m_ping(pinfer_ctx *c, int i) { return c->mbuf + (size_t)(1 + (i & 1)) * c->H; }

static nmx_commit_args commit_args(pinfer_ctx *c, int redo) {
    nmx_commit_args a = {c->n_lin, c->conv_dim, c->conv_k, c->conv_state, c->xin, c->log, c->pend,
                         c->cap, c->lv_heads * (c->lk_dim + c->lv_dim + 1), c->ctl,
                         redo ? NULL : c->vt, c->conv_bak, redo};
    return a;
}

/* The logged main pass over vt[0..ke], the head with the acceptance of vt[1..ke] and the
 * commit of e = a + 1 (engine/src/spec.c:323-351, engine/src/forward_lin.c:185-204): (a, bonus,
 * vt) to the host mailbox, ctl[1] = e, cur <- vt[e], and the rollback commit of every linear
 * layer. With linear layers the head leaves partial argmax keys and every workgroup of the
 * commit resolves the acceptance itself (one launch fewer); without, the head's last kernel
 * does, and a kernel of its own sets cur. */
static int seq_verify_commit(pinfer_ctx *c, int ke, int keys_last) {
    TRY(e_forward(c, c->vt, ke + 1, 1, keys_last));
    e_scratch *sc = &c->s;
    const int n = ke + 1;
    if (c->n_lin && n <= 16) {
        CK(nmx_head_keys(c->dev, c->head.w, c->vocab, c->H, n, sc->a_h.q, sc->a_h.d, sc->a_h.fs,
                         c->vt + 1, c->hwork, c->dcopy));
        const nmx_commit_args a = commit_args(c, 0);
        const nmx_accept_keys k = {c->hwork, nmx_head_nkeys(c->vocab, c->H, n), n, c->dcopy,
                                   c->hout, c->mbox, ke + 2};
        CK(nmx_lin_commit_keys(c->dev, &a, &k));
        return PINFER_OK;
    }
    CK(nmx_head_accept_commit(c->dev, c->head.w, c->vocab, c->H, n, sc->a_h.q, sc->a_h.d,
                              sc->a_h.fs, c->vt + 1, c->hwork, c->hout, c->vt, c->ctl, c->mbox,
                              ke + 2));
    const nmx_commit_args a = commit_args(c, 0);
    if (c->n_lin) CK(nmx_lin_commit(c->dev, &a));
    else CK(nmx_copy_token(c->dev, c->vt, c->ctl));
    return PINFER_OK;
}

/* The linear layers' commit redone for a smaller e = ctl[1] from the conv rows the round's
 * commit kept, leaving vt alone (engine/src/forward_lin.c:185-204). */
static int commit_lin_redo(pinfer_ctx *c) {
    const nmx_commit_args a = commit_args(c, 1);
    if (c->n_lin) CK(nmx_lin_commit(c->dev, &a));
    return PINFER_OK;
}

/* One plain greedy step (engine/src/spec.c:238-262) at n_past = ctl[0]: cur = vt[0] through
 * the model, its argmax to vt[0] and the host mailbox, n_past += 1 on the device (every path
 * that changes n_past leaves ctl[0] equal to it, so a captured step needs no position upload).
 * The final-normed row stays in s.xn for the MTP pass the host may queue it for. */
static int seq_plain(pinfer_ctx *c) {
    TRY(e_forward(c, c->vt, 1, 0, 0));
    e_scratch *sc = &c->s;
    CK(nmx_head_step(c->dev, c->head.w, c->vocab, c->H, sc->a_h.q, sc->a_h.d, sc->a_h.fs,
                     c->hwork, c->hout, c->vt, c->ctl, c->mbox, 2));
    return PINFER_OK;
}

/* One MTP round of ke drafts (engine/src/spec.c:303-365): the chain d2..dk, the verify, the
 * commit of e = ctl[1], the MTP head over the committed rows (its hidden of row e - 1 and the
 * next d1; the pass reads the verify's final-normed rows, s.xn, which at hidden <= 1024 it
 * never writes, and otherwise writes only after its last read), n_past += e (done by the
 * pass's last kernel). The chain's drafts d2..dk pass as argmax keys: each one's consumer (the
 * next MTP pass, then the verify's first norm) resolves it and writes it to vt. */
static int seq_round(pinfer_ctx *c, int ke, int nv) {
    if (ke == 0) return seq_plain(c); /* a round without drafts: a plain step */
    const int keys = e_keys_ok(c);
    for (int s = 1; s < ke; s++) {
        const float *h = s == 1 ? m_cur(c) : m_ping(c, s - 1);
        const int io = keys ? E_KEYS_OUT | (s > 1 ? E_KEYS_IN : 0) : 0;
        TRY(e_mtp_forward(c, h, c->vt + s, 1, s - 1, 0, nv, c->vt + s + 1, m_ping(c, s), 0, io));
    }
    TRY(seq_verify_commit(c, ke, keys && ke > 1 ? nmx_head_row_nkeys(nv) : 0));
    TRY(e_mtp_forward(c, c->s.xn, c->vt + 1, ke + 1, 0, 1, nv, c->vt + 1, m_cur(c), 1, 0));
    return PINFER_OK;
}

/* One n-gram round (the host uploaded the drafts into vt[1..ke]): the verify, the commit,
 * n_past += e. The committed rows stay in s.xn for the host to queue for the MTP pass. */
static int seq_round_ng(pinfer_ctx *c, int ke) {
    TRY(seq_verify_commit(c, ke, 0));
    CK(nmx_ctl_advance(c->dev, c->ctl));
    return PINFER_OK;
}

static int graph_for(pinfer_ctx *c, int ke, int nv, int ng, nmx_graph **out) {
    nmx_graph **slot = ng ? &c->g_round_ng[ke] : &c->g_round[ke];
    if (c->graph_nv != nv) { /* a replay of the old graphs may still run: wait for it */
        CK(nmx_sync(c->dev));
        e_drop_graphs(c);
        c->graph_nv = nv;
    }
    if (!*slot) {
        CK(nmx_graph_begin(c->dev));
        int rc = ng ? seq_round_ng(c, ke) : seq_round(c, ke, nv);
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

/* Enqueue one round; its mailbox flag (mbox[2 + ke + 2]) is cleared first. */
static int launch_round(pinfer_ctx *c, int ke, int nv, int ng) {
    __atomic_store_n(c->mbox + 2 + ke + 2, 0, __ATOMIC_RELAXED);
    if (!c->use_graphs) return ng ? seq_round_ng(c, ke) : seq_round(c, ke, nv);
    nmx_graph *g;
    TRY(graph_for(c, ke, nv, ng, &g));
    CK(nmx_graph_launch(c->dev, g));
    return PINFER_OK;
}

/* A stop inside the accepted run: commit e (< a + 1) instead of the device's a + 1, after the
 * round on the stream: ctl[1] = e, the linear layers' commit redone from the kept conv rows,
 * ctl[0] = P + e, cur = the host's vt[e] (the round's MTP pass has overwritten vt[1]). */
static int recommit(pinfer_ctx *c, int P, int e, int32_t cur, int e_device) {
    /* the device's commit of e = 1 keeps no conv rows (nmx_commit_args): a redo needs e >= 2 */
    if (e < 1 || e >= e_device || e_device < 2) return PINFER_E_ARG;
    CK(nmx_ctl_set(c->dev, c->ctl, 1, e));
    TRY(commit_lin_redo(c));
    CK(nmx_ctl_set(c->dev, c->ctl, 0, P + e));
    CK(nmx_upload(c->dev, c->vt, &cur, sizeof cur));
    return PINFER_OK;
}

static double now_sec(void);

/* Waits for a round's mailbox flag (mbox[2 + ke + 2], set by the accept kernel with a
 * system-scope release): a spin on the host copy, then, after 2 s, the stream
 * synchronisation, which also reports a failed launch. */
static int wait_mailbox(pinfer_ctx *c, int ke) {
    const int32_t *flag = c->mbox + 2 + ke + 2;
    const double t0 = now_sec();
    for (long spins = 0; !__atomic_load_n(flag, __ATOMIC_ACQUIRE); spins++)
        if ((spins & 1023) == 1023 && now_sec() - t0 > 2.0) {
            if (nmx_sync(c->dev)) return -1;
            return __atomic_load_n(flag, __ATOMIC_ACQUIRE) ? 0 : -1;
        }
    return 0;
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
    TRY(e_kv_zero_rows(c, c->mkc, p0, p1));
    return e_kv_zero_rows(c, c->mvc, p0, p1);
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
        TRY(e_forward(c, c->tok, nb, 0, 0));
        if (last) TRY(e_head_last(c, nb, c->vt, 0));
        if (use_mtp) {
            CK(nmx_copy_d2d(c->dev, c->hbuf, c->s.xn, (size_t)nb * c->H * sizeof(float)));
            for (int i = 0; i < nb; i++) next[i] = c0 + i + 1 < n ? prompt[c0 + i + 1] : 0;
            CK(nmx_upload(c->dev, c->tok, next, (size_t)nb * sizeof(int32_t)));
            if (last) CK(nmx_copy_d2d(c->dev, c->tok + nb - 1, c->vt, sizeof(int32_t)));
            TRY(e_mtp_forward(c, c->hbuf, c->tok, nb, 0, 0, nv, last ? c->vt + 1 : NULL,
                              last ? m_cur(c) : NULL, 0, 0));
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

/* Committed rows waiting for the MTP pass (plain steps, n-gram rounds), in c->pbuf:
 * rows [0, n) hold the final-normed hiddens of positions pos.., tok the tokens after them
 * (engine/src/spec.c:110-131). */
typedef struct {
    int n, pos;
    int32_t tok[E_MAX_BATCH];
} e_pending;

/* The MTP pass over the pending rows (leaves d1 in vt[1], its hidden in m_cur). */
static int flush_pending(pinfer_ctx *c, e_pending *pd, int nv) {
    if (pd->n == 0) return PINFER_OK;
    CK(nmx_upload(c->dev, c->tok, pd->tok, (size_t)pd->n * sizeof(int32_t)));
    TRY(e_set_pos(c, pd->pos));
    TRY(e_mtp_forward(c, c->pbuf, c->tok, pd->n, 0, 0, nv, c->vt + 1, m_cur(c), 0, 0));
    c->mtp_rows = pd->pos + pd->n;
    pd->n = 0;
    TRY(e_set_pos(c, c->n_past));
    return PINFER_OK;
}

/* Queue the first m rows of s.xn (positions pos..) with the tokens that follow them. */
static int defer_rows(pinfer_ctx *c, e_pending *pd, const int32_t *tok, int m, int pos) {
    if (pd->n == 0) pd->pos = pos;
    CK(nmx_copy_d2d(c->dev, c->pbuf + (size_t)pd->n * c->H, c->s.xn,
                    (size_t)m * c->H * sizeof(float)));
    memcpy(pd->tok + pd->n, tok, (size_t)m * sizeof(int32_t));
    pd->n += m;
    return PINFER_OK;
}

/* One plain step (engine/src/spec.c:238-262): cur through the model at n_past, argmax; with
 * the MTP head the final-normed row is queued for a later MTP pass. With graphs the step is
 * one launch (the round graph of 0 drafts) whose head writes the token to the mailbox. */
static int plain_step(pinfer_ctx *c, int use_mtp, e_pending *pd, int nv, int32_t *next) {
    const int P = c->n_past;
    if (use_mtp && pd->n == E_MAX_BATCH) TRY(flush_pending(c, pd, nv));
    if (c->use_graphs) {
        TRY(launch_round(c, 0, nv, 0));
        if (wait_mailbox(c, 0)) return PINFER_E_ARG;
        *next = c->mbox[1];
    } else {
        TRY(e_set_pos(c, P));
        TRY(seq_plain(c));
        CK(nmx_download(c->dev, next, c->vt, sizeof(int32_t)));
    }
    c->keep = 0;
    if (use_mtp) TRY(defer_rows(c, pd, next, 1, P));
    e_ngram_push(&c->ng, next, 1);
    c->n_past = P + 1;
    return PINFER_OK;
}

/* The n-gram draft of the coming round (engine/src/spec.c:133-151): its length, or 0 for MTP
 * drafts / a plain step. A match of E_NG_ASK..E_NG_TRUST-1 tokens must start with the MTP
 * head's d1, which may need the pending rows' MTP pass first. */
static int ngram_pick(pinfer_ctx *c, const pinfer_spec_params *sp, int left, int32_t *d,
                      e_pending *pd, int nv, int *rc) {
    int match = 0;
    const int max = sp->ngram < left ? sp->ngram : left;
    const int n = max > 0 ? e_ngram_draft(&c->ng, d, max, &match) : 0;
    if (n == 0) return 0;
    if (match >= E_NG_TRUST) return n;
    if (sp->k == 0) return n < E_NG_SHORT ? n : E_NG_SHORT; /* no MTP head to ask */
    if (match < E_NG_ASK) return 0;
    if (pd->n > 0 && (*rc = flush_pending(c, pd, nv)) != PINFER_OK) return 0;
    int32_t d1;
    if (nmx_download(c->dev, &d1, c->vt + 1, sizeof d1)) {
        *rc = PINFER_E_ARG;
        return 0;
    }
    if (d[0] != d1) return 0;
    return n < E_NG_SHORT ? n : E_NG_SHORT;
}

static double now_sec(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + (double)ts.tv_nsec * 1e-9;
}

int e_generate_timed(pinfer_ctx *c, const int32_t *prompt, int n_prompt, int32_t *out,
                     int n_max, const pinfer_spec_params *sp_in, const pinfer_gen_opts *opts,
                     pinfer_spec_stats *st, int *status, int no_eos, int append,
                     double *t_prefill, double *t_decode) {
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
    const int drafting = sp->k > 0 || sp->ngram > 0;
    const int adaptive = sp->adaptive && drafting;
    e_stop stop = {no_eos ? -1 : c->eos, opts ? opts->stop_ids : NULL, opts ? opts->n_stop : 0,
                   opts ? opts->on_token : NULL, opts ? opts->user : NULL};
    /* the n-gram history is the fed tokens plus the last emitted one, with which a continuation
     * prompt leads; any other context starts a new history (engine/src/spec.c:165-170) */
    if (append && c->ng.n == c->n_past + 1) e_ngram_pop(&c->ng);
    else e_ngram_reset(&c->ng);
    e_ngram_push(&c->ng, prompt, n_prompt);
    const double t0 = now_sec();
    int rc = prefill(c, prompt, n_prompt, use_mtp, nv);
    if (rc != PINFER_OK) return *status = rc;
    int32_t cur;
    if (nmx_download(c->dev, &cur, c->vt, sizeof cur)) return *status = PINFER_E_ARG;
    e_ngram_push(&c->ng, &cur, 1);
    const double t1 = now_sec();
    if (t_prefill) *t_prefill = t1 - t0;
    int count = 0, done = emit(out, &count, n_max, cur, &stop);
    e_pending pd;
    pd.n = pd.pos = 0;
    e_adapt ad;
    e_adapt_init(&ad, sp->k > 0 ? sp->k : sp->ngram);
    double t_last = now_sec(); /* end of the last round: a round's cost runs to its results */
    int32_t vt[E_MAX_K + 2];
    while (!done) {
        const int P = c->n_past;
        int left = n_max - count - 1;
        if (left > c->max_ctx - P - 1) left = c->max_ctx - P - 1;
        if (left < 0) {
            rc = PINFER_E_CTX_FULL;
            break;
        }
        /* drafts wanted: the adaptive policy's width - 1 (0: a plain step), else k; prompt
         * lookup first, else MTP drafts (engine/src/spec.c:300-312) */
        const int want = adaptive ? e_adapt_width(&ad) - 1 : sp->k;
        int ke = 0, use_ng = 0;
        if (sp->ngram > 0 && left > 0 && !(adaptive && want == 0)) {
            ke = ngram_pick(c, sp, left, vt + 1, &pd, nv, &rc);
            if (rc != PINFER_OK) break;
            use_ng = ke > 0;
        }
        if (!use_ng && use_mtp) ke = want < left ? want : left;
        if (ke == 0) {
            if (st && drafting) st->rounds++;
            if ((rc = plain_step(c, use_mtp, &pd, nv, &cur)) != PINFER_OK) break;
            const double t = now_sec();
            if (adaptive) e_adapt_observe(&ad, 1, 0, t - t_last);
            t_last = t;
            done = emit(out, &count, n_max, cur, &stop);
            continue;
        }
        if (use_ng) {
            /* room for this round's rows among the pending ones */
            if (use_mtp && pd.n + ke + 1 > E_MAX_BATCH && (rc = flush_pending(c, &pd, nv)) != PINFER_OK)
                break;
            if (nmx_upload(c->dev, c->vt + 1, vt + 1, (size_t)ke * sizeof(int32_t))) {
                rc = PINFER_E_ARG;
                break;
            }
        } else if ((rc = flush_pending(c, &pd, nv)) != PINFER_OK) { /* d1 current */
            break;
        }
        if ((rc = launch_round(c, ke, nv, use_ng)) != PINFER_OK) break;
        if (wait_mailbox(c, ke)) { /* the verify wrote (a, bonus, vt) to the host mailbox */
            rc = PINFER_E_ARG;
            break;
        }
        const int a = c->mbox[0];
        memcpy(vt, c->mbox + 2, (size_t)(ke + 2) * sizeof(int32_t));
        int e = 0;
        while (e <= a && !done) done = emit(out, &count, n_max, vt[++e], &stop);
        if (e != a + 1 && (rc = recommit(c, P, e, vt[e], a + 1)) != PINFER_OK) break;
        if (use_ng) {
            if (use_mtp && (rc = defer_rows(c, &pd, vt + 1, e, P)) != PINFER_OK) break;
        } else {
            c->mtp_rows = P + e;
        }
        c->n_past = P + e;
        c->keep = e - 1;
        cur = vt[e];
        e_ngram_push(&c->ng, vt + 1, e);
        if (st) {
            st->rounds++;
            st->drafted += ke;
            st->accepted += a;
            if (use_ng) {
                st->ngram_rounds++;
                st->ngram_drafted += ke;
                st->ngram_accepted += a;
            }
        }
        const double t = now_sec();
        /* prompt-lookup rounds cost and accept differently from MTP rounds of the same width:
         * they stay out of the MTP width model */
        if (adaptive && !use_ng) e_adapt_observe(&ad, ke + 1, a, t - t_last);
        t_last = t;
    }
    if (rc == PINFER_OK && use_mtp) rc = flush_pending(c, &pd, nv);
    int frc = lin_flush(c);
    if (rc == PINFER_OK) rc = frc;
    if (nmx_sync(c->dev) && rc == PINFER_OK) rc = PINFER_E_ARG;
    if (t_decode) *t_decode = now_sec() - t1;
    *status = rc;
    return count;
}

int e_generate(pinfer_ctx *c, const int32_t *prompt, int n_prompt, int32_t *out, int n_max,
               const pinfer_spec_params *sp, const pinfer_gen_opts *opts,
               pinfer_spec_stats *st, int *status, int append) {
    return e_generate_timed(c, prompt, n_prompt, out, n_max, sp, opts, st, status, 0, append,
                            NULL, NULL);
}
