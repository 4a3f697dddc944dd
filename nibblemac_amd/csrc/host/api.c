/* Public API (include/pinfer.h) of the MI355X engine: context allocation on the device,
 * reset, eval, greedy / speculative generation. The reference's counterparts are
 * engine/src/pinfer.c (load, reset, eval, argmax, version) and engine/src/spec.c:385-439
 * (spec params, generate). */
#define _GNU_SOURCE
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "engine.h"

#define STR2(x) #x
#define STR(x) STR2(x)

pinfer_params pinfer_default_params(void) {
    pinfer_params p = {4, 4096, PINFER_KV_F32, 0.0f};
    return p;
}

const char *pinfer_version(void) {
    return STR(PINFER_VERSION_MAJOR) "." STR(PINFER_VERSION_MINOR) "." STR(PINFER_VERSION_PATCH);
}

pinfer_spec_params pinfer_default_spec_params(void) {
    pinfer_spec_params p = {4, 32768, 1, 7}; /* engine/src/spec.c:385-391 */
    return p;
}

static void *dalloc(pinfer_ctx *c, size_t bytes, int *ok) {
    if (!*ok) return NULL;
    if (c->n_allocs == E_MAX_ALLOCS) {
        *ok = 0;
        return NULL;
    }
    void *p = nmx_alloc(c->dev, bytes ? bytes : 4);
    if (p) c->allocs[c->n_allocs++] = p;
    if (!p || nmx_fill_zero(c->dev, p, bytes ? bytes : 4)) {
        *ok = 0;
        return NULL;
    }
    return p;
}

static nmx_a8 a8_alloc(pinfer_ctx *c, int width, int rows, int *ok) {
    nmx_a8 a;
    a.q = dalloc(c, (size_t)rows * width, ok);
    a.d = dalloc(c, (size_t)rows * (width / 32) * 4, ok);
    a.fs = dalloc(c, (size_t)rows * (width / 32) * 4, ok);
    return a;
}

static int imax(int a, int b) { return a > b ? a : b; }

/* engine/src/forward.c:19-32 (cos / sin tables): inv = 1 / theta^(2i / rot) and
 * angle = (float)pos * inv in binary32 with the host libm, for every position. */
static int rope_tables(pinfer_ctx *c, int *ok) {
    const int h = c->rot / 2, P = c->max_ctx;
    float *cs = malloc((size_t)P * (h ? h : 1) * 4), *sn = malloc((size_t)P * (h ? h : 1) * 4);
    if (!cs || !sn) {
        free(cs);
        free(sn);
        return PINFER_E_NOMEM;
    }
    for (int i = 0; i < h; i++) {
        const float inv = 1.0f / powf(c->rope_theta, (float)(2 * i) / (float)c->rot);
        for (int p = 0; p < P; p++) {
            const float ang = (float)p * inv;
            cs[(size_t)p * h + i] = cosf(ang);
            sn[(size_t)p * h + i] = sinf(ang);
        }
    }
    c->rope_cos = dalloc(c, (size_t)P * (h ? h : 1) * 4, ok);
    c->rope_sin = dalloc(c, (size_t)P * (h ? h : 1) * 4, ok);
    if (*ok && h) {
        if (nmx_upload(c->dev, c->rope_cos, cs, (size_t)P * h * 4) ||
            nmx_upload(c->dev, c->rope_sin, sn, (size_t)P * h * 4))
            *ok = 0;
    }
    free(cs);
    free(sn);
    return *ok ? PINFER_OK : PINFER_E_NOMEM;
}

static int alloc_state(pinfer_ctx *c) {
    int ok = 1;
    const int B = E_MAX_BATCH, H = c->H, S = c->conv_k - 1;
    const size_t logw = (size_t)c->lk_dim + c->lv_dim + 1;
    c->cap = E_MAX_K + 1;
    c->conv_state = dalloc(c, (size_t)imax(c->n_lin, 1) * (S ? S : 1) * c->conv_dim * 4, &ok);
    c->conv_bak = dalloc(c, (size_t)imax(c->n_lin, 1) * (S ? S : 1) * c->conv_dim * 4, &ok);
    c->rec = dalloc(c, (size_t)imax(c->n_lin, 1) * c->lv_heads * c->lk_dim * c->lv_dim * 4, &ok);
    c->kv_bytes = nmx_kv_bytes(c->kv_dtype, c->n_kv, c->max_ctx, c->hd);
    if (!c->kv_bytes) return PINFER_E_ARG;
    c->kc = dalloc(c, (size_t)imax(c->n_full, 1) * c->kv_bytes, &ok);
    c->vc = dalloc(c, (size_t)imax(c->n_full, 1) * c->kv_bytes, &ok);
    c->mkc = dalloc(c, c->kv_bytes, &ok);
    c->mvc = dalloc(c, c->kv_bytes, &ok);
    c->xin = dalloc(c, (size_t)imax(c->n_lin, 1) * c->cap * c->conv_dim * 4, &ok);
    c->log = dalloc(c, (size_t)imax(c->n_lin, 1) * c->cap * c->lv_heads * logw * 4, &ok);
    c->pend = dalloc(c, (size_t)imax(c->n_lin, 1) * c->cap * c->lv_heads * logw * 4, &ok);
    e_scratch *s = &c->s;
    const int qw = 2 * c->n_heads * c->hd, kvw = c->n_kv * c->hd;
    const int wa = imax(imax(c->conv_dim, qw), imax(c->ffn, 2 * H));
    const int wb = imax(imax(c->vd, kvw), c->ffn);
    const int wide = imax(imax(c->vd, c->n_heads * c->hd), 2 * H);
    s->x = dalloc(c, (size_t)B * H * 4, &ok);
    s->x2 = dalloc(c, (size_t)B * H * 4, &ok);
    s->xn = dalloc(c, (size_t)B * H * 4, &ok);
    s->out = dalloc(c, (size_t)B * H * 4, &ok);
    s->ta = dalloc(c, (size_t)B * wa * 4, &ok);
    s->tb = dalloc(c, (size_t)B * wb * 4, &ok);
    s->tc = dalloc(c, (size_t)B * kvw * 4, &ok);
    s->to = dalloc(c, (size_t)B * imax(c->vd, c->n_heads * c->hd) * 4, &ok);
    s->conv = dalloc(c, (size_t)B * c->conv_dim * 4, &ok);
    s->ba = dalloc(c, (size_t)B * c->lv_heads * 4, &ok);
    s->aa = dalloc(c, (size_t)B * c->lv_heads * 4, &ok);
    s->beta = dalloc(c, (size_t)B * c->lv_heads * 4, &ok);
    s->decay = dalloc(c, (size_t)B * c->lv_heads * 4, &ok);
    s->cat = dalloc(c, (size_t)B * 2 * H * 4, &ok);
    s->emb = dalloc(c, (size_t)B * H * 4, &ok);
    s->sc = dalloc(c, (size_t)B * imax(c->n_heads, 1) * c->max_ctx * 4, &ok);
    s->row1 = dalloc(c, (size_t)H * 4, &ok);
    s->a_h = a8_alloc(c, H, B, &ok);
    s->a_w = a8_alloc(c, wide, B, &ok);
    s->a_f = a8_alloc(c, c->ffn, B, &ok);
    s->a_1 = a8_alloc(c, H, 1, &ok);
    c->hbuf = dalloc(c, (size_t)B * H * 4, &ok);
    c->pbuf = dalloc(c, (size_t)B * H * 4, &ok);
    c->mbuf = dalloc(c, (size_t)3 * H * 4, &ok);
    c->ctl = dalloc(c, 16 * 4, &ok);
    c->vt = dalloc(c, (E_MAX_K + 2) * 4, &ok);
    c->tok = dalloc(c, B * 4, &ok);
    c->hout = dalloc(c, (2 + B) * 4, &ok);
    c->hout2 = dalloc(c, 4 * 4, &ok);
    c->dcopy = dalloc(c, (E_MAX_K + 2) * 4, &ok);
    c->mbox = ok ? (int32_t *)nmx_host_alloc(c->dev, (2 + E_MAX_K + 2 + 1) * sizeof(int32_t)) : NULL;
    if (!c->mbox) ok = 0;
    c->hwork = dalloc(c, nmx_head_work_bytes(c->vocab, E_MAX_K + 1), &ok);
    c->logits = dalloc(c, (size_t)c->vocab * 4, &ok);
    if (!ok || e_ngram_init(&c->ng, c->max_ctx + 1)) return PINFER_E_NOMEM;
    return rope_tables(c, &ok);
}

pinfer_ctx *pinfer_load(const char *path, const pinfer_params *params, int *err) {
    pinfer_params p = params ? *params : pinfer_default_params();
    if (p.max_ctx <= 0) p.max_ctx = 4096;
    int rc = PINFER_OK;
    pinfer_ctx *c = NULL;
    if (!path) rc = PINFER_E_ARG;
    else if (!isfinite(p.gpu_split) || p.gpu_split < 0.0f || p.gpu_split > 1.0f) rc = PINFER_E_ARG;
    else if (p.kv_dtype != PINFER_KV_F32 && p.kv_dtype != PINFER_KV_F16 &&
             p.kv_dtype != PINFER_KV_I8)
        rc = PINFER_E_ARG;
    else if (p.max_ctx > (1 << 20)) {
        fprintf(stderr, "pinfer: max_ctx %d above the attention kernels' 1048576\n", p.max_ctx);
        rc = PINFER_E_ARG;
    } else if ((rc = e_model_check(path)) != PINFER_OK) {
        /* refused before any device call */
    } else if (!(c = calloc(1, sizeof *c))) rc = PINFER_E_NOMEM;
    if (rc == PINFER_OK) {
        const char *dv = getenv("PINFER_DEVICE");
        c->dev = nmx_create(dv ? atoi(dv) : 0);
        if (!c->dev) {
            fprintf(stderr, "pinfer: %s\n", nmx_create_error());
            rc = PINFER_E_NOMEM;
        }
    }
    if (rc == PINFER_OK) {
        c->max_ctx = p.max_ctx;
        c->kv_dtype = p.kv_dtype;
        rc = e_model_load(c, path);
    }
    if (rc == PINFER_OK) rc = alloc_state(c);
    if (rc == PINFER_OK) {
        const char *g = getenv("PINFER_GRAPHS");
        c->use_graphs = g ? atoi(g) != 0 : 1;
        if (nmx_sync(c->dev)) rc = PINFER_E_NOMEM;
    }
    if (rc != PINFER_OK) {
        pinfer_free(c);
        c = NULL;
    }
    if (err) *err = rc;
    return c;
}

void pinfer_free(pinfer_ctx *c) {
    if (!c) return;
    if (c->dev) {
        nmx_sync(c->dev); /* nothing of the stream in flight when its graphs are destroyed */
        e_drop_graphs(c);
        nmx_host_free(c->dev, c->mbox);
        pinfer_checkpoint_clear(c);
        nmx_sync(c->dev);
        nmx_free(c->dev, c->blob);
        for (int i = 0; i < c->n_allocs; i++) nmx_free(c->dev, c->allocs[i]);
        nmx_destroy(c->dev);
    }
    e_ngram_free(&c->ng);
    free(c->layers);
    free(c);
}

void pinfer_reset(pinfer_ctx *c) {
    if (!c) return;
    const size_t S = (size_t)(c->conv_k - 1);
    if (c->n_lin) {
        nmx_fill_zero(c->dev, c->conv_state, (size_t)c->n_lin * (S ? S : 1) * c->conv_dim * 4);
        nmx_fill_zero(c->dev, c->rec, (size_t)c->n_lin * c->lv_heads * c->lk_dim * c->lv_dim * 4);
    }
    nmx_ctl_set(c->dev, c->ctl, 0, 0);
    nmx_ctl_set(c->dev, c->ctl, 1, 0);
    nmx_ctl_set(c->dev, c->ctl, 2, 0);
    c->n_past = 0;
    c->mtp_rows = 0;
    c->keep = 0;
    c->ck_valid = 0; /* the checkpoint's memory is kept until pinfer_checkpoint_clear */
    nmx_sync(c->dev);
}

static int check_tokens(const pinfer_ctx *c, const int32_t *tokens, int n) {
    if (!c || !tokens || n <= 0) return PINFER_E_ARG;
    for (int i = 0; i < n; i++)
        if (tokens[i] < 0 || tokens[i] >= c->vocab) return PINFER_E_ARG;
    if (n > c->max_ctx - c->n_past) return PINFER_E_CTX_FULL;
    return PINFER_OK;
}

/* engine/src/forward.c:154-165 with logits of the last token only. */
static int eval_chunks(pinfer_ctx *c, const int32_t *tokens, int n, int want_logits) {
    for (int t0 = 0; t0 < n; t0 += E_MAX_BATCH) {
        const int nb = n - t0 < E_MAX_BATCH ? n - t0 : E_MAX_BATCH;
        if (nmx_upload(c->dev, c->tok, tokens + t0, (size_t)nb * 4)) return PINFER_E_ARG;
        int rc = e_set_pos(c, c->n_past);
        if (rc == PINFER_OK) rc = e_forward(c, c->tok, nb, 0, 0);
        if (rc != PINFER_OK) return rc;
        c->keep = 0;
        if (t0 + nb == n && want_logits) {
            rc = e_head_last(c, nb, NULL, 1);
            if (rc != PINFER_OK) return rc;
        }
        c->n_past += nb;
    }
    return e_set_pos(c, c->n_past);
}

int pinfer_eval(pinfer_ctx *c, const int32_t *tokens, int n, float *logits) {
    int rc = check_tokens(c, tokens, n);
    if (rc != PINFER_OK) return rc;
    rc = eval_chunks(c, tokens, n, logits != NULL);
    if (rc == PINFER_OK && logits &&
        nmx_download(c->dev, logits, c->logits, (size_t)c->vocab * sizeof(float)))
        rc = PINFER_E_ARG;
    return rc;
}

int pinfer_eval_select(pinfer_ctx *c, const int32_t *tokens, int n, const int32_t *ids,
                       int n_ids, float *out) {
    if (!c || n_ids < 0 || (n_ids > 0 && (!ids || !out))) return PINFER_E_ARG;
    for (int i = 0; i < n_ids; i++)
        if (ids[i] < 0 || ids[i] >= c->vocab) return PINFER_E_ARG;
    int rc = check_tokens(c, tokens, n);
    if (rc != PINFER_OK) return rc;
    rc = eval_chunks(c, tokens, n, n_ids > 0);
    if (rc != PINFER_OK || n_ids == 0) return rc;
    float *all = malloc((size_t)c->vocab * sizeof(float));
    if (!all) return PINFER_E_NOMEM;
    if (nmx_download(c->dev, all, c->logits, (size_t)c->vocab * sizeof(float))) rc = PINFER_E_ARG;
    for (int i = 0; rc == PINFER_OK && i < n_ids; i++) out[i] = all[ids[i]];
    free(all);
    return rc;
}

int pinfer_has_mtp(const pinfer_ctx *c) { return c && c->has_mtp ? 1 : 0; }
int pinfer_n_vocab(const pinfer_ctx *c) { return c ? c->vocab : 0; }
int pinfer_n_past(const pinfer_ctx *c) { return c ? c->n_past : 0; }
int pinfer_eos_id(const pinfer_ctx *c) { return c ? c->eos : -1; }

/* First index of the maximum (engine/src/forward_ops.c:387-409). */
int pinfer_argmax(const float *v, int n) {
    if (!v || n <= 0) return -1;
    float mx = v[0];
    for (int i = 1; i < n; i++)
        if (v[i] > mx) mx = v[i];
    for (int i = 0; i < n; i++)
        if (v[i] == mx) return i;
    return 0;
}

int pinfer_generate_greedy_ex(pinfer_ctx *c, const int32_t *prompt, int n_prompt, int32_t *out,
                              int n_max, const pinfer_spec_params *sp,
                              const pinfer_gen_opts *opts, pinfer_spec_stats *stats,
                              int *status) {
    if (c) pinfer_reset(c);
    return e_generate(c, prompt, n_prompt, out, n_max, sp, opts, stats, status, 0);
}

int pinfer_generate_greedy_cont(pinfer_ctx *c, const int32_t *prompt, int n_prompt,
                                int32_t *out, int n_max, const pinfer_spec_params *sp,
                                const pinfer_gen_opts *opts, pinfer_spec_stats *stats,
                                int *status) {
    return e_generate(c, prompt, n_prompt, out, n_max, sp, opts, stats, status, 1);
}

int pinfer_generate_greedy(pinfer_ctx *c, const int32_t *prompt, int n_prompt, int32_t *out,
                           int n_max, const pinfer_spec_params *sp, pinfer_spec_stats *stats) {
    int status;
    const int n = pinfer_generate_greedy_ex(c, prompt, n_prompt, out, n_max, sp, NULL, stats,
                                            &status);
    return status != PINFER_OK ? status : n;
}

/* The timing of the reference CLI's benchmark (engine/tools/pinfer_run.c:384-397,425-430):
 * reset, prefill the prompt (timed), then generate n_gen tokens ignoring EOS (timed); decode
 * tok/s is (n_gen - 1) / decode seconds. Returns the count or a negative PINFER_E* code. */
int pinfer_bench_generate(pinfer_ctx *c, const int32_t *prompt, int n_prompt, int32_t *out,
                          int n_gen, const pinfer_spec_params *sp, pinfer_spec_stats *stats,
                          double *prefill_s, double *decode_s) {
    int status;
    if (c) pinfer_reset(c);
    const int n = e_generate_timed(c, prompt, n_prompt, out, n_gen, sp, NULL, stats, &status, 1,
                                   0, prefill_s, decode_s);
    return status != PINFER_OK ? status : n;
}
