/* Internal definitions of the MI355X engine (libpinfer.so): the context, the device-resident
 * model and state, and the forward / speculative-decoding entry points shared by the host
 * source files. Not part of the public API (include/pinfer.h). */
#ifndef NMXE_ENGINE_H
#define NMXE_ENGINE_H

#include <stddef.h>
#include <stdint.h>

#include "nmx.h"
#include "pinfer.h"

#define E_MAX_BATCH 64   /* rows per forward chunk (the reference's PF_MAX_BATCH) */
#define E_MAX_K PINFER_SPEC_MAX_K
#define E_MAX_ALLOCS 96  /* device allocations per context besides the weight blob */

/* .pq dtypes and layout constants (engine/src/pq_format.h, pq_quant.h) */
enum { PQ_F32 = 0, PQ_BF16 = 1, PQ_Q4K = 4 };

typedef struct {
    const void *w;      /* device pointer to Q4K_G32 bytes */
    int rows, cols;
} e_mat;

typedef struct {
    int is_full;
    const float *in_norm, *post_norm;   /* device, stored effective multipliers */
    e_mat gate, up, down;
    /* Gated DeltaNet */
    int lin;                            /* index among the linear layers, -1 */
    e_mat qkv, z, b, a, out;
    const float *conv_w, *A_log, *A, *dt_bias, *lin_norm;
    /* gated full attention */
    int full;                           /* index among the full-attention layers, -1 */
    e_mat q, k, v, o;
    const float *q_norm, *k_norm;
} e_layer;

/* one set of per-row scratch buffers (E_MAX_BATCH rows) */
typedef struct {
    float *x, *x2, *xn, *out, *ta, *tb, *tc, *to, *conv, *ba, *aa, *beta, *decay, *cat, *emb;
    float *sc; /* attention scores [B][n_heads][max_ctx] */
    nmx_a8 a_h;        /* A8 of width hidden */
    nmx_a8 a_w;        /* A8 of the wide inputs: vd, n_heads * head_dim, 2 * hidden */
    nmx_a8 a_f;        /* A8 of width ffn */
    nmx_a8 a_1;        /* A8 of one hidden row (the head of a single row) */
    float *row1;       /* [hidden] */
} e_scratch;

/* Prompt-lookup drafts (ngram.c; the role of engine/src/ngram.h:13-47): a draft continues the
 * most recent earlier occurrence of the history's tail that agrees with it over the most
 * tokens (at least E_NG_MIN, counted up to E_NG_EXT). The draft rule of the speculative loop
 * (spec.c ngram_pick): an agreement of at least E_NG_TRUST tokens drafts in full; E_NG_ASK..
 * tokens only when the draft's first token equals the MTP head's d1, then at most E_NG_SHORT
 * tokens; without the MTP head, shorter agreements draft E_NG_SHORT tokens. */
#define E_NG_MIN 2
#define E_NG_EXT 32
#define E_NG_TRUST 16
#define E_NG_ASK 4
#define E_NG_SHORT 3

typedef struct {
    int32_t *tok;   /* [cap] token history, oldest first */
    int32_t *link;  /* [cap] next older position whose 2-gram shares the bucket, -1: none */
    int32_t *head;  /* [1 << bits] newest indexed position per 2-gram bucket, -1: none */
    int cap, n;     /* capacity, tokens in the history */
    int indexed;    /* positions [1, indexed) are in the chains */
    int bits;
} e_ngram;

int e_ngram_init(e_ngram *g, int cap);
void e_ngram_free(e_ngram *g);
void e_ngram_reset(e_ngram *g);
void e_ngram_push(e_ngram *g, const int32_t *t, int m);
void e_ngram_pop(e_ngram *g);
/* Up to max tokens that followed the chosen earlier occurrence of the history's tail; returns
 * the count (0: no occurrence) and, if match != NULL, how many tokens the occurrence agrees
 * with the tail, counted backwards from the newest (E_NG_MIN .. E_NG_EXT). */
int e_ngram_draft(e_ngram *g, int32_t *out, int max, int *match);

/* The adaptive speculation policy (adapt.c; the role of engine/src/spec_adapt.c): the verify
 * width of the next round (1 = a plain step) from decayed acceptance counts per draft position
 * and the measured seconds of each width's rounds. */
#define E_AD_W (PINFER_SPEC_MAX_K + 2) /* widths 1..PINFER_SPEC_MAX_K + 1 */
typedef struct {
    int k;                 /* largest draft count: widths 1..k + 1 */
    double t[E_AD_W];      /* running seconds of a round of width w, 0 = not measured */
    long seen[E_AD_W];     /* round count when width w was last measured */
    double hits[E_AD_W], tries[E_AD_W]; /* decayed counts: draft j reached / accepted */
    long rounds;           /* widths chosen so far */
} e_adapt;

void e_adapt_init(e_adapt *a, int k);
int e_adapt_width(e_adapt *a);
/* a round of width w (w - 1 drafts) accepted `accepted` drafts and took sec seconds */
void e_adapt_observe(e_adapt *a, int w, int accepted, double sec);

struct pinfer_ctx {
    nmx_ctx *dev;
    /* dimensions (engine/src/pinfer.c:45-63) */
    int H, ffn, n_layers, vocab;
    int n_heads, n_kv, hd, rot;
    int lk_heads, lv_heads, lk_dim, lv_dim, conv_k, kd, vd, conv_dim;
    int eos;
    float rms_eps, rope_theta;
    int n_lin, n_full, has_mtp;
    int max_ctx;

    /* weights: the .pq data section uploaded as one block */
    void *blob;
    e_layer *layers;
    e_mat embed;              /* token embedding [vocab][H] */
    e_mat head;               /* output head [vocab][H] (the embedding when tied) */
    const float *norm;
    /* MTP head (engine/src/mtp.c:8-34) */
    e_mat mtp_fc;
    const float *mtp_norm_emb, *mtp_norm_hid, *mtp_norm_out;
    e_layer mtp;

    /* state in HBM */
    float *conv_state;        /* [n_lin][conv_k-1][conv_dim] */
    float *rec;               /* [n_lin][lv_heads][lv_dim][lk_dim] */
    int kv_dtype;             /* PINFER_KV_*: storage of every KV cache (nmx.h nmx_kv_bytes) */
    size_t kv_bytes;          /* bytes of one cache: [n_kv][max_ctx] rows (+ int8 scales) */
    void *kc, *vc;            /* [n_full] caches of kv_bytes each */
    void *mkc, *mvc;          /* MTP caches */
    float *xin;               /* [n_lin][cap][conv_dim] raw conv inputs of a logged pass */
    float *log, *pend;        /* [n_lin][cap][lv_heads][lk_dim + lv_dim + 1] */
    int cap;                  /* rows per log = E_MAX_K + 1 */
    float *rope_cos, *rope_sin;

    e_scratch s;
    float *hbuf;              /* [E_MAX_BATCH][H] final-normed rows kept for the MTP pass */
    float *pbuf;              /* [E_MAX_BATCH][H] committed rows waiting for the MTP pass
                               * (plain steps, n-gram rounds) */
    float *mbuf;              /* [3][H]: MTP hidden of the current draft + chain ping-pong */
    int32_t *ctl;             /* [16] control block (see nmx.h) */
    int32_t *vt;              /* [E_MAX_K + 2] verify tokens */
    int32_t *tok;             /* [E_MAX_BATCH] tokens of an eager forward */
    int32_t *hout;            /* [2 + E_MAX_BATCH] head output */
    int32_t *hout2;           /* [2 + 1] MTP head output */
    int32_t *dcopy;           /* [E_MAX_K + 2] the verify head's copy of the drafts */
    int32_t *mbox;            /* host memory [2 + E_MAX_K + 2 + 1]: a verify round's (a, bonus, vt), flag */
    void *hwork;              /* head argmax scratch */
    float *logits;            /* [vocab] logits of one row when requested */

    /* host mirror of the position state */
    int n_past, mtp_rows, keep;
    /* captured rounds, one graph per draft count: MTP rounds (MTP chain, verify pass, head
     * and acceptance, commit, MTP pass over the committed rows) and n-gram rounds (verify
     * pass, head and acceptance, commit) */
    nmx_graph *g_round[E_MAX_K + 1], *g_round_ng[E_MAX_K + 1];
    float *conv_bak;          /* [n_lin][conv_k-1][conv_dim]: conv state before the last commit */
    e_ngram ng;               /* token history of the prompt-lookup drafts */
    int graph_nv;             /* draft vocabulary the graphs were captured with */
    int use_graphs;
    void *allocs[E_MAX_ALLOCS]; /* every device allocation besides the weight blob */
    int n_allocs;
    uint64_t model_fp;          /* fingerprint of the .pq file (state blobs) */
    /* in-context checkpoint: device copy of the conv and recurrent states */
    void *ck_dev;
    int ck_valid, ck_n_past, ck_mtp_rows;
};

/* forward.c */
int e_forward(pinfer_ctx *c, int32_t *tok_dev, int n, int logged, int keys_last);
int e_head_last(pinfer_ctx *c, int n, int32_t *dst_dev, int want_logits);
int e_mtp_forward(pinfer_ctx *c, const float *h_dev, int32_t *tok_dev, int n, int pos_off,
                  int head_row_dynamic, int nv, int32_t *draft_dst, float *m_dst, int advance,
                  int keys_io);
/* e_keys_ok: the draft heads and their consumers can pass a draft as argmax keys in c->hwork
 * (keys_io of e_mtp_forward: E_KEYS_IN = the one input token from the keys, written to
 * tok_dev[0]; E_KEYS_OUT = the draft left as keys, draft_dst unused; keys_last of e_forward:
 * row n - 1's token from the keys, written to tok_dev[n - 1]). */
enum { E_KEYS_IN = 1, E_KEYS_OUT = 2 };
int e_keys_ok(const pinfer_ctx *c);
int e_set_pos(pinfer_ctx *c, int pos);

/* spec.c */
/* append: a continuation of the context (pinfer_generate_greedy_cont), which keeps the
 * n-gram history when the prompt leads with the last emitted token */
int e_generate(pinfer_ctx *c, const int32_t *prompt, int n_prompt, int32_t *out, int n_max,
               const pinfer_spec_params *sp, const pinfer_gen_opts *opts,
               pinfer_spec_stats *stats, int *status, int append);
int e_generate_timed(pinfer_ctx *c, const int32_t *prompt, int n_prompt, int32_t *out,
                     int n_max, const pinfer_spec_params *sp, const pinfer_gen_opts *opts,
                     pinfer_spec_stats *stats, int *status, int no_eos, int append,
                     double *t_prefill, double *t_decode);
void e_drop_graphs(pinfer_ctx *c);

/* state.c: KV rows of the context's format */
size_t e_kv_row_bytes(const pinfer_ctx *c);
int e_kv_zero_rows(pinfer_ctx *c, void *cache, int p0, int p1);

/* model.c: e_model_check validates a .pq file (header, directory, every tensor the engine
 * maps, the kernels' limits) with no device call; e_model_load does the same, then uploads the
 * data section and builds the device views */
int e_model_check(const char *path);
int e_model_load(pinfer_ctx *c, const char *path);

#endif
