/* The forward pass of the Qwen3.5 hybrid on the device: the per-layer sequence of
 * engine/src/forward.c:92-147 (forward_chunk), forward_lin.c:94-133 (pf_linear_attn),
 * forward_attn.c:231-266 (pf_full_attn) and mtp.c:60-100 (pf_mtp_forward), each step an nmx
 * kernel on the context's stream. Nothing here touches the host copy of any activation, so a
 * sequence can be captured into a HIP graph; positions come from the control block c->ctl
 * (ctl[0] = n_past at the start of the pass). Residual adds are fused into the following
 * RMSNorm, the RMSNorms into the prologue of the matmul that consumes them (input projections,
 * gate/up), SwiGLU into the gate/up matmul's epilogue, and every other matmul input is
 * A8-quantized by the kernel that produces it. */
#include <math.h>
#include <stdio.h>

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

int e_set_pos(pinfer_ctx *c, int pos) {
    CK(nmx_ctl_set(c->dev, c->ctl, 0, pos));
    return PINFER_OK;
}

/* the KV caches of full-attention layer f (c->kv_bytes each) */
static void *kv_of(void *base, const pinfer_ctx *c, int f) { return (char *)base + (size_t)f * c->kv_bytes; }

/* The residual stream: rows in one of two buffers; a fused norm reads the current one (plus
 * the pending residual add) and writes the sum to the other, which becomes current. */
typedef struct {
    float *cur, *alt;
    const float *add; /* residual to add before the next norm (NULL: none) */
} e_resid;

/* The norm input over the residual stream: cur (+ add, the sum written to alt) with weight w;
 * resid_done then makes the sum current. */
static nmx_norm_in resid_norm(const pinfer_ctx *c, const e_resid *r, const float *w) {
    const nmx_norm_in in = {r->cur, c->H, r->add, c->H, r->add ? r->alt : NULL, c->H, w, c->rms_eps};
    return in;
}

static void resid_done(e_resid *r) {
    if (r->add) {
        float *t = r->cur;
        r->cur = r->alt;
        r->alt = t;
        r->add = NULL;
    }
}

/* The input projections of a block: from the A8 rows in s->a_h, or (in != NULL) with the
 * block's input RMSNorm as a prologue of the matmul's workgroups (nmx_q4k_matmul_norm: every
 * workgroup redoes the norm of the n x H rows while its weight loads are in flight, one
 * launch fewer; s->a_h is its fallback's buffer). */
static int proj_in(pinfer_ctx *c, int count, const void *const *W, const int *R, float *const *Y,
                   int n, const nmx_norm_in *in) {
    e_scratch *s = &c->s;
    if (in) CK(nmx_q4k_matmul_norm(c->dev, count, W, R, Y, R, c->H, n, in, s->a_h));
    else CK(nmx_q4k_matmul_multi(c->dev, count, W, R, Y, R, c->H, n, s->a_h.q, s->a_h.d, s->a_h.fs));
    return PINFER_OK;
}

/* Gated full attention (engine/src/forward_attn.c:231-266) on the normed rows (A8 in s->a_h,
 * or normed by the projection itself: in): q (query | gate per head), k, v in one launch;
 * kc / vc: the block's caches; pos_off: position of row 0 relative to ctl[0]. Output (o_proj)
 * to s->out. */
static int attn_block(pinfer_ctx *c, const e_layer *L, int n, void *kc, void *vc, int pos_off,
                      const nmx_norm_in *in) {
    nmx_ctx *D = c->dev;
    e_scratch *s = &c->s;
    const int H = c->H, hd = c->hd, qw = 2 * c->n_heads * hd, kvw = c->n_kv * hd;
    const void *W[3] = {L->q.w, L->k.w, L->v.w};
    const int R[3] = {qw, kvw, kvw};
    float *Y[3] = {s->ta, s->tb, s->tc};
    TRY(proj_in(c, 3, W, R, Y, n, in));
    nmx_attn_args a = {n, c->n_heads, c->n_kv, hd, c->rot, c->max_ctx, s->ta, s->tb, s->tc,
                       L->q_norm, L->k_norm, c->rms_eps, 1.0f / sqrtf((float)hd), c->rope_cos,
                       c->rope_sin, kc, vc, c->ctl, pos_off, s->to, s->a_w, s->sc, c->kv_dtype};
    CK(nmx_attn_fused(D, &a)); /* prep + scores in one launch, then P.V */
    CK(nmx_q4k_matmul(D, L->o.w, H, c->n_heads * hd, n, s->a_w.q, s->a_w.d, s->a_w.fs, s->out,
                      H, NULL));
    return PINFER_OK;
}

/* post norm + SwiGLU MLP (engine/src/forward.c:49-58): x += mix out; xn = norm(x);
 * out = down(silu(gate xn) * up xn). One launch does the residual add, the RMSNorm and its A8
 * (a prologue of each workgroup, overlapping its weight loads), the gate / up products and
 * silu(g) * u with its A8: 9.1 us against 3.3 + 6.8 us for a separate norm launch. */
static int mlp_block(pinfer_ctx *c, const e_layer *L, int n, e_resid *r) {
    nmx_ctx *D = c->dev;
    e_scratch *s = &c->s;
    const int H = c->H, F = c->ffn;
    const nmx_norm_in in = {r->cur, H, s->out, H, r->alt, H, L->post_norm, c->rms_eps};
    CK(nmx_q4k_swiglu(D, L->gate.w, L->up.w, F, H, n, NULL, NULL, NULL, &in, NULL, s->a_f, s->a_h,
                      s->ta, s->tb));
    float *t = r->cur; /* the sum x + out is the residual stream now */
    r->cur = r->alt;
    r->alt = t;
    r->add = NULL;
    CK(nmx_q4k_matmul(D, L->down.w, H, F, n, s->a_f.q, s->a_f.d, s->a_f.fs, s->out, H, NULL));
    r->add = s->out;
    return PINFER_OK;
}

/* Gated DeltaNet mixer (engine/src/forward_lin.c:94-133) on the normed rows (A8 in s->a_h, or
 * normed by the projection itself: in). logged: a verify pass (token 0 committed in place,
 * tokens 1.. logged for the commit); pending replays of the last commit are applied first
 * (keep = ctl[2]). */
static int lin_block(pinfer_ctx *c, const e_layer *L, int n, int logged, const nmx_norm_in *in) {
    nmx_ctx *D = c->dev;
    e_scratch *s = &c->s;
    const int H = c->H, C = c->conv_dim, vd = c->vd, nv = c->lv_heads, li = L->lin;
    const int logw = c->lk_dim + c->lv_dim + 1;
    const size_t lrow = (size_t)c->cap * nv * logw;
    const void *W[4] = {L->qkv.w, L->z.w, L->b.w, L->a.w};
    const int R[4] = {C, vd, nv, nv};
    float *Y[4] = {s->ta, s->tb, s->ba, s->aa};
    TRY(proj_in(c, 4, W, R, Y, n, in));
    nmx_lin_pre_args p = {n, C, c->conv_k, c->lk_dim, c->kd, s->ta, C, s->conv,
                          c->conv_state + (size_t)li * (c->conv_k - 1) * C, L->conv_w,
                          logged ? c->xin + (size_t)li * c->cap * C : NULL,
                          1.0f / sqrtf((float)c->lk_dim), 1e-6f, s->ba, s->aa, nv, nv, L->A_log,
                          L->A, L->dt_bias, s->beta, s->decay};
    nmx_lin_args a = {n, nv, nv / c->lk_heads, c->lk_dim, c->lv_dim, C, vd, s->conv, s->decay,
                      s->beta, c->rec + (size_t)li * nv * c->lk_dim * c->lv_dim, s->to,
                      logged ? c->log + (size_t)li * lrow : NULL, c->pend + (size_t)li * lrow,
                      c->cap - 1, 0, c->ctl + 2};
    /* conv + gates, recurrence, gated norm + A8 of o: one launch */
    nmx_lin_mix_args m = {p, a, s->tb, vd, L->lin_norm, c->rms_eps, NULL, 0, s->a_w};
    CK(nmx_lin_mix(D, &m));
    CK(nmx_q4k_matmul(D, L->out.w, H, vd, n, s->a_w.q, s->a_w.d, s->a_w.fs, s->out, H, NULL));
    return PINFER_OK;
}

int e_keys_ok(const pinfer_ctx *c) { return c->H % 256 == 0 && c->H <= 1024; }

/* n tokens (device ids) at positions ctl[0].. through the main model; leaves the final-normed
 * rows in s->xn and their A8 in s->a_h (the head's input). keys_last > 0: row n - 1's token is
 * the argmax of that many partial keys in c->hwork (written to tok_dev[n - 1]). */
int e_forward(pinfer_ctx *c, int32_t *tok_dev, int n, int logged, int keys_last) {
    nmx_ctx *D = c->dev;
    e_scratch *s = &c->s;
    const int H = c->H;
    e_resid r = {s->x, s->x2, NULL};
    /* the embedding rows (the residual stream) and the first layer's input norm, one launch */
    const nmx_a8 none = {NULL, NULL, NULL};
    if (keys_last > 0)
        CK(nmx_embed_norm_keys(D, c->embed.w, c->vocab, tok_dev, n, H, c->rms_eps,
                               c->layers[0].in_norm, r.cur, H, s->a_h, c->hwork, keys_last));
    else
        CK(nmx_embed_norm(D, c->embed.w, c->vocab, tok_dev, n, H, c->rms_eps, c->layers[0].in_norm,
                          r.cur, H, NULL, 0, s->a_h, NULL, 0, NULL, NULL, 0, none));
    for (int l = 0; l < c->n_layers; l++) {
        const e_layer *L = &c->layers[l];
        /* layer 0's input norm ran with the embedding; the others run in the projections */
        const nmx_norm_in in = resid_norm(c, &r, L->in_norm);
        const nmx_norm_in *pin = l > 0 ? &in : NULL;
        int rc = L->is_full ? attn_block(c, L, n, kv_of(c->kc, c, L->full),
                                         kv_of(c->vc, c, L->full), 0, pin)
                            : lin_block(c, L, n, logged, pin);
        if (rc) return rc;
        if (l > 0) resid_done(&r);
        if ((rc = mlp_block(c, L, n, &r))) return rc;
    }
    CK(nmx_rmsnorm_xo(D, r.cur, H, r.add, H, NULL, 0, c->norm, n, H, c->rms_eps, s->xn, H, s->a_h));
    /* every linear layer applied the pending rows: keep = 0, except after a logged pass, which
     * the commit always follows and whose kernel sets keep = e - 1 itself */
    if (!logged) CK(nmx_ctl_set(D, c->ctl, 2, 0));
    return PINFER_OK;
}

/* Head of one row of s->xn (row index *idx + off): argmax over the first `rows` head rows to
 * dst_dev (if not NULL); the logits of that row to c->logits when want_logits. */
/* The head over the first `rows` rows for the one row whose A8 is in s->a_1: its argmax to
 * dst_dev (when not NULL), the logits to c->logits when wanted. */
static int head_a8(pinfer_ctx *c, int rows, int32_t *dst_dev, int want_logits) {
    nmx_ctx *D = c->dev;
    e_scratch *s = &c->s;
    CK(nmx_head_accept_to(D, c->head.w, rows, c->H, 1, s->a_1.q, s->a_1.d, s->a_1.fs,
                          want_logits ? c->logits : NULL, NULL, c->hwork, c->hout2, dst_dev));
    return PINFER_OK;
}

static int head_row(pinfer_ctx *c, const int32_t *idx, int off, int rows, int32_t *dst_dev,
                    int want_logits) {
    nmx_ctx *D = c->dev;
    e_scratch *s = &c->s;
    CK(nmx_select_row(D, s->xn, c->H, idx, off, c->H, s->row1));
    CK(nmx_quant_a8(D, s->row1, 1, c->H, s->a_1.q, s->a_1.d, s->a_1.fs));
    return head_a8(c, rows, dst_dev, want_logits);
}

int e_head_last(pinfer_ctx *c, int n, int32_t *dst_dev, int want_logits) {
    return head_row(c, c->ctl + 15, n - 1, c->vocab, dst_dev, want_logits);
}

/* The MTP draft head (engine/src/mtp.c:60-100) over n rows: h_dev [n][H] final-normed
 * hiddens, tok_dev [n] the tokens that follow them, positions ctl[0] + pos_off + i. The
 * selected row (n - 1, or ctl[1] - 1 when head_row_dynamic) gives the draft (argmax over the
 * first nv head rows) to draft_dst and its MTP hidden to m_dst (each may be NULL). advance:
 * ctl[0] += ctl[1] at the end (folded into the draft head's last kernel where it can be).
 * keys_io (e_keys_ok shapes, one row): E_KEYS_IN, the token from the partial keys in c->hwork
 * (written to tok_dev[0]); E_KEYS_OUT, the draft left there as keys (draft_dst unused). */
int e_mtp_forward(pinfer_ctx *c, const float *h_dev, int32_t *tok_dev, int n, int pos_off,
                  int head_row_dynamic, int nv, int32_t *draft_dst, float *m_dst, int advance,
                  int keys_io) {
    nmx_ctx *D = c->dev;
    e_scratch *s = &c->s;
    const int H = c->H;
    const nmx_a8 none = {NULL, NULL, NULL};
    /* fc input [pre_fc_norm_embedding(embed(tok)) | pre_fc_norm_hidden(h)]: each norm gives
     * the A8 blocks of its half of the 2H row (blocks [0, H/32) and [H/32, 2H/32)); a block
     * never straddles the halves (H % 32 == 0). At most 8 rows, the embedding and both norms
     * run inside the fc matmul's workgroups; else one launch for them, then the matmul */
    e_resid r = {s->x, s->x2, NULL};
    const int nkeys = nmx_head_row_nkeys(nv);
    if (keys_io && (n != 1 || !e_keys_ok(c) || head_row_dynamic || advance)) return PINFER_E_ARG;
    if (n <= 8 && H % 256 == 0 && H <= 1024) {
        /* the embedding and both norms inside the fc matmul's workgroups */
        CK(nmx_q4k_matmul_embed_norm(D, c->mtp_fc.w, H, r.cur, H, n, H, c->embed.w, c->vocab,
                                     tok_dev, c->mtp_norm_emb, h_dev, H, c->mtp_norm_hid,
                                     c->rms_eps, s->a_w, (keys_io & E_KEYS_IN) ? c->hwork : NULL,
                                     nkeys));
    } else {
        const size_t hb = (size_t)(H / 32) * n;
        const nmx_a8 a8_emb = s->a_w, a8_hid = {s->a_w.q + hb * 32, s->a_w.d + hb, s->a_w.fs + hb};
        CK(nmx_embed_norm(D, c->embed.w, c->vocab, tok_dev, n, H, c->rms_eps, c->mtp_norm_emb,
                          s->emb, H, s->cat, 2 * H, a8_emb, h_dev, H, c->mtp_norm_hid, s->cat + H,
                          2 * H, a8_hid));
        CK(nmx_q4k_matmul(D, c->mtp_fc.w, H, 2 * H, n, s->a_w.q, s->a_w.d, s->a_w.fs, r.cur, H,
                          NULL));
    }
    const e_layer *L = &c->mtp;
    const nmx_norm_in in = resid_norm(c, &r, L->in_norm);
    int rc = attn_block(c, L, n, c->mkc, c->mvc, pos_off, &in);
    if (rc) return rc;
    resid_done(&r);
    if ((rc = mlp_block(c, L, n, &r))) return rc;
    const int32_t *idx = head_row_dynamic ? c->ctl + 1 : c->ctl + 15;
    const int off = head_row_dynamic ? -1 : n - 1;
    if (keys_io & E_KEYS_OUT) { /* the draft as partial argmax keys for its consumer */
        CK(nmx_head_row_keys(D, c->head.w, nv, H, r.cur, H, r.add, H, c->mtp_norm_out,
                             c->rms_eps, idx, off, n, m_dst ? m_dst : s->xn, c->hwork));
        return PINFER_OK;
    }
    if (draft_dst && H <= 1024 && H % 256 == 0) {
        /* the selected row's final norm (its MTP hidden to m_dst; a single row always to s->xn)
         * inside the draft head's workgroups */
        float *y = m_dst ? m_dst : n == 1 && !head_row_dynamic ? s->xn : NULL;
        CK(nmx_head_row_accept_to(D, c->head.w, nv, H, r.cur, H, r.add, H, c->mtp_norm_out,
                                  c->rms_eps, idx, off, n, y, c->hwork, c->hout2, draft_dst,
                                  s->a_1, advance ? c->ctl : NULL));
        return PINFER_OK;
    }
    if (n == 1 && !head_row_dynamic) {
        /* one row: the final norm writes the MTP hidden and the head's A8 input itself */
        CK(nmx_rmsnorm_xo(D, r.cur, H, r.add, H, NULL, 0, c->mtp_norm_out, 1, H, c->rms_eps,
                          m_dst ? m_dst : s->xn, H, draft_dst ? s->a_1 : none));
        if (draft_dst) TRY(head_a8(c, nv, draft_dst, 0));
    } else if (H <= 1024 && H % 32 == 0 && (m_dst || draft_dst)) {
        /* only the selected row: its MTP hidden and the head's A8 input, one launch */
        CK(nmx_rmsnorm_row(D, r.cur, H, r.add, H, c->mtp_norm_out, H, c->rms_eps, idx, off, n,
                           m_dst, draft_dst ? s->a_1 : none));
        if (draft_dst) TRY(head_a8(c, nv, draft_dst, 0));
    } else {
        CK(nmx_rmsnorm_xo(D, r.cur, H, r.add, H, NULL, 0, c->mtp_norm_out, n, H, c->rms_eps, s->xn,
                          H, none));
        if (m_dst) CK(nmx_select_row(D, s->xn, H, idx, off, H, m_dst));
        if (draft_dst) TRY(head_row(c, idx, off, nv, draft_dst, 0));
    }
    if (advance) CK(nmx_ctl_advance(D, c->ctl));
    return PINFER_OK;
}
