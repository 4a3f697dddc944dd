/* Conversation state snapshot / restore and the in-context checkpoint (include/pinfer.h) for
 * the device-resident state; the counterpart of engine/src/state.c:1-224.
 *
 * The blob has the reference's format (header of dims, n_past, KV dtype, MTP rows and the
 * model fingerprint; then per linear layer the conv state [(conv_k-1)][conv_dim] and the
 * recurrent state; per full-attention layer the K rows [n_kv][n_past] then the V rows; then
 * the MTP head's K and V rows), so a state moves between this engine and the reference's.
 * The recurrent state lives on the device in the recurrence kernels' layout
 * (nmx_state_index: a value column's keys in quarters, tiled so that each wave's loads are
 * contiguous) and is written to the blob in the reference's [heads][dk][dv] order.
 *
 * The checkpoint keeps a device copy of the conv and recurrent states only, like the
 * reference: KV rows below the checkpoint's n_past are never rewritten while it is valid. */
#include <stdlib.h>
#include <string.h>

#include "engine.h"

#define STATE_MAGIC "PINFERS"
#define STATE_VERSION 2u

typedef struct {
    char magic[8];
    uint32_t version, n_past, kv_dtype, mtp_rows;
    uint32_t n_layers, hidden, n_kv, head_dim, lk_heads, lv_heads, lk_dim, lv_dim, conv_k;
    uint32_t full_mask;
    uint64_t model_fp;
} state_hdr;

_Static_assert(sizeof(state_hdr) == 72, "state header layout");

static size_t conv_bytes(const pinfer_ctx *c) {
    return (size_t)(c->conv_k - 1) * c->conv_dim * sizeof(float);
}
static size_t rec_bytes(const pinfer_ctx *c) {
    return (size_t)c->lv_heads * c->lk_dim * c->lv_dim * sizeof(float);
}
/* bytes of one cache row in the context's format, and of rows [0, n) of every group with
 * their int8 scales (engine/src/state.c:40-44) */
size_t e_kv_row_bytes(const pinfer_ctx *c) {
    return (size_t)c->hd * (c->kv_dtype == PINFER_KV_F32 ? 4 : c->kv_dtype == PINFER_KV_F16 ? 2 : 1);
}
static size_t rows_bytes(const pinfer_ctx *c, int n) {
    return (size_t)c->n_kv * (size_t)n *
           (e_kv_row_bytes(c) + (c->kv_dtype == PINFER_KV_I8 ? sizeof(float) : 0));
}
static float *kv_scales(const pinfer_ctx *c, void *cache) {
    return (float *)(void *)((char *)cache + (size_t)c->n_kv * c->max_ctx * e_kv_row_bytes(c));
}

/* Zero rows [p0, p1) of every group of a cache (and their int8 scales): positions whose values
 * were never computed must not reach an attention pass (forward_kv.c:128-139). */
int e_kv_zero_rows(pinfer_ctx *c, void *cache, int p0, int p1) {
    if (p1 <= p0) return PINFER_OK;
    const size_t rb = e_kv_row_bytes(c);
    for (int g = 0; g < c->n_kv; g++) {
        const size_t r0 = (size_t)g * c->max_ctx + p0;
        if (nmx_fill_zero(c->dev, (char *)cache + r0 * rb, (size_t)(p1 - p0) * rb) ||
            (c->kv_dtype == PINFER_KV_I8 &&
             nmx_fill_zero(c->dev, kv_scales(c, cache) + r0, (size_t)(p1 - p0) * sizeof(float))))
            return PINFER_E_ARG;
    }
    return PINFER_OK;
}
static int mtp_rows(const pinfer_ctx *c) {
    return c->has_mtp && c->mtp_rows > 0 ? (c->mtp_rows < c->n_past ? c->mtp_rows : c->n_past) : 0;
}
static size_t state_bytes(const pinfer_ctx *c, int n_past, int n_mtp) {
    return sizeof(state_hdr) + (size_t)c->n_lin * (conv_bytes(c) + rec_bytes(c)) +
           (size_t)c->n_full * 2 * rows_bytes(c, n_past) + 2 * rows_bytes(c, n_mtp);
}
static uint32_t full_mask(const pinfer_ctx *c) {
    uint32_t m = 0;
    for (int l = 0; l < c->n_layers; l++)
        if (c->layers[l].is_full) m |= 1u << l;
    return m;
}

size_t pinfer_state_size(const pinfer_ctx *c) {
    return c ? state_bytes(c, c->n_past, mtp_rows(c)) : 0;
}

/* rows [0, n) of every KV group of one cache <-> the blob cursor: per group the rows, then
 * (int8) their scales (engine/src/state.c:64-83) */
static int copy_rows(pinfer_ctx *c, void *cache, int n, char *cur, int to_blob, char **next) {
    const size_t rb = e_kv_row_bytes(c), len = (size_t)n * rb, sl = (size_t)n * sizeof(float);
    for (int g = 0; g < c->n_kv; g++) {
        char *rows = (char *)cache + (size_t)g * c->max_ctx * rb;
        if (len && (to_blob ? nmx_download(c->dev, cur, rows, len) : nmx_upload(c->dev, rows, cur, len)))
            return PINFER_E_ARG;
        cur += len;
        if (c->kv_dtype == PINFER_KV_I8) {
            float *sc = kv_scales(c, cache) + (size_t)g * c->max_ctx;
            if (sl && (to_blob ? nmx_download(c->dev, cur, sc, sl) : nmx_upload(c->dev, sc, cur, sl)))
                return PINFER_E_ARG;
            cur += sl;
        }
    }
    *next = cur;
    return PINFER_OK;
}

/* one linear layer's conv and recurrent states <-> the blob cursor ([heads][dk][dv] there) */
static int copy_lin(pinfer_ctx *c, int li, char *cur, int to_blob, float *tmp, char **next) {
    const size_t cb = conv_bytes(c), sb = rec_bytes(c);
    float *conv = c->conv_state + (size_t)li * (c->conv_k - 1) * c->conv_dim;
    float *rec = c->rec + (size_t)li * c->lv_heads * c->lk_dim * c->lv_dim;
    const int dk = c->lk_dim, dv = c->lv_dim;
    float *blob_s = (float *)(void *)(cur + cb);
    if (to_blob) {
        if (nmx_download(c->dev, cur, conv, cb) || nmx_download(c->dev, tmp, rec, sb)) return PINFER_E_ARG;
        for (int h = 0; h < c->lv_heads; h++)
            for (int j = 0; j < dv; j++)
                for (int i = 0; i < dk; i++)
                    blob_s[((size_t)h * dk + i) * dv + j] = tmp[nmx_state_index(h, j, i, dk, dv)];
    } else {
        for (int h = 0; h < c->lv_heads; h++)
            for (int j = 0; j < dv; j++)
                for (int i = 0; i < dk; i++)
                    tmp[nmx_state_index(h, j, i, dk, dv)] = blob_s[((size_t)h * dk + i) * dv + j];
        if (nmx_upload(c->dev, conv, cur, cb) || nmx_upload(c->dev, rec, tmp, sb)) return PINFER_E_ARG;
    }
    *next = cur + cb + sb;
    return PINFER_OK;
}

int pinfer_state_save(const pinfer_ctx *cc, void *buf, size_t cap) {
    pinfer_ctx *c = (pinfer_ctx *)cc; /* device transfers only; the context is not changed */
    if (!c || !buf) return PINFER_E_ARG;
    const int n_mtp = mtp_rows(c);
    if (cap < state_bytes(c, c->n_past, n_mtp)) return PINFER_E_ARG;
    state_hdr hdr = {STATE_MAGIC, STATE_VERSION, (uint32_t)c->n_past, (uint32_t)c->kv_dtype,
                     (uint32_t)n_mtp, (uint32_t)c->n_layers, (uint32_t)c->H, (uint32_t)c->n_kv,
                     (uint32_t)c->hd, (uint32_t)c->lk_heads, (uint32_t)c->lv_heads,
                     (uint32_t)c->lk_dim, (uint32_t)c->lv_dim, (uint32_t)c->conv_k,
                     full_mask(c), c->model_fp};
    char *cur = buf;
    memcpy(cur, &hdr, sizeof hdr);
    cur += sizeof hdr;
    float *tmp = c->n_lin ? malloc(rec_bytes(c)) : NULL;
    if (c->n_lin && !tmp) return PINFER_E_NOMEM;
    int rc = PINFER_OK;
    for (int l = 0; rc == PINFER_OK && l < c->n_layers; l++)
        if (!c->layers[l].is_full) rc = copy_lin(c, c->layers[l].lin, cur, 1, tmp, &cur);
    free(tmp);
    for (int l = 0; rc == PINFER_OK && l < c->n_layers; l++)
        if (c->layers[l].is_full) {
            const size_t off = (size_t)c->layers[l].full * c->kv_bytes;
            rc = copy_rows(c, (char *)c->kc + off, c->n_past, cur, 1, &cur);
            if (rc == PINFER_OK) rc = copy_rows(c, (char *)c->vc + off, c->n_past, cur, 1, &cur);
        }
    if (rc == PINFER_OK && n_mtp > 0) {
        rc = copy_rows(c, c->mkc, n_mtp, cur, 1, &cur);
        if (rc == PINFER_OK) rc = copy_rows(c, c->mvc, n_mtp, cur, 1, &cur);
    }
    return rc;
}

int pinfer_state_load(pinfer_ctx *c, const void *buf, size_t len) {
    if (!c || !buf || len < sizeof(state_hdr)) return PINFER_E_ARG;
    state_hdr hdr;
    memcpy(&hdr, buf, sizeof hdr);
    if (memcmp(hdr.magic, STATE_MAGIC, 8) != 0 || hdr.version != STATE_VERSION)
        return PINFER_E_FORMAT;
    if (hdr.n_layers != (uint32_t)c->n_layers || hdr.hidden != (uint32_t)c->H ||
        hdr.n_kv != (uint32_t)c->n_kv || hdr.head_dim != (uint32_t)c->hd ||
        hdr.lk_heads != (uint32_t)c->lk_heads || hdr.lv_heads != (uint32_t)c->lv_heads ||
        hdr.lk_dim != (uint32_t)c->lk_dim || hdr.lv_dim != (uint32_t)c->lv_dim ||
        hdr.conv_k != (uint32_t)c->conv_k || hdr.full_mask != full_mask(c) ||
        hdr.kv_dtype != (uint32_t)c->kv_dtype || hdr.model_fp != c->model_fp)
        return PINFER_E_FORMAT; /* another model file, or another KV storage format */
    if (hdr.n_past > (uint32_t)c->max_ctx) return PINFER_E_CTX_FULL;
    if (hdr.mtp_rows > hdr.n_past || len < state_bytes(c, (int)hdr.n_past, (int)hdr.mtp_rows))
        return PINFER_E_FORMAT;
    const int n_past = (int)hdr.n_past, n_mtp = c->has_mtp ? (int)hdr.mtp_rows : 0;
    char *cur = (char *)buf + sizeof hdr;
    float *tmp = c->n_lin ? malloc(rec_bytes(c)) : NULL;
    if (c->n_lin && !tmp) return PINFER_E_NOMEM;
    int rc = PINFER_OK;
    for (int l = 0; rc == PINFER_OK && l < c->n_layers; l++)
        if (!c->layers[l].is_full) rc = copy_lin(c, c->layers[l].lin, cur, 0, tmp, &cur);
    free(tmp);
    for (int l = 0; rc == PINFER_OK && l < c->n_layers; l++)
        if (c->layers[l].is_full) {
            const size_t off = (size_t)c->layers[l].full * c->kv_bytes;
            rc = copy_rows(c, (char *)c->kc + off, n_past, cur, 0, &cur);
            if (rc == PINFER_OK) rc = copy_rows(c, (char *)c->vc + off, n_past, cur, 0, &cur);
        }
    if (rc == PINFER_OK && n_mtp > 0) {
        rc = copy_rows(c, c->mkc, n_mtp, cur, 0, &cur);
        if (rc == PINFER_OK) rc = copy_rows(c, c->mvc, n_mtp, cur, 0, &cur);
    }
    if (rc == PINFER_OK && c->has_mtp && n_past > n_mtp) { /* rows without saved values */
        rc = e_kv_zero_rows(c, c->mkc, n_mtp, n_past);
        if (rc == PINFER_OK) rc = e_kv_zero_rows(c, c->mvc, n_mtp, n_past);
    }
    if (rc != PINFER_OK) {
        pinfer_reset(c); /* a partial restore must not pass for a state */
        return rc;
    }
    c->n_past = n_past;
    c->mtp_rows = n_mtp;
    c->keep = 0;
    c->ck_valid = 0; /* the KV rows below the checkpoint were replaced */
    e_ngram_reset(&c->ng); /* a loaded context is not described by the history (state.c:210) */
    if (nmx_ctl_set(c->dev, c->ctl, 0, n_past) || nmx_ctl_set(c->dev, c->ctl, 2, 0) ||
        nmx_sync(c->dev))
        return PINFER_E_ARG;
    return PINFER_OK;
}

/* ---- in-context checkpoint (engine/src/state.c:158-224) ---------------------------------- */
static size_t ck_bytes(const pinfer_ctx *c) {
    return (size_t)c->n_lin * (conv_bytes(c) + rec_bytes(c));
}

int pinfer_checkpoint(pinfer_ctx *c) {
    if (!c) return PINFER_E_ARG;
    const size_t cb = (size_t)c->n_lin * conv_bytes(c), sb = (size_t)c->n_lin * rec_bytes(c);
    if (!c->ck_dev) {
        c->ck_dev = nmx_alloc(c->dev, ck_bytes(c) ? ck_bytes(c) : 4);
        if (!c->ck_dev) return PINFER_E_NOMEM;
    }
    if ((cb && nmx_copy_d2d(c->dev, c->ck_dev, c->conv_state, cb)) ||
        (sb && nmx_copy_d2d(c->dev, (char *)c->ck_dev + cb, c->rec, sb)) || nmx_sync(c->dev))
        return PINFER_E_ARG;
    c->ck_n_past = c->n_past;
    c->ck_mtp_rows = mtp_rows(c);
    c->ck_valid = 1;
    return PINFER_OK;
}

int pinfer_rewind(pinfer_ctx *c) {
    if (!c || !c->ck_valid) return PINFER_E_ARG;
    if (c->n_past < c->ck_n_past) { /* cannot happen through the API */
        c->ck_valid = 0;
        return PINFER_E_ARG;
    }
    const size_t cb = (size_t)c->n_lin * conv_bytes(c), sb = (size_t)c->n_lin * rec_bytes(c);
    if ((cb && nmx_copy_d2d(c->dev, c->conv_state, c->ck_dev, cb)) ||
        (sb && nmx_copy_d2d(c->dev, c->rec, (char *)c->ck_dev + cb, sb)))
        return PINFER_E_ARG;
    c->n_past = c->ck_n_past;
    c->mtp_rows = c->ck_mtp_rows;
    c->keep = 0;
    if (nmx_ctl_set(c->dev, c->ctl, 0, c->n_past) || nmx_ctl_set(c->dev, c->ctl, 2, 0) ||
        nmx_sync(c->dev))
        return PINFER_E_ARG;
    return PINFER_OK;
}

void pinfer_checkpoint_clear(pinfer_ctx *c) {
    if (!c) return;
    if (c->ck_dev) nmx_free(c->dev, c->ck_dev);
    c->ck_dev = NULL;
    c->ck_valid = 0;
}

int pinfer_checkpoint_n_past(const pinfer_ctx *c) { return c && c->ck_valid ? c->ck_n_past : -1; }
