/* The reference engine's operator contract (engine/src/ops.h:14-95) on the MI355X kernels of
 * libnmx.so: a drop-in for engine/src/matvec_ref.c / matvec_fast.c that keeps the reference's
 * C forward pass, DeltaNet mixer, rollback log and speculative loop and runs their matrix
 * products (pf_matmul / pf_matvec) and the DeltaNet recurrence (pf_lin_rule / pf_lin_apply) on
 * the device.
 *
 * Build inside the reference tree: place this file in engine/src/, accept `nmx` as a MATVEC
 * value (engine/Makefile:12-15), and compile with -I<this repo>/include -ffp-contract=off,
 * linking -lnmx from nibblemac_amd/lib.
 *
 * Weights: each Q4K_G32 matrix is uploaded on its first product (or by pf_pool_gpu_enable) and
 * stays on the device until pf_pool_destroy; a matrix is identified by its data pointer, so
 * the matrices must stay mapped and unchanged while the pool lives (the engine destroys its
 * pool before it frees the model, engine/src/pinfer.c:185-186).
 * Activations and the recurrent state stay where the engine keeps them, in host memory: the
 * engine's own code reads and writes them directly (pinfer_reset zeroes the state,
 * engine/src/pinfer.c:196; the state blob copies it, state.c:89-90). Every call therefore
 * stages its inputs to the device and its outputs back, synchronously; that PCIe traffic
 * bounds this integration, while libpinfer.so keeps the whole verify round on the device.
 * The recurrent state has the device kernels' layout (nmx_state_index; ops.h:74-75 leaves the
 * layout to the implementation), so state blobs of this build hold that layout.
 * Results are bit-identical to the reference's operators (same fp32 roundings, in the same
 * order); the contract has no error return, so a device failure prints the nmx error and
 * aborts. Work handed to pf_pool_run runs on the calling thread. */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "nmx.h"
#include "ops.h"
#include "pq_quant.h"

#define PLUG_MAX_N 64      /* vectors per nmx_q4k_matmul and tokens per nmx_lin_rule call */
#define PLUG_ALIGN 256

typedef struct {
    const void *host;
    void *dev;
    int rows; /* rows of the device copy */
} plug_weight;

struct pf_pool {
    nmx_ctx *dev;
    plug_weight *w;
    int n_w, cap_w;
    char *stage;           /* device staging, grown on demand */
    size_t stage_cap;
};

static void plug_die(pf_pool *p, const char *what) {
    fprintf(stderr, "matvec_nmx: %s: %s\n", what, p && p->dev ? nmx_error(p->dev) : "");
    abort();
}

/* Offset of the next staging slice of `bytes`, advancing *end. */
static size_t slice(size_t *end, size_t bytes) {
    const size_t o = *end;
    *end += (bytes + PLUG_ALIGN - 1) / PLUG_ALIGN * PLUG_ALIGN;
    return o;
}

static char *staging(pf_pool *p, size_t bytes) {
    if (bytes > p->stage_cap) {
        const size_t cap = (bytes + (1u << 20) - 1) & ~(size_t)((1u << 20) - 1);
        if (p->stage && nmx_free(p->dev, p->stage)) plug_die(p, "free staging");
        p->stage = nmx_alloc(p->dev, cap);
        if (!p->stage) plug_die(p, "staging allocation");
        p->stage_cap = cap;
    }
    return p->stage;
}

static void up(pf_pool *p, void *dst, const void *src, size_t bytes) {
    if (nmx_upload(p->dev, dst, src, bytes)) plug_die(p, "upload");
}

static void down(pf_pool *p, void *dst, const void *src, size_t bytes) {
    if (nmx_download(p->dev, dst, src, bytes)) plug_die(p, "download");
}

static size_t q4k_bytes(const pf_mat *W) {
    return (size_t)(W->rows / 4) * (size_t)(W->cols / PQ_SB_COLS) * pq_sb_bytes(PQ_Q4K_G32);
}

/* Device copy of W, uploaded on first use. The same host data may come with fewer rows (the
 * MTP draft head passes the head's data with rows = draft vocabulary, engine/src/mtp.c:94-95):
 * a copy serves every request of at most its rows, and a request of more rows replaces it. */
static void *weights(pf_pool *p, const pf_mat *W) {
    int slot = -1;
    for (int i = p->n_w - 1; i >= 0 && slot < 0; i--)
        if (p->w[i].host == W->data) slot = i;
    if (slot >= 0 && p->w[slot].rows >= W->rows) return p->w[slot].dev;
    if (W->dtype != PQ_Q4K_G32 || W->rows % 4 || W->cols % PQ_SB_COLS) {
        fprintf(stderr, "matvec_nmx: matrix %dx%d of dtype %u: only Q4K_G32 with rows %% 4 == 0 "
                "and cols %% %d == 0 runs on the device\n", W->rows, W->cols, W->dtype, PQ_SB_COLS);
        abort();
    }
    if (slot >= 0) { /* more rows than the cached copy: upload the larger one in its place */
        if (nmx_free(p->dev, p->w[slot].dev)) plug_die(p, "free weights");
        const size_t bytes = q4k_bytes(W);
        void *d = nmx_alloc(p->dev, bytes);
        if (!d) plug_die(p, "weight allocation");
        up(p, d, W->data, bytes);
        p->w[slot].dev = d;
        p->w[slot].rows = W->rows;
        return d;
    }
    if (p->n_w == p->cap_w) {
        const int cap = p->cap_w ? 2 * p->cap_w : 256;
        plug_weight *w = realloc(p->w, (size_t)cap * sizeof *w);
        if (!w) plug_die(p, "weight table");
        p->w = w;
        p->cap_w = cap;
    }
    const size_t bytes = q4k_bytes(W);
    void *d = nmx_alloc(p->dev, bytes);
    if (!d) plug_die(p, "weight allocation");
    up(p, d, W->data, bytes);
    p->w[p->n_w].host = W->data;
    p->w[p->n_w].dev = d;
    p->w[p->n_w].rows = W->rows;
    p->n_w++;
    return d;
}

pf_pool *pf_pool_create(int n_threads) {
    (void)n_threads;
    pf_pool *p = calloc(1, sizeof *p);
    if (!p) return NULL;
    const char *dv = getenv("PINFER_DEVICE");
    p->dev = nmx_create(dv ? atoi(dv) : 0);
    if (!p->dev) {
        fprintf(stderr, "matvec_nmx: %s\n", nmx_create_error());
        free(p);
        return NULL;
    }
    return p;
}

void pf_pool_destroy(pf_pool *p) {
    if (!p) return;
    nmx_sync(p->dev);
    for (int i = 0; i < p->n_w; i++) nmx_free(p->dev, p->w[i].dev);
    if (p->stage) nmx_free(p->dev, p->stage);
    nmx_destroy(p->dev);
    free(p->w);
    free(p);
}

int pf_pool_threads(const pf_pool *p) {
    (void)p;
    return 1;
}

void *pf_pool_state_alloc(pf_pool *p, size_t bytes) {
    (void)p;
    return calloc(1, bytes);
}

void pf_pool_state_free(pf_pool *p, void *state) {
    (void)p;
    free(state);
}

/* Declined: the engine's unfused MLP (three pf_matmul calls around its own SiLU) runs. */
int pf_pool_mlp(pf_pool *p, const pf_mat *gate, const pf_mat *up_, const pf_mat *down_,
                const float *x, float *y, int n) {
    (void)p; (void)gate; (void)up_; (void)down_; (void)x; (void)y; (void)n;
    return 0;
}

/* Uploads the listed matrices now (the rest follow on first use); HBM holds a whole model, so
 * `share` is not needed. */
int pf_pool_gpu_enable(pf_pool *p, const pf_mat *const *w, int count, float share) {
    (void)share;
    for (int i = 0; i < count; i++)
        if (w[i]->dtype == PQ_Q4K_G32) weights(p, w[i]);
    return 0;
}

/* Every product runs on the device, the verify pass included. */
void pf_pool_gpu_pause(pf_pool *p, int pause) {
    (void)p;
    (void)pause;
}

void pf_pool_run(pf_pool *p, pf_task fn, void *arg, int max_threads) {
    (void)p;
    (void)max_threads;
    fn(arg, 0, 1);
}

int pf_dtype_supported(uint32_t dtype) { return dtype == PQ_Q4K_G32; }

void pf_matmul(pf_pool *p, const pf_mat *W, const float *X, float *Y, int n) {
    void *w = weights(p, W);
    const int rows = W->rows, cols = W->cols, nb = cols / 32;
    for (int t0 = 0; t0 < n; t0 += PLUG_MAX_N) {
        const int m = n - t0 < PLUG_MAX_N ? n - t0 : PLUG_MAX_N;
        size_t end = 0;
        const size_t ox = slice(&end, (size_t)m * cols * 4), oq = slice(&end, (size_t)m * cols),
                     od = slice(&end, (size_t)m * nb * 4), of = slice(&end, (size_t)m * nb * 4),
                     oy = slice(&end, (size_t)m * rows * 4);
        char *b = staging(p, end);
        up(p, b + ox, X + (size_t)t0 * cols, (size_t)m * cols * 4);
        if (nmx_quant_a8(p->dev, (const float *)(b + ox), m, cols, (int8_t *)(b + oq),
                         (float *)(b + od), (float *)(b + of)) ||
            nmx_q4k_matmul(p->dev, w, rows, cols, m, (const int8_t *)(b + oq),
                           (const float *)(b + od), (const float *)(b + of), (float *)(b + oy),
                           rows, NULL))
            plug_die(p, "pf_matmul");
        down(p, Y + (size_t)t0 * rows, b + oy, (size_t)m * rows * 4);
    }
}

void pf_matvec(pf_pool *p, const pf_mat *W, const float *x, float *y) { pf_matmul(p, W, x, y, 1); }

/* IEEE binary16 bits -> float (exact). */
static float half_bits(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31u, man = h & 1023u;
    float f;
    if (e == 0) {
        f = (float)man * 0x1p-24f;     /* zero or subnormal: man * 2^-24, exact in fp32 */
        uint32_t u;
        memcpy(&u, &f, 4);
        u |= sign;
        memcpy(&f, &u, 4);
        return f;
    }
    const uint32_t u = sign | (e == 31 ? 0x7f800000u | man << 13 : (e + 112) << 23 | man << 13);
    memcpy(&f, &u, 4);
    return f;
}

/* Entry j (0..31) of a packed 6-bit array: low nibbles in bytes 0..15 (entries j and j + 16
 * share byte j % 16), then two high bits per entry in bytes 16..23 (entry j at bit 2 (j / 8) of
 * byte 16 + j % 8). */
static int six_bit(const uint8_t *a, int j) {
    const int lo = (a[j & 15] >> (j & 16 ? 4 : 0)) & 15;
    const int hi = (a[16 + (j & 7)] >> (2 * (j >> 3))) & 3;
    return lo | hi << 4;
}

/* Row `row` of a Q4K_G32 matrix, decoded on the host (the embedding lookup; kern_get_row_q,
 * engine/src/kern_act.c:53-88): per 32-column sub-block k of a superblock,
 * x = (D s_k) u - (M m_k) with D, M the row's fp16 scales and s_k, m_k its 6-bit sub-scales. */
void pf_get_row(const pf_mat *W, int row, float *dst) {
    if (W->dtype != PQ_Q4K_G32) {
        fprintf(stderr, "matvec_nmx: pf_get_row of dtype %u\n", W->dtype);
        abort();
    }
    const int nsb = W->cols / PQ_SB_COLS, r = row % 4;
    const size_t sbb = pq_sb_bytes(PQ_Q4K_G32);
    const uint8_t *sb = (const uint8_t *)W->data + (size_t)(row / 4) * nsb * sbb;
    for (int s = 0; s < nsb; s++, sb += sbb, dst += PQ_SB_COLS) {
        uint16_t dh, mh;
        memcpy(&dh, sb + 2 * r, 2);
        memcpy(&mh, sb + 2 * (4 + r), 2);
        const float D = half_bits(dh), M = half_bits(mh);
        for (int k = 0; k < 8; k++) {
            const float scale = D * (float)six_bit(sb + 16, 4 * k + r);
            const float minv = M * (float)six_bit(sb + 40, 4 * k + r);
            const uint8_t *u = sb + PQ_SB_SCALE_BYTES + 64 * k + 16 * r;
            for (int j = 0; j < 16; j++) {
                dst[32 * k + j] = scale * (float)(u[j] & 15) - minv;
                dst[32 * k + 16 + j] = scale * (float)(u[j] >> 4) - minv;
            }
        }
    }
}

/* One nmx_lin_rule call over m <= PLUG_MAX_N tokens starting at token t0 of a; keep rows of
 * pend (the deferred commit) are applied first when keep > 0. */
static void lin_chunk(pf_pool *p, const pf_lin_args *a, int t0, int m, int keep) {
    const size_t row = (size_t)a->heads * (a->dk + a->dv + 1);
    const size_t sb = (size_t)a->heads * a->dk * a->dv * 4, qb = (size_t)m * a->qkv_stride * 4,
                 gb = (size_t)m * a->heads * 4, ob = (size_t)m * a->o_stride * 4,
                 lb = a->log ? (size_t)m * row * 4 : 0, pb = (size_t)keep * row * 4;
    size_t end = 0;
    const size_t oS = slice(&end, sb), oq = slice(&end, qb), od = slice(&end, gb),
                 ob_ = slice(&end, gb), oo = slice(&end, ob), ol = slice(&end, lb),
                 op = slice(&end, pb);
    char *b = staging(p, end);
    up(p, b + oS, a->S, sb);
    up(p, b + oq, a->qkv + (size_t)t0 * a->qkv_stride, qb);
    up(p, b + od, a->decay + (size_t)t0 * a->heads, gb);
    up(p, b + ob_, a->beta + (size_t)t0 * a->heads, gb);
    if (keep) up(p, b + op, a->pend, pb);
    nmx_lin_args g;
    memset(&g, 0, sizeof g);
    g.n = m;
    g.heads = a->heads;
    g.rep = a->rep;
    g.dk = a->dk;
    g.dv = a->dv;
    g.qkv_stride = a->qkv_stride;
    g.o_stride = a->o_stride;
    g.qkv = (const float *)(b + oq);
    g.decay = (const float *)(b + od);
    g.beta = (const float *)(b + ob_);
    g.S = (float *)(b + oS);
    g.o = (float *)(b + oo);
    g.log = a->log ? (float *)(b + ol) : NULL;   /* the reference's logged pass (log0 = 0) */
    g.pend = keep ? (const float *)(b + op) : NULL;
    g.keep = keep;
    if (nmx_lin_rule(p->dev, &g)) plug_die(p, "pf_lin_rule");
    down(p, a->S, b + oS, sb);
    float *o = a->o + (size_t)t0 * a->o_stride;
    const size_t width = (size_t)a->heads * a->dv * 4;
    if ((size_t)a->o_stride * 4 == width) down(p, o, b + oo, ob);
    else
        for (int t = 0; t < m; t++)
            down(p, o + (size_t)t * a->o_stride, b + oo + (size_t)t * a->o_stride * 4, width);
    if (a->log && m > 1)   /* rows 1..m-1; row 0 is not written */
        down(p, a->log + row, b + ol + row * 4, (size_t)(m - 1) * row * 4);
}

void pf_lin_rule(pf_pool *p, const pf_lin_args *a) {
    if (a->n <= 0 && a->keep <= 0) return;
    if (a->log && a->n > PLUG_MAX_N) {
        fprintf(stderr, "matvec_nmx: logged pass of %d tokens (at most %d)\n", a->n, PLUG_MAX_N);
        abort();
    }
    int keep = a->keep;
    if (keep > PLUG_MAX_N) {   /* the replay is sequential: apply the surplus first */
        pf_lin_apply(p, a->S, a->pend, keep - PLUG_MAX_N, a->heads, a->dk, a->dv);
        pf_lin_args b = *a;
        b.pend = a->pend + (size_t)(keep - PLUG_MAX_N) * a->heads * (a->dk + a->dv + 1);
        b.keep = PLUG_MAX_N;
        pf_lin_rule(p, &b);
        return;
    }
    if (a->n <= 0) {
        pf_lin_apply(p, a->S, a->pend, keep, a->heads, a->dk, a->dv);
        return;
    }
    /* Plain passes (prefill) are sequential in the tokens, so chunking them is exact. */
    for (int t0 = 0; t0 < a->n; t0 += PLUG_MAX_N) {
        const int m = a->n - t0 < PLUG_MAX_N ? a->n - t0 : PLUG_MAX_N;
        lin_chunk(p, a, t0, m, t0 == 0 ? keep : 0);
    }
}

void pf_lin_apply(pf_pool *p, float *S, const float *log, int keep, int heads, int dk, int dv) {
    const size_t row = (size_t)heads * (dk + dv + 1), sb = (size_t)heads * dk * dv * 4;
    for (int r0 = 0; r0 < keep; r0 += PLUG_MAX_N) {
        const int m = keep - r0 < PLUG_MAX_N ? keep - r0 : PLUG_MAX_N;
        size_t end = 0;
        const size_t oS = slice(&end, sb), ol = slice(&end, (size_t)m * row * 4);
        char *b = staging(p, end);
        up(p, b + oS, S, sb);
        up(p, b + ol, log + (size_t)r0 * row, (size_t)m * row * 4);
        if (nmx_lin_apply(p->dev, (float *)(b + oS), (const float *)(b + ol), m, heads, dk, dv))
            plug_die(p, "pf_lin_apply");
        down(p, S, b + oS, sb);
    }
}
