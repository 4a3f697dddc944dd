/* .pq loader for the MI355X engine: map the file, validate the header and the whole tensor
 * directory against the file size before any weight is touched (the checks of the reference
 * loader, engine/src/model.c:60-202, restated), then upload the data section to HBM in one copy
 * and build per-layer device views. Every 2-D weight must be Q4K_G32 (the dtype of this
 * engine's kernels); vectors are F32. */
#define _GNU_SOURCE
#include <fcntl.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "engine.h"

/* On-disk structures (engine/FORMAT.md "Header", "Tensor directory entry"). */
typedef struct {
    char magic[8];
    uint32_t version, n_tensors;
    uint64_t dir_offset, data_offset;
    uint32_t arch, hidden, n_layers, vocab, ffn;
    uint32_t n_heads, n_kv_heads, head_dim, rot_dim;
    uint32_t lin_k_heads, lin_v_heads, lin_k_dim, lin_v_dim, conv_k;
    uint32_t full_attn_mask, eos_id, tied_embeddings, has_mtp;
    float rms_eps, rope_theta;
} pq_hdr;

typedef struct {
    char name[80];
    uint32_t dtype, ndim, shape[4];
    uint64_t offset, nbytes;
    uint8_t reserved[8];
} pq_entry;

_Static_assert(sizeof(pq_hdr) == 112, "pq header layout");
_Static_assert(sizeof(pq_entry) == 128, "pq entry layout");

#define FAIL(...)                                                                             \
    do {                                                                                      \
        fprintf(stderr, "pinfer: " __VA_ARGS__);                                              \
        fputc('\n', stderr);                                                                  \
        return PINFER_E_FORMAT;                                                               \
    } while (0)

typedef struct {
    const uint8_t *map;
    size_t size;
    const pq_hdr *h;
    const pq_entry *dir;
    const uint8_t *dev_base; /* device address of map + data_offset */
} loader;

static const pq_entry *find(const loader *L, const char *name) {
    for (uint32_t i = 0; i < L->h->n_tensors; i++)
        if (strcmp(L->dir[i].name, name) == 0) return &L->dir[i];
    return NULL;
}

/* bytes the dtype and shape imply, built factor by factor against the file size */
static int entry_bytes(const pq_entry *e, uint64_t limit, uint64_t *bytes) {
    const uint64_t es = e->dtype == PQ_F32 ? 4 : e->dtype == PQ_BF16 ? 2 : 0;
    if (es) {
        uint64_t n = es;
        for (uint32_t d = 0; d < e->ndim; d++) {
            if (!e->shape[d]) FAIL("%s: zero dimension", e->name);
            if (n > limit / e->shape[d]) FAIL("%s: shape larger than the file", e->name);
            n *= e->shape[d];
        }
        *bytes = n;
        return PINFER_OK;
    }
    if (e->dtype < 2 || e->dtype > 4) FAIL("%s: unknown dtype %u", e->name, e->dtype);
    const uint64_t rows = e->shape[0], cols = e->shape[1];
    if (e->ndim != 2 || !rows || !cols || rows % 4 || cols % 256)
        FAIL("%s: quantized dtype %u needs a [rows %% 4, cols %% 256] matrix", e->name, e->dtype);
    const uint64_t sb = e->dtype == 2 ? 1088 : 576, tiles = rows / 4 * (cols / 256);
    if (tiles > limit / sb) FAIL("%s: shape larger than the file", e->name);
    *bytes = tiles * sb;
    return PINFER_OK;
}

static int check_header(const pq_hdr *h) {
    if (memcmp(h->magic, "PINFERQ", 8) != 0) FAIL("bad magic");
    if (h->version != 1) FAIL("unsupported version %u", h->version);
    if (h->arch != 1) FAIL("unsupported arch %u", h->arch);
    if (!h->hidden || h->hidden > 65536 || !h->ffn || h->ffn > 65536 || !h->vocab ||
        h->vocab > (1u << 21) || !h->n_layers || h->n_layers > 32)
        FAIL("bad model dimensions");
    if (h->eos_id >= h->vocab) FAIL("eos_id %u outside the vocabulary", h->eos_id);
    if (!h->n_heads || h->n_heads > 256 || !h->n_kv_heads || h->n_heads % h->n_kv_heads ||
        !h->head_dim || h->head_dim > 1024 || h->rot_dim % 2 || h->rot_dim > h->head_dim)
        FAIL("bad attention dimensions");
    if (!h->lin_k_heads || h->lin_k_heads > 256 || !h->lin_v_heads || h->lin_v_heads > 256 ||
        h->lin_v_heads % h->lin_k_heads || !h->lin_k_dim || h->lin_k_dim > 1024 ||
        !h->lin_v_dim || h->lin_v_dim > 1024 || h->conv_k < 1 || h->conv_k > 8)
        FAIL("bad linear-attention dimensions");
    if (h->tied_embeddings > 1) FAIL("bad tied_embeddings %u", h->tied_embeddings);
    if (!(h->rms_eps > 0.0f) || !isfinite(h->rms_eps) || !(h->rope_theta > 0.0f) ||
        !isfinite(h->rope_theta))
        FAIL("bad eps / rope_theta");
    return PINFER_OK;
}

static int check_directory(loader *L) {
    const pq_hdr *h = L->h;
    const uint64_t size = L->size;
    if (h->dir_offset < sizeof(pq_hdr) || h->dir_offset > size || h->dir_offset % 8 ||
        (uint64_t)h->n_tensors * sizeof(pq_entry) > size - h->dir_offset)
        FAIL("tensor directory out of bounds or misaligned");
    if (h->data_offset > size) FAIL("data_offset out of bounds");
    L->dir = (const pq_entry *)(L->map + h->dir_offset);
    for (uint32_t i = 0; i < h->n_tensors; i++) {
        const pq_entry *e = &L->dir[i];
        if (!memchr(e->name, 0, sizeof e->name)) FAIL("tensor %u: name not terminated", i);
        if (e->ndim < 1 || e->ndim > 4) FAIL("%s: bad ndim %u", e->name, e->ndim);
        if (e->offset % 64 || e->offset < h->data_offset || e->offset > size ||
            e->nbytes > size - e->offset)
            FAIL("%s: data out of bounds or misaligned", e->name);
        uint64_t want = 0;
        if (entry_bytes(e, size, &want) != PINFER_OK) return PINFER_E_FORMAT;
        if (want != e->nbytes) FAIL("%s: nbytes %llu != %llu", e->name,
                                    (unsigned long long)e->nbytes, (unsigned long long)want);
    }
    return PINFER_OK;
}

static const void *dev_ptr(const loader *L, const pq_entry *e) {
    return L->dev_base + (e->offset - L->h->data_offset);
}

static int vec(const loader *L, const char *name, uint32_t n, const float **out) {
    const pq_entry *e = find(L, name);
    if (!e) FAIL("missing tensor %s", name);
    if (e->dtype != PQ_F32 || e->ndim != 1 || e->shape[0] != n) FAIL("%s: expected F32 [%u]", name, n);
    *out = (const float *)dev_ptr(L, e);
    return PINFER_OK;
}

static int mat(const loader *L, const char *name, uint32_t rows, uint32_t cols, e_mat *out) {
    const pq_entry *e = find(L, name);
    if (!e) FAIL("missing tensor %s", name);
    if (e->ndim != 2 || e->shape[0] != rows || e->shape[1] != cols)
        FAIL("%s: expected shape [%u, %u]", name, rows, cols);
    if (e->dtype != PQ_Q4K) FAIL("%s: dtype %u not supported (this engine runs Q4K_G32)", name, e->dtype);
    out->w = dev_ptr(L, e);
    out->rows = (int)rows;
    out->cols = (int)cols;
    return PINFER_OK;
}

static int full_block(const loader *L, const char *p, e_layer *Ly, const pq_hdr *h) {
    char nm[160];
    int rc = 0;
    const uint32_t H = h->hidden, hd = h->head_dim;
#define N(s) (snprintf(nm, sizeof nm, "%s%s", p, s), nm)
    rc |= mat(L, N("self_attn.q_proj.weight"), h->n_heads * hd * 2, H, &Ly->q);
    rc |= mat(L, N("self_attn.k_proj.weight"), h->n_kv_heads * hd, H, &Ly->k);
    rc |= mat(L, N("self_attn.v_proj.weight"), h->n_kv_heads * hd, H, &Ly->v);
    rc |= mat(L, N("self_attn.o_proj.weight"), H, h->n_heads * hd, &Ly->o);
    rc |= vec(L, N("self_attn.q_norm.weight"), hd, &Ly->q_norm);
    rc |= vec(L, N("self_attn.k_norm.weight"), hd, &Ly->k_norm);
#undef N
    return rc ? PINFER_E_FORMAT : PINFER_OK;
}

static int common_block(const loader *L, const char *p, e_layer *Ly, const pq_hdr *h) {
    char nm[160];
    int rc = 0;
    const uint32_t H = h->hidden;
#define N(s) (snprintf(nm, sizeof nm, "%s%s", p, s), nm)
    rc |= vec(L, N("input_layernorm.weight"), H, &Ly->in_norm);
    rc |= vec(L, N("post_attention_layernorm.weight"), H, &Ly->post_norm);
    rc |= mat(L, N("mlp.gate_proj.weight"), h->ffn, H, &Ly->gate);
    rc |= mat(L, N("mlp.up_proj.weight"), h->ffn, H, &Ly->up);
    rc |= mat(L, N("mlp.down_proj.weight"), H, h->ffn, &Ly->down);
#undef N
    return rc ? PINFER_E_FORMAT : PINFER_OK;
}

/* engine/src/model.c:156-202 */
static int build_layer(const loader *L, int i, e_layer *Ly, pinfer_ctx *c) {
    const pq_hdr *h = L->h;
    char p[64], nm[160];
    snprintf(p, sizeof p, "layers.%d.", i);
    Ly->is_full = (h->full_attn_mask >> i) & 1;
    Ly->lin = Ly->full = -1;
    if (common_block(L, p, Ly, h)) return PINFER_E_FORMAT;
    if (Ly->is_full) {
        Ly->full = c->n_full++;
        return full_block(L, p, Ly, h);
    }
    Ly->lin = c->n_lin++;
    const uint32_t kd = h->lin_k_heads * h->lin_k_dim, vd = h->lin_v_heads * h->lin_v_dim;
    const uint32_t C = 2 * kd + vd, H = h->hidden;
    int rc = 0;
#define N(s) (snprintf(nm, sizeof nm, "%s%s", p, s), nm)
    rc |= mat(L, N("linear_attn.in_proj_qkv.weight"), C, H, &Ly->qkv);
    rc |= mat(L, N("linear_attn.in_proj_z.weight"), vd, H, &Ly->z);
    rc |= mat(L, N("linear_attn.in_proj_b.weight"), h->lin_v_heads, H, &Ly->b);
    rc |= mat(L, N("linear_attn.in_proj_a.weight"), h->lin_v_heads, H, &Ly->a);
    rc |= mat(L, N("linear_attn.out_proj.weight"), H, vd, &Ly->out);
    const int has_a = find(L, N("linear_attn.A")) != NULL;
    if (has_a && find(L, N("linear_attn.A_log"))) FAIL("layer %d: both linear_attn.A and A_log", i);
    if (has_a) rc |= vec(L, N("linear_attn.A"), h->lin_v_heads, &Ly->A);
    else rc |= vec(L, N("linear_attn.A_log"), h->lin_v_heads, &Ly->A_log);
    rc |= vec(L, N("linear_attn.dt_bias"), h->lin_v_heads, &Ly->dt_bias);
    rc |= vec(L, N("linear_attn.norm.weight"), h->lin_v_dim, &Ly->lin_norm);
    const pq_entry *e = find(L, N("linear_attn.conv1d.weight"));
#undef N
    if (!e || e->dtype != PQ_F32 || e->ndim != 2 || e->shape[0] != C || e->shape[1] != h->conv_k)
        FAIL("layer %d: bad or missing conv1d.weight", i);
    Ly->conv_w = (const float *)dev_ptr(L, e);
    return rc ? PINFER_E_FORMAT : PINFER_OK;
}

static int map_mtp(const loader *L, pinfer_ctx *c) {
    const pq_hdr *h = L->h;
    const uint32_t H = h->hidden;
    int rc = 0;
    rc |= mat(L, "mtp.fc.weight", H, 2 * H, &c->mtp_fc);
    rc |= vec(L, "mtp.pre_fc_norm_embedding.weight", H, &c->mtp_norm_emb);
    rc |= vec(L, "mtp.pre_fc_norm_hidden.weight", H, &c->mtp_norm_hid);
    rc |= vec(L, "mtp.norm.weight", H, &c->mtp_norm_out);
    c->mtp.is_full = 1;
    c->mtp.lin = -1;
    c->mtp.full = 0;
    rc |= common_block(L, "mtp.layers.0.", &c->mtp, h);
    rc |= full_block(L, "mtp.layers.0.", &c->mtp, h);
    return rc ? PINFER_E_FORMAT : PINFER_OK;
}

/* 64-bit FNV-1a (offset basis 14695981039346656037, prime 1099511628211) */
static uint64_t fnv1a(uint64_t h, const void *p, size_t n) {
    const unsigned char *b = p;
    for (size_t i = 0; i < n; i++) h = (h ^ b[i]) * 1099511628211ull;
    return h;
}

/* The model fingerprint a state blob carries (engine/src/model.c:142-154): FNV-1a over the
 * header, the directory, and the first, middle and last 64 bytes of every tensor. */
static uint64_t fingerprint(const loader *L) {
    const pq_hdr *h = L->h;
    uint64_t f = fnv1a(14695981039346656037ull, h, sizeof(pq_hdr));
    const uint8_t *dir = L->map + h->dir_offset;
    f = fnv1a(f, dir, (size_t)h->n_tensors * sizeof(pq_entry));
    for (uint32_t i = 0; i < h->n_tensors; i++) {
        const pq_entry *e = (const pq_entry *)(dir + (size_t)i * sizeof(pq_entry));
        const unsigned char *d = (const unsigned char *)L->map + e->offset;
        const size_t n = (size_t)e->nbytes, s = n < 64 ? n : 64;
        f = fnv1a(f, d, s);
        f = fnv1a(f, d + (n - s) / 2, s);
        f = fnv1a(f, d + (n - s), s);
    }
    return f;
}

/* upload = 0: every check and view of the load with no device call (the views point into a
 * dummy base that is never dereferenced), so a file is refused before a device is touched. */
static int model_load(pinfer_ctx *c, const char *path, int upload) {
    int fd = open(path, O_RDONLY);
    if (fd < 0) {
        perror(path);
        return PINFER_E_IO;
    }
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 4096) {
        close(fd);
        fprintf(stderr, "pinfer: %s: too small for a .pq file\n", path);
        return PINFER_E_FORMAT;
    }
    void *map = mmap(NULL, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) {
        perror("mmap");
        return PINFER_E_IO;
    }
    loader L = {map, (size_t)st.st_size, map, NULL, NULL};
    int rc = check_header(L.h);
    if (rc == PINFER_OK) rc = check_directory(&L);
    const pq_hdr *h = L.h;
    if (rc == PINFER_OK) {
        /* engine limits: the reference's (engine/src/pinfer.c:152-156) and the kernels' */
        const int dk = (int)h->lin_k_dim;
        if (h->lin_v_dim > 512 || h->lin_v_dim % 32 || h->head_dim > 512 || h->head_dim % 64 ||
            (dk != 32 && dk != 64 && dk != 128 && dk != 256) || h->hidden % 256 || h->ffn % 256 ||
            (h->lin_v_heads * h->lin_v_dim) % 256 || (h->n_heads * h->head_dim) % 256 ||
            h->vocab % 4) {
            fprintf(stderr, "pinfer: dimensions not supported by the MI355X kernels\n");
            rc = PINFER_E_FORMAT;
        }
    }
    if (rc == PINFER_OK && upload) {
        const size_t bytes = L.size - h->data_offset;
        c->blob = nmx_alloc(c->dev, bytes ? bytes : 1);
        if (!c->blob) rc = PINFER_E_NOMEM;
        else if (nmx_upload(c->dev, c->blob, L.map + h->data_offset, bytes)) rc = PINFER_E_NOMEM;
        L.dev_base = c->blob;
    } else if (rc == PINFER_OK) {
        L.dev_base = (const uint8_t *)(uintptr_t)4096;
    }
    if (rc == PINFER_OK) {
        c->H = (int)h->hidden;
        c->ffn = (int)h->ffn;
        c->n_layers = (int)h->n_layers;
        c->vocab = (int)h->vocab;
        c->n_heads = (int)h->n_heads;
        c->n_kv = (int)h->n_kv_heads;
        c->hd = (int)h->head_dim;
        c->rot = (int)h->rot_dim;
        c->lk_heads = (int)h->lin_k_heads;
        c->lv_heads = (int)h->lin_v_heads;
        c->lk_dim = (int)h->lin_k_dim;
        c->lv_dim = (int)h->lin_v_dim;
        c->conv_k = (int)h->conv_k;
        c->kd = c->lk_heads * c->lk_dim;
        c->vd = c->lv_heads * c->lv_dim;
        c->conv_dim = 2 * c->kd + c->vd;
        c->eos = (int)h->eos_id;
        c->rms_eps = h->rms_eps;
        c->rope_theta = h->rope_theta;
        c->has_mtp = (int)h->has_mtp;
        rc = mat(&L, "embed_tokens.weight", h->vocab, h->hidden, &c->embed);
        c->head = c->embed;
        if (rc == PINFER_OK && !h->tied_embeddings)
            rc = mat(&L, "lm_head.weight", h->vocab, h->hidden, &c->head);
        if (rc == PINFER_OK) rc = vec(&L, "norm.weight", h->hidden, &c->norm);
    }
    if (rc == PINFER_OK) {
        c->layers = calloc(h->n_layers, sizeof(e_layer));
        if (!c->layers) rc = PINFER_E_NOMEM;
    }
    for (uint32_t i = 0; rc == PINFER_OK && i < h->n_layers; i++)
        rc = build_layer(&L, (int)i, &c->layers[i], c);
    if (rc == PINFER_OK && c->has_mtp) rc = map_mtp(&L, c);
    if (rc == PINFER_OK) c->model_fp = fingerprint(&L);
    munmap(map, L.size);
    return rc;
}

int e_model_check(const char *path) {
    pinfer_ctx *t = calloc(1, sizeof *t);
    if (!t) return PINFER_E_NOMEM;
    const int rc = model_load(t, path, 0);
    free(t->layers);
    free(t);
    return rc;
}

int e_model_load(pinfer_ctx *c, const char *path) { return model_load(c, path, 1); }
