/* ORACLE — test infrastructure only (see oracle.h).
 *
 * An implementation of the reference engine's operator contract (engine/src/ops.h:14-95) for
 * the Q4K_G32 dtype, built from the oracle's restated kernels: pf_matmul = A8 quantization
 * (kern_act.c:14-42) + the exact Q4K x A8 product (kern_quant.c:148-245); pf_lin_rule /
 * pf_lin_apply = the scalar DeltaNet of matvec_ref.c:114-188; pf_get_row = kern_act.c:53-88.
 * `make -C oracle ref` links it with the reference's own forward pass, attention, DeltaNet
 * mixer + rollback log, MTP head and speculative loop (the engine/src C files minus the
 * kernel files, compiled from where they lie) into oracle/_ref/libpinfer_refq4k.so: the reference engine
 * running Q4K models on the CPU, the end-to-end checker of the MI355X engine. The DeltaNet gate
 * exp / log1p calls of those sources are bound to the oracle's binary64 versions (orc_num.c),
 * the values the device computes. */
#include <stdlib.h>
#include <string.h>

#include "ops.h"
#include "oracle.h"

struct pf_pool {
    int n_threads;
};

pf_pool *pf_pool_create(int n_threads) {
    pf_pool *p = malloc(sizeof *p);
    if (p) p->n_threads = n_threads < 1 ? 1 : n_threads;
    return p;
}
void pf_pool_destroy(pf_pool *pool) { free(pool); }
int pf_pool_threads(const pf_pool *pool) { (void)pool; return 1; }
void *pf_pool_state_alloc(pf_pool *pool, size_t bytes) { (void)pool; return calloc(1, bytes); }
void pf_pool_state_free(pf_pool *pool, void *state) { (void)pool; free(state); }
int pf_pool_mlp(pf_pool *pool, const pf_mat *gate, const pf_mat *up, const pf_mat *down,
                const float *x, float *y, int n) {
    (void)pool; (void)gate; (void)up; (void)down; (void)x; (void)y; (void)n;
    return 0;
}
int pf_pool_gpu_enable(pf_pool *pool, const pf_mat *const *weights, int count, float share) {
    (void)pool; (void)weights; (void)count; (void)share;
    return -1;
}
void pf_pool_gpu_pause(pf_pool *pool, int pause) { (void)pool; (void)pause; }
void pf_pool_run(pf_pool *pool, pf_task fn, void *arg, int max_threads) {
    (void)pool; (void)max_threads;
    fn(arg, 0, 1);
}

int pf_dtype_supported(uint32_t dtype) { return dtype == 4; }

void pf_matmul(pf_pool *pool, const pf_mat *W, const float *X, float *Y, int n) {
    const size_t nb = (size_t)W->cols / 32;
    int8_t *q = malloc((size_t)n * W->cols);
    float *d = malloc((size_t)n * nb * sizeof(float)), *fs = malloc((size_t)n * nb * sizeof(float));
    if (!q || !d || !fs) abort();
    orc_quant_a8(X, n, W->cols, q, d, fs);
    orc_q4k_matmul_mt(W->data, W->rows, W->cols, q, d, fs, n, Y, pool ? pool->n_threads : 1);
    free(q);
    free(d);
    free(fs);
}

void pf_matvec(pf_pool *pool, const pf_mat *W, const float *x, float *y) { pf_matmul(pool, W, x, y, 1); }

void pf_get_row(const pf_mat *W, int row, float *dst) {
    orc_q4k_get_row(W->data, W->rows, W->cols, row, dst);
}

void pf_lin_rule(pf_pool *pool, const pf_lin_args *a) {
    (void)pool;
    orc_lin_args o = {a->n, a->heads, a->rep, a->dk, a->dv, a->qkv_stride, a->o_stride, a->qkv,
                      a->decay, a->beta, a->S, a->o, a->log, a->pend, a->keep, 0};
    orc_lin_rule(&o);
}

void pf_lin_apply(pf_pool *pool, float *S, const float *log, int keep, int heads, int dk, int dv) {
    (void)pool;
    orc_lin_apply(S, log, keep, heads, dk, dv);
}
