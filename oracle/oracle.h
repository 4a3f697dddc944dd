/* ORACLE — test infrastructure only.
 *
 * A portable scalar C11 restatement of the reference engine's arithmetic on the speculative
 * verify path (nibblemac, engine/src). Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it, and only as the checker or the timed CPU baseline; the product
 * (nibblemac_amd) never links, loads or calls it.
 *
 * Compiled with -O2 -std=c11 -ffp-contract=off (no contraction: every a*b+c rounds twice
 * unless the reference itself fuses, where the code calls fmaf explicitly).
 *
 * How each function is pinned (tests/test_oracle_*.py):
 *   orc_get6 / orc_q4k_get_row      FORMAT.md bit layout; closed-form identity-input test
 *                                   (engine/metal/check.c:147-201 restated) over all 64
 *                                   sub-scale / sub-min values and both nibble halves
 *   orc_quant_a8                    closed forms (amax, codes, d, fsum) on hand-built blocks;
 *                                   round-half-even cases; numpy vectorised restatement
 *   orc_q4k_matmul                  int64 brute force of every sub-block dot; tolerance
 *                                   vs a float64 dequantised reference (< 1e-5,
 *                                   engine/bench/kbench_util.c:223-227); batch == single;
 *                                   planted-mistake checks (dropped min term, swapped nibbles)
 *   orc_lin_rule / orc_lin_apply    oracle/_ref (the reference's own matvec_ref.c, compiled
 *                                   from its sources) bit for bit; closed-form rank-1 update;
 *                                   replay == direct run
 *   orc_argmax / orc_accept         brute force; oracle/_ref pf_argmax
 *   orc_expf_cephes                 oracle/_ref pf_expf bit for bit over a dense sweep
 *   orc_top1_prob                   oracle/_ref pf_softmax_max + pf_softmax_exp on random and
 *                                   peaked rows; one-hot closed form (p = 1)
 *   orc_q4k_quantize                numpy restatement byte-for-byte; dequantised error bound
 */
#ifndef NMX_ORACLE_H
#define NMX_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- binary16 ------------------------------------------------------------------------ */
uint16_t orc_f32_to_f16(float f); /* round to nearest even, subnormals, inf/NaN */
float orc_f16_to_f32(uint16_t h);

/* ---- Q4K_G32 packed matrices (engine/src/pq_quant.h, engine/FORMAT.md:107-136) -------- */
size_t orc_q4k_nbytes(int rows, int cols);
int orc_get6(const uint8_t *p, int j);
void orc_q4k_get_row(const uint8_t *W, int rows, int cols, int row, float *dst);
/* Seeded benchmark quantizer: a restatement of engine/bench/kbench_util.c:100-132
 * (pack_q4k_sb): min/max per group, 6-bit sub-scales under per-row fp16 maxima. */
void orc_q4k_quantize(const float *w, int rows, int cols, uint8_t *out);

/* ---- A8 activations (engine/src/kern_act.c:14-42) ------------------------------------ */
void orc_quant_a8(const float *X, int n, int cols, int8_t *q, float *d, float *fsum);

/* ---- Q4K x A8 matmul (engine/src/kern_quant.c:148-245,296-304) ------------------------
 * Y [n][rows]; dots (may be NULL) receives the int32 sub-block sums [n][rows][cols/32]. */
void orc_q4k_matmul(const uint8_t *W, int rows, int cols, const int8_t *q, const float *d,
                    const float *fsum, int n, float *Y, int32_t *dots);
/* Row range [r0, r1) only (multiples of 4), for the threaded CPU baseline. */
void orc_q4k_matmul_rows(const uint8_t *W, int rows, int cols, const int8_t *q, const float *d,
                         const float *fsum, int n, float *Y, int r0, int r1);
/* The same split over `threads` pthreads (whole 4-row tiles: identical bits). */
void orc_q4k_matmul_mt(const uint8_t *W, int rows, int cols, const int8_t *q, const float *d,
                       const float *fsum, int n, float *Y, int threads);

/* ---- Gated DeltaNet recurrence (engine/src/matvec_ref.c:114-188, ops.h:54-93) ----------
 * S is [heads][dk][dv] row-major (row = key index). log rows are [n][heads][dk + dv + 1]
 * (k | delta | decay); pend rows [keep][heads][dk + dv + 1].
 * log0 = 0: reference semantics (token 0 in place, tokens 1.. on a copy, log rows t >= 1).
 * log0 = 1: S is left after the pending updates only and every token 0..n-1 is logged, so
 *           any prefix 0..n can be committed by replay (extension, no reference counterpart). */
typedef struct {
    int n, heads, rep, dk, dv;
    int qkv_stride, o_stride;
    const float *qkv;
    const float *decay, *beta;
    float *S;
    float *o;
    float *log;        /* NULL = plain pass */
    const float *pend; /* NULL when keep == 0 */
    int keep;
    int log0;
} orc_lin_args;
void orc_lin_rule(const orc_lin_args *a);
void orc_lin_apply(float *S, const float *log, int keep, int heads, int dk, int dv);

/* ---- argmax + acceptance (engine/src/forward_ops.c:387-409, spec.c:337-351) ----------- */
int orc_argmax(const float *v, int n);
/* logits [k+1][V]; drafts d[0..k-1] (the verify row t+1 token); returns a (accepted drafts),
 * *bonus = argmax of row a, argmax_rows[0..k] (may be NULL) = argmax of every row. */
int orc_accept(const float *logits, int V, const int32_t *drafts, int k, int32_t *bonus,
               int32_t *argmax_rows);

/* ---- scalar primitives of the forward pass (engine/src/forward_ops.c) ------------------- */
float orc_expf_cephes(float x); /* pf_expf, forward_ops.c:41-56 */
/* top-1 softmax probability of l[0, n) (spec.c:93-97 top1_prob over pf_softmax_max /
 * pf_softmax_exp, forward_ops.c:294-353): p = s > 0 ? 1 / s : 0 */
float orc_top1_prob(const float *l, int n);

/* exp / log1p for the DeltaNet gates: the reference calls libm expf / log1pf
 * (forward_lin.c:18-19,59-66); these restate this platform's (glibc 2.35 on x86-64: Arm's
 * optimized-routines expf as glibc's FMA build runs it, fdlibm's log1pf) operation for
 * operation. orc_libm_mismatches counts the inputs on which they differ from the host's
 * functions over all 2^32 bit patterns (which: 0 expf, 1 log1pf); orc_libm_eval writes the
 * host's values for the inputs with bit patterns first .. first + n - 1 (threads threads);
 * orc_exp2_tab is entry i of expf's 2^(i/32) table. */
float orc_gate_expf(float x);
float orc_gate_log1pf(float x);
long long orc_libm_mismatches(int which, int threads);
void orc_libm_eval(int which, uint32_t first, long n, float *y, int threads);
uint64_t orc_exp2_tab(int i);

#ifdef __cplusplus
}
#endif
#endif
