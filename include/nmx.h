/* nmx — the MI355X (gfx950) device layer of nibblemac_amd: a thin C ABI over hand-written HIP
 * kernels for the speculative-verify path. Host code (C11) and the Python ctypes binding call
 * it; no torch, no CUDA types, plain pointers and sizes.
 *
 * Conventions (the same as the reference's device ABI, engine/metal/metal.h:1-72):
 *   - every call returns 0 on success and -1 on failure; nmx_error(ctx) holds the message;
 *   - shapes, sizes and aliasing are validated on the host BEFORE anything is enqueued, so an
 *     invalid call never reaches the GPU;
 *   - device pointers come from nmx_alloc (or any hipMalloc'd memory of the context's device);
 *   - work is enqueued on the context's stream and is asynchronous unless stated otherwise;
 *     nmx_sync waits; there is no silent CPU fallback (engine/metal/metal.h:5);
 *   - a context is used from one thread at a time (engine/metal/metal.h:4).
 *
 * Numerics are bit-exact restatements of the reference's CPU kernels (comments cite them).
 */
#ifndef NMX_H
#define NMX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct nmx_ctx nmx_ctx;
typedef struct nmx_event nmx_event;
typedef struct nmx_graph nmx_graph;

/* ---- context, memory, streams ----------------------------------------------------------
 * Replaces nm_metal_create / destroy / buffer_* (engine/metal/metal.h:18-26) and the
 * allocator hooks of the operator contract (pf_pool_state_alloc/free, engine/src/ops.h:26-29).
 */
nmx_ctx *nmx_create(int device);            /* NULL on failure (see nmx_create_error) */
const char *nmx_create_error(void);         /* message of the last failed nmx_create */
void nmx_destroy(nmx_ctx *ctx);
const char *nmx_error(const nmx_ctx *ctx);  /* last error of ctx ("" if none) */
const char *nmx_device_name(nmx_ctx *ctx);
int nmx_device_count(void);                 /* without creating a context; 0 if none */

void *nmx_alloc(nmx_ctx *ctx, size_t bytes);               /* device memory, NULL on failure */
int nmx_free(nmx_ctx *ctx, void *ptr);
/* Page-locked, coherent (fine-grained) host memory that kernels may write (hipHostMalloc with
 * hipHostMallocCoherent): the host may read it with no copy after a synchronisation, or poll a
 * flag that a kernel sets with a system-scope release while the stream still runs. No
 * counterpart in the reference, whose engine runs on the host. NULL on failure. */
void *nmx_host_alloc(nmx_ctx *ctx, size_t bytes);
int nmx_host_free(nmx_ctx *ctx, void *ptr);
int nmx_upload(nmx_ctx *ctx, void *dst, const void *src, size_t bytes);   /* synchronous */
int nmx_download(nmx_ctx *ctx, void *dst, const void *src, size_t bytes); /* synchronous */
int nmx_copy_d2d(nmx_ctx *ctx, void *dst, const void *src, size_t bytes); /* enqueued */
int nmx_fill_zero(nmx_ctx *ctx, void *dst, size_t bytes);  /* enqueued fill kernel */
int nmx_sync(nmx_ctx *ctx);

/* Timing on the context's stream (HIP events). */
nmx_event *nmx_event_create(nmx_ctx *ctx);
void nmx_event_destroy(nmx_event *ev);
int nmx_event_record(nmx_ctx *ctx, nmx_event *ev);
int nmx_event_elapsed_ms(nmx_ctx *ctx, nmx_event *start, nmx_event *stop, float *ms);

/* Stream capture into a HIP graph: every call enqueued between begin and end is recorded
 * instead of run; nmx_graph_launch replays it as one submit. */
int nmx_graph_begin(nmx_ctx *ctx);
nmx_graph *nmx_graph_end(nmx_ctx *ctx);
int nmx_graph_launch(nmx_ctx *ctx, nmx_graph *g);
void nmx_graph_destroy(nmx_graph *g);

/* ---- A8 activation quantization --------------------------------------------------------
 * Replaces kern_quant_act (engine/src/kern_act.c:14-42) / nm_quant_a8
 * (engine/metal/kernels.metal:9-27). X [n][cols] fp32, cols % 32 == 0 ->
 * q [cols/32][n][32] int8, d [cols/32][n], fsum [cols/32][n] (block-major, engine/src/kern.h:19-27).
 */
int nmx_quant_a8(nmx_ctx *ctx, const float *X, int n, int cols, int8_t *q, float *d,
                 float *fsum);

/* ---- Q4K_G32 x A8 matmul ---------------------------------------------------------------
 * Replaces pf_matmul / pf_matvec for PQ_Q4K_G32 (engine/src/ops.h:47-52, kern_q4k
 * engine/src/kern_quant.c:296-304) and nm_metal_matmul_a8 (engine/metal/metal.h:42-44).
 * W: .pq Q4K_G32 bytes [rows/4][cols/256][576] on the device (rows % 4 == 0, cols % 256 == 0).
 * A8 inputs as nmx_quant_a8 writes them for n vectors. Y [n][y_stride] fp32 (y_stride >= rows).
 * dots (may be NULL): int32 sub-block sums [n][rows][cols/32] (exactness checks).
 * n: 1..64 (split into register passes of <= 8 vectors; results do not depend on n).
 */
int nmx_q4k_matmul(nmx_ctx *ctx, const void *W, int rows, int cols, int n, const int8_t *q,
                   const float *d, const float *fsum, float *Y, int y_stride, int32_t *dots);

/* Several matrices that share one input (e.g. the in-projections of a layer) in one launch:
 * matrix s is W[s] [rows[s]][cols], output Y[s] [n][y_stride[s]]. count 1..NMX_MAX_SEGS. */
#define NMX_MAX_SEGS 6
int nmx_q4k_matmul_multi(nmx_ctx *ctx, int count, const void *const *W, const int *rows,
                         float *const *Y, const int *y_stride, int cols, int n,
                         const int8_t *q, const float *d, const float *fsum);

/* ---- Gated DeltaNet recurrence with the speculative rollback log -------------------------
 * Replaces pf_lin_rule / pf_lin_apply (engine/src/ops.h:54-93, matvec_ref.c:140-188,
 * kern_lin.c:155-185) and nm_metal_lin_rule / _apply (engine/metal/metal.h:66-71).
 * S: heads x dv x dk fp32 in HBM, element (head h, value column j, key i) at
 * nmx_state_index(h, j, i, dk, dv) below (the layout is private to this contract; zero =
 * reset). qkv [n][qkv_stride] = q | k (heads/rep heads of dk) | v (heads x dv);
 * decay, beta [n][heads]; o [n][o_stride]. log [n][heads][dk + dv + 1] = k | delta | decay.
 * log == NULL: plain pass, S advances by all n tokens.
 * log != NULL, log0 == 0 (the reference's logged pass): S advances by token 0 only; rows
 *   t >= 1 are logged (row 0 untouched); commit keeps e >= 1 tokens.
 * log != NULL, log0 == 1 (extension): S is left after the pending updates, every row 0..n-1 is
 *   logged, so any prefix 0..n can be committed by replay.
 * keep > 0: S first advances by the keep rows of pend ([keep][heads][dk + dv + 1]), with the
 *   replay arithmetic (row = row * decay; row = row + k_i * delta_j).
 * dk in {32, 64, 128, 256}; dv <= 1024; n <= 64; keep <= 64. */
/* The state's layout: per head, the value columns in groups of 16 (one wave of the
 * recurrence kernels: a quad of lanes per column, lane c holding keys [c dk/4, (c+1) dk/4)),
 * and within a group of W columns (W = 16, or fewer for the last group) the float4 slot k of
 * every lane (keys c dk/4 + 4k .. + 3 of column j at lane 4 (j mod 16) + c) contiguous: a
 * wave's state loads and stores are 16 B per lane over one contiguous 64 x 16 B run. */
size_t nmx_state_index(int h, int j, int i, int dk, int dv);

typedef struct {
    int n, heads, rep, dk, dv;
    int qkv_stride, o_stride;
    const float *qkv;
    const float *decay, *beta;
    float *S;
    float *o;
    float *log;
    const float *pend;
    int keep;
    int log0;
    const int32_t *keep_dev; /* non-NULL: keep = min(*keep_dev, keep) read on the device */
} nmx_lin_args;
int nmx_lin_rule(nmx_ctx *ctx, const nmx_lin_args *a);
/* S advances by the first `keep` rows of log (the commit replay). */
int nmx_lin_apply(nmx_ctx *ctx, float *S, const float *log, int keep, int heads, int dk, int dv);

/* ---- LM head fused with greedy argmax and draft acceptance -------------------------------
 * Replaces the verify tail of pf_spec_decode: pf_matmul(head, k+1 rows) (engine/src/forward.c:
 * 142-143), pinfer_argmax per row (forward_ops.c:387-409) and the acceptance loop
 * (engine/src/spec.c:340-345). W is the Q4K head [rows][cols]; A8 inputs for n = k + 1 rows.
 * logits (may be NULL) receives [n][rows] fp32. drafts [k] int32 on the device: the draft for
 * row t + 1. out [2 + n] int32 on the device: out[0] = a (accepted drafts), out[1] = bonus =
 * argmax(row a), out[2 + t] = argmax(row t) (first index of the maximum). work: device scratch
 * of nmx_head_work_bytes(rows, n) bytes. k = 0 is a plain greedy step (out[1] = argmax). */
size_t nmx_head_work_bytes(int rows, int n);
int nmx_head_accept(nmx_ctx *ctx, const void *W, int rows, int cols, int n, const int8_t *q,
                    const float *d, const float *fsum, float *logits, const int32_t *drafts,
                    void *work, int32_t *out);
/* The same, also writing out[1] (the bonus / greedy token) to tok_dst (device int32, may be
 * NULL): the MTP draft lands in the verify token row without a copy. */
int nmx_head_accept_to(nmx_ctx *ctx, const void *W, int rows, int cols, int n, const int8_t *q,
                       const float *d, const float *fsum, float *logits, const int32_t *drafts,
                       void *work, int32_t *out, int32_t *tok_dst);

/* nmx_head_accept followed by the commit of the accepted run in the same last kernel: what
 * nmx_accept_commit_mb (mailbox != NULL, nvt >= n + 1) or nmx_accept_commit (mailbox NULL)
 * does after it (engine/src/spec.c:340-351: the acceptance loop, then vt[a + 1] = bonus and
 * e = a + 1), without the extra launch. No logits. */
int nmx_head_accept_commit(nmx_ctx *ctx, const void *W, int rows, int cols, int n,
                           const int8_t *q, const float *d, const float *fsum,
                           const int32_t *drafts, void *work, int32_t *out, int32_t *vt,
                           int32_t *ctl, int32_t *mailbox, int nvt);

/* The head of a plain greedy step (engine/src/spec.c:238-262) on the one A8 row q / d / fsum:
 * its argmax g to vt[0] (the next step's input token) and to vt[1], ctl[1] = 1, ctl[0] += 1
 * (n_past advanced by the step) and, when mailbox is not NULL, the host mailbox [0, g, vt[0..nvt)
 * as nmx_head_accept_commit writes it] and its flag, all in the head's last kernel: a captured
 * step needs no host read of the token and no position upload. out [3] as nmx_head_accept. */
int nmx_head_step(nmx_ctx *ctx, const void *W, int rows, int cols, const int8_t *q,
                  const float *d, const float *fsum, void *work, int32_t *out, int32_t *vt,
                  int32_t *ctl, int32_t *mailbox, int nvt);

/* The head of nmx_head_accept_commit without its reduction launch: the dots and the
 * per-workgroup partial argmax keys ([n][nmx_head_nkeys(rows, cols, n)] 64-bit keys in work,
 * nmx_head_work_bytes(rows, n) bytes), and the drafts d1..d(n-1) copied to drafts_copy (n - 1
 * int32, device). The argmax per row, the acceptance loop and the commit of the accepted run
 * (engine/src/spec.c:340-351) then run in the consumer's workgroups: nmx_lin_commit_keys. The
 * verify head of one round is thus one launch, and the reduction costs the commit no launch
 * of its own. n <= 16. No logits. */
int nmx_head_nkeys(int rows, int cols, int n);
int nmx_head_keys(nmx_ctx *ctx, const void *W, int rows, int cols, int n, const int8_t *q,
                  const float *d, const float *fsum, const int32_t *drafts, void *work,
                  int32_t *drafts_copy);

/* nmx_head_accept without the workspace argument: allocates nothing and takes no workspace.
 * No counterpart in the reference: it is for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). The
 * partial argmax keys live in a static device array of NMX_HEAD_SCRATCH_BYTES per GPU (held
 * until the process ends), so nmx_head_work_bytes(rows, n) must not exceed it (rows <= 2^20
 * at n <= 16; larger shapes fail with an error). The caller passes inputs and outputs as for
 * nmx_head_accept and gets the same results. Calls on one GPU share the array: calls that
 * overlap in time on one GPU (two streams, two contexts) race; calls on one stream do not. */
#define NMX_HEAD_SCRATCH_BYTES (512 * 1024)
int nmx_head_accept_noalloc(nmx_ctx *ctx, const void *W, int rows, int cols, int n,
                            const int8_t *q, const float *d, const float *fsum, float *logits,
                            const int32_t *drafts, int32_t *out);

/* ---- verify-step glue (the rest of one forward pass, engine/src/forward*.c) -------------
 * All enqueue on the context's stream; positions come from a device control block so a
 * captured HIP graph can be replayed at any position: ctl[0] = n_past at the start of the
 * pass, ctl[1] = e (tokens committed by the last verify pass), ctl[2] = keep (pending
 * replay rows, e - 1 after a commit). */
typedef struct {
    int8_t *q;   /* NULL: no A8 output */
    float *d, *fs;
} nmx_a8;

/* Embedding rows of a Q4K matrix (pf_get_row / kern_get_row_q, engine/src/kern_act.c:53-88):
 * X[t][c] = (D s) u - (M m) for the token ids tok[0..n) (device). */
int nmx_embed_q4k(nmx_ctx *ctx, const void *W, int vocab, int cols, const int32_t *tok, int n,
                  float *X, int x_stride);

/* y = rmsnorm(x) * w per row (pf_rmsnorm, engine/src/forward_ops.c:191-200), after
 * x += add when add != NULL (pf_add_rows, engine/src/forward.c:68-73); y may be NULL; a8.q
 * != NULL also writes the A8 quantization of y (n vectors, block-major). */
int nmx_rmsnorm(nmx_ctx *ctx, float *x, int x_stride, const float *add, int add_stride,
                const float *w, int n, int cols, float eps, float *y, int y_stride, nmx_a8 a8);

/* nmx_rmsnorm with the residual sum x + add written to xo instead of in place (xo NULL: not
 * written; xo may equal x). */
int nmx_rmsnorm_xo(nmx_ctx *ctx, const float *x, int x_stride, const float *add, int add_stride,
                   float *xo, int xo_stride, const float *w, int n, int cols, float eps, float *y,
                   int y_stride, nmx_a8 a8);
/* Two independent nmx_rmsnorm calls of n rows each (no residual), in one launch when
 * cols <= 1024 and the rows are 16-byte aligned (else two launches): the MTP head's fc input
 * [norm_e(embed(tok)) | norm_h(h)] (engine/src/mtp.c:60-75). Returns 0 or -1. */
/* nmx_rmsnorm of the single row *idx + off of x (+ add), the index read on the device and
 * clamped to [0, nrows), into y [cols] and a one-vector A8 (either may be NULL; cols a multiple
 * of 32, at most 1024; 16-byte aligned rows): the MTP head's final norm of the row whose draft
 * is wanted (engine/src/mtp.c:88-100). */
int nmx_rmsnorm_row(nmx_ctx *ctx, const float *x, int x_stride, const float *add,
                    int add_stride, const float *w, int cols, float eps, const int32_t *idx,
                    int off, int nrows, float *y, nmx_a8 a8);
/* nmx_rmsnorm_row (row *idx + off of x (+ add), clamped to [0, nrows), normed with w into y,
 * which may be NULL) followed by nmx_head_accept_to over that one row without drafts: the MTP
 * draft head on its final norm (engine/src/mtp.c:88-100). The norm runs inside the head's
 * workgroups (one launch fewer; y, out and tok_dst equal those of the two calls bit for bit)
 * when cols is a multiple of 256 up to 1024 and x, add, w, y are 16-byte aligned rows; else
 * the two calls, with a8_tmp (one cols-column A8 row) for the norm's output. advance (a
 * control block, may be NULL): nmx_ctl_advance(advance) after the head, done by its last
 * kernel (a round ending with the MTP pass over the committed rows). */
int nmx_head_row_accept_to(nmx_ctx *ctx, const void *W, int rows, int cols, const float *x,
                           int x_stride, const float *add, int add_stride, const float *w,
                           float eps, const int32_t *idx, int off, int nrows, float *y,
                           void *work, int32_t *out, int32_t *tok_dst, nmx_a8 a8_tmp,
                           int32_t *advance);

/* The first kernel of nmx_head_row_accept_to alone, for its fused shapes (cols a multiple of
 * 256 up to 1024, 16-byte aligned rows): the normed row to y (may be NULL) and the argmax over
 * the rows of W left as nmx_head_row_nkeys(rows) partial keys in keys (8-byte aligned), for a
 * consumer that resolves the token itself (nmx_q4k_matmul_embed_norm, nmx_embed_norm_keys):
 * one launch fewer than a head with its own reduction. No reference counterpart of its own:
 * the reference's draft head (engine/src/mtp.c:88-100) split at the argmax. */
int nmx_head_row_keys(nmx_ctx *ctx, const void *W, int rows, int cols, const float *x,
                      int x_stride, const float *add, int add_stride, const float *w, float eps,
                      const int32_t *idx, int off, int nrows, float *y, void *keys);
int nmx_head_row_nkeys(int rows);

int nmx_rmsnorm_pair(nmx_ctx *ctx, int n, int cols, float eps, const float *x0, int x0_stride,
                     const float *w0, float *y0, int y0_stride, nmx_a8 a0, const float *x1,
                     int x1_stride, const float *w1, float *y1, int y1_stride, nmx_a8 a1);
/* The embedding rows tok[0..n) of the Q4K matrix E (nmx_embed_q4k), written to xo0 when not
 * NULL, RMS-normalised with w0 into y0 / a0 as nmx_rmsnorm, and, when x1 is not NULL, a second
 * norm as in nmx_rmsnorm_pair, in one launch when cols <= 1024 and the rows are 16-byte
 * aligned: the first layer's input norm (engine/src/forward.c:92-100) and the MTP head's fc
 * input (engine/src/mtp.c:60-75). Returns 0 or -1. */
int nmx_embed_norm(nmx_ctx *ctx, const void *E, int vocab, const int32_t *tok, int n, int cols,
                   float eps, const float *w0, float *xo0, int xo0_stride, float *y0, int y0_stride,
                   nmx_a8 a0, const float *x1, int x1_stride, const float *w1, float *y1,
                   int y1_stride, nmx_a8 a1);

/* nmx_embed_norm with one set (no second norm, no y0) whose row n - 1 takes its token from the
 * nkeys partial argmax keys of nmx_head_row_keys (written to tok[n - 1]) instead of reading it:
 * the verify pass's first norm on a draft that no separate reduction resolved. cols a multiple
 * of 256 up to 1024, 16-byte aligned rows. */
int nmx_embed_norm_keys(nmx_ctx *ctx, const void *E, int vocab, int32_t *tok, int n, int cols,
                        float eps, const float *w, float *xo, int xo_stride, nmx_a8 a8,
                        const void *keys, int nkeys);

/* Gated DeltaNet pre (engine/src/forward_lin.c:36-67): causal conv + SiLU per channel with the
 * conv state, q/k L2 norm (+ q scale), beta = sigmoid(b), decay = exp(A softplus(a + dt_bias)).
 * xin != NULL marks a logged pass: the state advances by token 0 only and the raw inputs of
 * tokens 1..n-1 are kept in xin [n][C] for the commit. */
typedef struct {
    int n, C, conv_k, dk, kd;
    const float *raw;
    int raw_stride;
    float *out;
    float *state;
    const float *conv_w;
    float *xin;
    float qscale, l2eps;
    const float *b_in, *a_in;
    int g_stride, heads;
    const float *A_log, *A, *dt_bias;
    float *beta, *decay;
} nmx_lin_pre_args;
int nmx_lin_pre(nmx_ctx *ctx, const nmx_lin_pre_args *p);

/* Gated RMSNorm (engine/src/forward_lin.c:70-81): per (token, head) y = rmsnorm(o) * w *
 * silu(z); y may be NULL; optional A8 of y. */
int nmx_lin_post(nmx_ctx *ctx, const float *o, int o_stride, const float *z, int z_stride,
                 const float *w, int n, int heads, int dv, float eps, float *y, int y_stride,
                 nmx_a8 a8);

/* The Gated DeltaNet mixer between in_proj and out_proj in one launch (engine/src/
 * forward_lin.c:36-81, 94-133): nmx_lin_pre for the q / k / v channels and gates of each value
 * head, nmx_lin_rule and nmx_lin_post (gated RMSNorm of o with z and norm_w, output y and / or
 * its A8), with identical results; the conv outputs, gates and o stay on chip. pre.out,
 * pre.beta, pre.decay, rule.qkv, rule.decay, rule.beta and rule.o are only used (and then
 * must be valid buffers) when the shape is outside the fused kernel's limits and the three
 * kernels run instead. */
typedef struct {
    nmx_lin_pre_args pre;
    nmx_lin_args rule;
    const float *z;
    int z_stride;
    const float *norm_w;
    float eps;
    float *y;
    int y_stride;
    nmx_a8 a8;
} nmx_lin_mix_args;
int nmx_lin_mix(nmx_ctx *ctx, const nmx_lin_mix_args *a);

/* RMSNorm input of a fused matmul: rows x (+ add, the residual, added first) of [n][cols],
 * normed with weight w (engine/src/forward_ops.c:191-200, forward.c pf_add_rows). x_out (if
 * not NULL) receives x + add, written once; it must not alias x or add. */
typedef struct {
    const float *x;
    int x_stride;
    const float *add;
    int add_stride;
    float *x_out;
    int xo_stride;
    const float *w;
    float eps;
} nmx_norm_in;

/* The launch geometry of the small-row matmul kernel behind nmx_q4k_matmul_norm,
 * nmx_q4k_swiglu, nmx_q4k_matmul_embed_norm (pair = 1: the MTP fc input, cols = 2 H) and the
 * plain projections of fewer than 32768 rows, for count matrices of rows[s] rows, cols columns
 * and n activation rows. Host only (no device, no context): returns 1 and fills g when that
 * kernel takes the shape, 0 when the shape goes to the other kernels, -1 when the geometry it
 * picks would leave one of the kernel's phases (weight units, chains, norm columns, norm
 * chains, PAIR decoders, SwiGLU epilogue, LDS) without the threads it assumes, which the
 * launch refuses with an error. No counterpart in the reference: its kernels are scalar. */
typedef struct {
    int rows_per_wg;       /* R: output rows of one workgroup */
    int threads;           /* T: threads per workgroup (every pass) */
    int blocks_per_unit;   /* 32-column blocks per weight unit (1, 2 or 4) */
    int workgroups;
    int passes;            /* passes of at most 8 vectors */
    int nv[8];             /* vectors of each pass */
    int lds_bytes[8];      /* dynamic LDS of each pass */
} nmx_mt_geometry;
int nmx_mt_plan(int count, const int *rows, int cols, int n, int norm, int swiglu, int pair,
                nmx_mt_geometry *g);

/* nmx_q4k_matmul_multi on the A8 of rmsnorm(in): the norm and the quantization run inside the
 * matmul's workgroups (equal to nmx_rmsnorm + the matmul bit for bit). a8_tmp (n x cols A8
 * buffers) is used only when the shape is outside the fused kernel's limits. */
int nmx_q4k_matmul_norm(nmx_ctx *ctx, int count, const void *const *W, const int *rows,
                        float *const *Y, const int *y_stride, int cols, int n,
                        const nmx_norm_in *in, nmx_a8 a8_tmp);

/* The MTP head's fc projection on its input pair (engine/src/mtp.c:60-75): Y[n][rows] = W a
 * (W rows x 2 H) with a the A8 of [rmsnorm(embedding rows tok[0..n) of the Q4K matrix E, w_emb)
 * | rmsnorm(h, w_hid)], equal bit for bit to nmx_embed_norm (both halves' A8 into one 2 H-column
 * buffer) followed by nmx_q4k_matmul. The embedding and both norms run inside the matmul's
 * workgroups (one launch) when n <= 8, H is a multiple of 256, h, w_emb and w_hid are 16-byte
 * aligned and the shape fits; otherwise a8_tmp (n x 2 H A8, the two calls; H <= 1024) is
 * used. tok_keys (may be NULL; one row, the fused shape): the token is the argmax of the nkeys
 * partial keys of nmx_head_row_keys, written to tok[0] (the draft lands in the token row). */
int nmx_q4k_matmul_embed_norm(nmx_ctx *ctx, const void *W, int rows, float *Y, int y_stride,
                              int n, int H, const void *E, int vocab, int32_t *tok,
                              const float *w_emb, const float *h, int h_stride,
                              const float *w_hid, float eps, nmx_a8 a8_tmp,
                              const void *tok_keys, int nkeys);

/* The SwiGLU MLP input (engine/src/forward.c:49-58, forward_ops.c:98-110): h = silu(Wg a) *
 * (Wu a) for a = the A8 input (q, d, fsum) or, when in is not NULL, the A8 of rmsnorm(in);
 * h is written as A8 to out (and as floats [n][ffn] to y if not NULL). Fused into one launch
 * when the shape fits; otherwise a8_tmp (n x cols) and gate_tmp / up_tmp ([n][ffn] floats)
 * hold the intermediate results. */
int nmx_q4k_swiglu(nmx_ctx *ctx, const void *Wg, const void *Wu, int ffn, int cols, int n,
                   const int8_t *q, const float *d, const float *fsum, const nmx_norm_in *in,
                   float *y, nmx_a8 out, nmx_a8 a8_tmp, float *gate_tmp, float *up_tmp);

/* SwiGLU (pf_silu_mul, engine/src/forward_ops.c:98-110): y = silu(gate) * up (+ A8). */
int nmx_silu_mul(nmx_ctx *ctx, const float *gate, const float *up, int stride, int n, int cols,
                 float *y, nmx_a8 a8);

/* Gated full attention (engine/src/forward_attn.c:231-266). prep: k rows normed + RoPE and
 * stored with the v rows at position *pos + pos_off + t; query heads normed + RoPE in place.
 * attn: causal GQA softmax attention over rows [0, position], o *= sigmoid(gate), + A8; two
 * launches (scores into the caller's workspace, then softmax + P.V).
 * KV caches (engine/src/forward_kv.c:1-14, pinfer.h PINFER_KV_*): kv_dtype 0 = fp32 rows
 * [nkv][max_ctx][hd]; 1 = IEEE binary16 rows (round to nearest even); 2 = int8 rows
 * q = rint(x * 127 / amax) followed by [nkv][max_ctx] fp32 scales amax / 127. Rows are stored
 * rounded and read widened (binary16 exactly, int8 as q * scale); nmx_kv_bytes gives the size
 * of one cache. */
size_t nmx_kv_bytes(int kv_dtype, int nkv, int max_ctx, int hd);
typedef struct {
    int n, nh, nkv, hd, rot, max_ctx;
    float *q;                    /* [n][nh][2 hd] query | gate */
    const float *k_in, *v_in;    /* [n][nkv hd] */
    const float *q_norm, *k_norm;
    float eps, scale;
    const float *rope_cos, *rope_sin; /* [max_ctx][rot/2] */
    void *kc, *vc;               /* caches of kv_dtype, nmx_kv_bytes each */
    const int32_t *pos;
    int pos_off;
    float *o;                    /* [n][nh hd] */
    nmx_a8 a8;
    float *scores;               /* attn workspace: [n][nh][max_ctx] floats */
    int kv_dtype;                /* 0 fp32, 1 binary16, 2 int8 + row scales */
} nmx_attn_args;
int nmx_attn_prep(nmx_ctx *ctx, const nmx_attn_args *p);
int nmx_attn(nmx_ctx *ctx, const nmx_attn_args *p);
/* nmx_attn_prep followed by nmx_attn in two launches instead of three: the scores kernel
 * normalises and rotates its own queries and the pass's new keys (rounded to the cache format
 * and back) and stores the new K / V rows itself (the steps of forward_attn.c:231-266 and
 * forward_kv.c:83-127). o, its A8, the scores and both caches equal those of the two calls
 * bit for bit; q keeps the unrotated queries. hd = 256, at most 4 query heads per KV group
 * and at most 8 tokens, else the two calls. */
int nmx_attn_fused(nmx_ctx *ctx, const nmx_attn_args *p);

/* The reference's chain gate (engine/src/spec_adapt.c:56, spec.c:89-97) as a device op, for a
 * caller that drives the reference's own confidence-gated adaptive chain on this device layer;
 * the engine's own adaptive policy (pinfer_spec_params.adaptive) decides on the host and does
 * not call it.
 * flag[0] = (top-1 probability of logits[0, n) >= tau): with mx = max (pf_softmax_max) and
 * s = sum of pf_expf(l_i - mx) in the reference's order (4 interleaved partial sums, tail,
 * pf_softmax_exp engine/src/forward_ops.c:294-353), p = s > 0 ? 1 / s : 0 (spec.c:93-97
 * top1_prob). One workgroup; the decision is exact (an fp64 sum decides unless p is within the
 * fp32 sum's error bound of tau, where the ordered fp32 sum itself is formed). */
int nmx_top1_gate(nmx_ctx *ctx, const float *logits, int n, float tau, int32_t *flag);

/* The DeltaNet gates' exp (which = 0) and log1p (1) as the mixer kernels evaluate them, for
 * the n binary32 inputs with bit patterns first .. first + n - 1 into y (device): a probe for
 * parity tests of the device against the host C library the reference calls
 * (engine/src/forward_lin.c:18-19,59-66). No reference counterpart of its own. */
int nmx_gate_eval(nmx_ctx *ctx, int which, uint32_t first, long n, float *y);

/* Rollback commit of every linear layer (pf_lin_commit, engine/src/forward_lin.c:185-204)
 * with e = ctl[1]: conv state <- last conv_k - 1 rows of [state after token 0, raw inputs
 * 1..e-1]; pend <- log rows 1..e-1; ctl[2] = e - 1. Arrays are [layers][...] contiguous.
 * state_bak (optional, the size of state) keeps the rows of the state after token 0; a later
 * call with redo = 1 commits a smaller e from them (the host's stop inside a run that the
 * device already committed). A commit of e = 1 returns before it touches state_bak (the state
 * after token 0 is then already the committed one), so a redo is valid only after a commit
 * of e >= 2 and for a smaller e, which is the only case in which the engine issues one. */
typedef struct {
    int layers, C, conv_k;
    float *state;          /* [layers][conv_k-1][C] */
    const float *xin;      /* [layers][cap][C] */
    const float *log;      /* [layers][cap][row] */
    float *pend;           /* [layers][cap][row] */
    int cap, row;
    int32_t *ctl;
    int32_t *vt;           /* optional: also vt[0] = vt[ctl[1]], as nmx_copy_token */
    float *state_bak;      /* optional: [layers][conv_k-1][C] */
    int redo;              /* commit from state_bak instead of state */
} nmx_commit_args;
int nmx_lin_commit(nmx_ctx *ctx, const nmx_commit_args *p);

/* nmx_lin_commit with e from the verify head's partial keys instead of ctl[1]: every
 * workgroup resolves the argmax of each of the n rows (n <= 16) from the nkeys keys per row
 * that nmx_head_keys left and runs the acceptance loop over the drafts copy; the first
 * workgroup then writes what nmx_head_accept_commit writes (out [2 + n], vt[a + 1] = bonus,
 * ctl[1] = e = a + 1, the mailbox of nvt <= 64 tokens when not NULL) and cur (vt[0] = bonus),
 * and the commit of e follows as in nmx_lin_commit. p->vt is required, p->redo must be 0.
 * Results equal nmx_head_accept_commit + nmx_lin_commit (engine/src/spec.c:340-351,
 * engine/src/forward_lin.c:185-204). */
typedef struct {
    const void *keys;       /* [n][nkeys] partial keys of nmx_head_keys */
    int nkeys, n;
    const int32_t *drafts;  /* nmx_head_keys' drafts_copy */
    int32_t *out;           /* [2 + n] */
    int32_t *mailbox;       /* optional, host memory */
    int nvt;
} nmx_accept_keys;
int nmx_lin_commit_keys(nmx_ctx *ctx, const nmx_commit_args *p, const nmx_accept_keys *k);

/* After nmx_head_accept: vt[a + 1] = bonus; ctl[1] = a + 1 (the reference's e without a stop,
 * engine/src/spec.c:346-349). */
int nmx_accept_commit(nmx_ctx *ctx, const int32_t *out, int32_t *vt, int32_t *ctl);
/* The same, also writing [a, bonus, vt[0..nvt) after the update] to mailbox (memory from
 * nmx_host_alloc, 3 + nvt int32) and then mailbox[2 + nvt] = 1 with a system-scope release:
 * a host that clears that word before the launch and polls it (acquire) reads the round's
 * result without a stream synchronisation (the reference's host loop reads them in place,
 * engine/src/spec.c:340-351). */
int nmx_accept_commit_mb(nmx_ctx *ctx, const int32_t *out, int32_t *vt, int32_t *ctl,
                         int32_t *mailbox, int nvt);
int nmx_ctl_set(nmx_ctx *ctx, int32_t *ctl, int idx, int value);
int nmx_ctl_advance(nmx_ctx *ctx, int32_t *ctl);   /* ctl[0] += ctl[1] */
int nmx_copy_token(nmx_ctx *ctx, int32_t *vt, const int32_t *ctl); /* vt[0] = vt[ctl[1]] */
/* dst[0..cols) = src[(*idx + off) * stride ..] (a device-chosen row) */
int nmx_select_row(nmx_ctx *ctx, const float *src, int stride, const int32_t *idx, int off,
                   int cols, float *dst);

#ifdef __cplusplus
}
#endif
#endif
