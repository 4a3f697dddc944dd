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

#ifdef __cplusplus
}
#endif
#endif
