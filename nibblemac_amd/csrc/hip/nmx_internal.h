/* Internal definitions shared by the nmx HIP translation units (not part of the ABI). */
#ifndef NMX_INTERNAL_H
#define NMX_INTERNAL_H

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>

#include "nmx.h"

struct nmx_ctx {
    int device;
    hipStream_t stream;
    char name[256];
    char err[1024];
    int capturing;
};

struct nmx_event {
    hipEvent_t ev;
};

struct nmx_graph {
    hipGraph_t graph;
    hipGraphExec_t exec;
};

/* Record an error message on ctx; always returns -1. */
int nmx_fail(nmx_ctx *ctx, const char *fmt, ...) __attribute__((format(printf, 2, 3)));

/* Map a HIP status to -1 + message. */
#define NMX_HIP(ctx, call)                                                                  \
    do {                                                                                    \
        hipError_t e_ = (call);                                                             \
        if (e_ != hipSuccess)                                                               \
            return nmx_fail((ctx), "%s: %s (%s:%d)", #call, hipGetErrorString(e_), __FILE__, \
                            __LINE__);                                                      \
    } while (0)

/* Launch-error check after a kernel launch (hipGetLastError). */
#define NMX_LAUNCHED(ctx, what)                                                             \
    do {                                                                                    \
        hipError_t e_ = hipGetLastError();                                                  \
        if (e_ != hipSuccess) return nmx_fail((ctx), "%s launch: %s", what, hipGetErrorString(e_)); \
    } while (0)

/* One matrix of a small-row Q4K matmul launch. */
struct nmx_mt_seg {
    const uint8_t *W;
    float *Y;
    int rows;
    int ystride;
};

/* The MTP head's fc input as a norm prologue: the embedding rows tok[] of the Q4K matrix E
 * normed with w_emb, then the rows of h (row stride h_stride, 16-byte aligned) normed with
 * norm->w; eps is norm->eps. */
struct nmx_mt_pair {
    const uint8_t *E;
    int32_t *tok;
    const float *w_emb;
    const float *h;
    int h_stride;
    const unsigned long long *keys; /* optional (one row): the token from nkeys argmax keys */
    int nkeys;
};

/* Small-row Q4K matmul with every vector of a pass in one workgroup (nmx_mt.hip), optionally
 * with the RMSNorm + A8 prologue (norm; with pair, the MTP input pair of norms) and the
 * SwiGLU + A8 epilogue (swiglu: segments gate, up). Returns 0, -1 on a launch error, or 1
 * when the shape is outside its limits. */
int nmx_mt_matmul(nmx_ctx *ctx, int count, const nmx_mt_seg *segs, int cols, int n,
                  const int8_t *q, const float *d, const float *fs, const nmx_norm_in *norm,
                  bool swiglu, nmx_a8 out, const nmx_mt_pair *pair = nullptr);


/* Resolve the device address of nmx_head_accept_noalloc's static scratch array for
 * ctx->device (current on the calling thread), once per device; nmx_create calls it. */
int nmx_head_scratch_init(nmx_ctx *ctx);

/* [a, a + na) and [b, b + nb) overlap (byte ranges). */
/* The DeltaNet state layout (nmx_state_index): per head, the value columns in groups of 16 (a
 * wave of the recurrence kernels: lane 4 (j mod 16) + c holds keys [c dk/4, (c+1) dk/4) of
 * column j), and within a group of W columns the float4 slot k of every lane contiguous. A
 * lane's keys 4k .. 4k + 3 of its quarter are at state_lane(..) + k state_slot(..). */
__host__ __device__ inline size_t state_lane(int h, int j, int c, int dk, int dv) {
    return ((size_t)h * dv + (j & ~15)) * dk + (size_t)(4 * (j & 15) + c) * 4;
}
__host__ __device__ inline int state_slot(int j, int dv) {
    const int w = dv - (j & ~15);
    return 16 * (w < 16 ? w : 16);
}
__host__ __device__ inline size_t state_index(int h, int j, int i, int dk, int dv) {
    const int dk4 = dk / 4;
    return state_lane(h, j, i / dk4, dk, dv) + (size_t)((i % dk4) / 4) * state_slot(j, dv) + i % 4;
}

static inline bool nmx_overlap(const void *a, size_t na, const void *b, size_t nb) {
    const char *pa = (const char *)a, *pb = (const char *)b;
    return na && nb && pa < pb + nb && pb < pa + na;
}

#endif
