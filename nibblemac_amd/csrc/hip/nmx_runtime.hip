/* nmx runtime: context, device memory, events and stream capture (include/nmx.h).
 *
 * One context = one device + one non-blocking stream of default priority. Errors are kept per
 * context as a message; nothing falls back to the CPU. */
#include <cstdlib>
#include <cstring>

#include "nmx_internal.h"

static char g_create_error[512];

int nmx_fail(nmx_ctx *ctx, const char *fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (ctx) snprintf(ctx->err, sizeof ctx->err, "%s", buf);
    else snprintf(g_create_error, sizeof g_create_error, "%s", buf);
    return -1;
}

/* Byte fill used instead of hipMemsetAsync, so captured graphs never hold memset nodes. */
__global__ void nmx_fill_zero_k(uint32_t *p, size_t words, uint8_t *tail, size_t tail_bytes) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t w = i; w < words; w += stride) p[w] = 0u;
    if (i < tail_bytes) tail[i] = 0;
}

extern "C" {

const char *nmx_create_error(void) { return g_create_error; }

int nmx_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

nmx_ctx *nmx_create(int device) {
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count <= 0) {
        nmx_fail(nullptr, "no HIP device available (%s)", hipGetErrorString(e));
        return nullptr;
    }
    if (device < 0 || device >= count) {
        nmx_fail(nullptr, "device %d out of range (%d devices)", device, count);
        return nullptr;
    }
    nmx_ctx *ctx = (nmx_ctx *)calloc(1, sizeof(nmx_ctx));
    if (!ctx) {
        nmx_fail(nullptr, "out of host memory");
        return nullptr;
    }
    ctx->device = device;
    hipDeviceProp_t prop;
    if ((e = hipSetDevice(device)) != hipSuccess ||
        (e = hipGetDeviceProperties(&prop, device)) != hipSuccess ||
        (e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking)) != hipSuccess) {
        nmx_fail(nullptr, "device %d setup: %s", device, hipGetErrorString(e));
        free(ctx);
        return nullptr;
    }
    snprintf(ctx->name, sizeof ctx->name, "%s (%s, %d CUs)", prop.name, prop.gcnArchName,
             prop.multiProcessorCount);
    if (nmx_head_scratch_init(ctx)) {
        nmx_fail(nullptr, "device %d setup: %s", device, ctx->err);
        (void)hipStreamDestroy(ctx->stream);
        free(ctx);
        return nullptr;
    }
    return ctx;
}

void nmx_destroy(nmx_ctx *ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    (void)hipStreamDestroy(ctx->stream);
    free(ctx);
}

const char *nmx_error(const nmx_ctx *ctx) { return ctx ? ctx->err : g_create_error; }
const char *nmx_device_name(nmx_ctx *ctx) { return ctx ? ctx->name : ""; }

void *nmx_alloc(nmx_ctx *ctx, size_t bytes) {
    if (!ctx) return nullptr;
    if (bytes == 0) {
        nmx_fail(ctx, "nmx_alloc: zero bytes");
        return nullptr;
    }
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) {
        nmx_fail(ctx, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
        return nullptr;
    }
    return p;
}

void *nmx_host_alloc(nmx_ctx *ctx, size_t bytes) {
    if (!ctx) return nullptr;
    if (bytes == 0) {
        nmx_fail(ctx, "nmx_host_alloc: zero bytes");
        return nullptr;
    }
    void *p = nullptr;
    /* coherent (fine-grained) memory: a host thread may poll what a kernel writes with a
     * system-scope release while the stream still runs; coarse-grained memory guarantees the
     * visibility of device writes only after a synchronisation */
    hipError_t e = hipHostMalloc(&p, bytes, hipHostMallocCoherent);
    if (e != hipSuccess) {
        nmx_fail(ctx, "hipHostMalloc(%zu): %s", bytes, hipGetErrorString(e));
        return nullptr;
    }
    return p;
}

int nmx_host_free(nmx_ctx *ctx, void *ptr) {
    if (!ctx) return -1;
    if (!ptr) return 0;
    NMX_HIP(ctx, hipHostFree(ptr));
    return 0;
}

int nmx_free(nmx_ctx *ctx, void *ptr) {
    if (!ctx) return -1;
    if (!ptr) return 0;
    NMX_HIP(ctx, hipFree(ptr));
    return 0;
}

int nmx_upload(nmx_ctx *ctx, void *dst, const void *src, size_t bytes) {
    if (!ctx) return -1;
    if (!bytes) return 0;
    if (!dst || !src) return nmx_fail(ctx, "nmx_upload: NULL pointer");
    NMX_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    NMX_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return 0;
}

int nmx_download(nmx_ctx *ctx, void *dst, const void *src, size_t bytes) {
    if (!ctx) return -1;
    if (!bytes) return 0;
    if (!dst || !src) return nmx_fail(ctx, "nmx_download: NULL pointer");
    NMX_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    NMX_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return 0;
}

int nmx_copy_d2d(nmx_ctx *ctx, void *dst, const void *src, size_t bytes) {
    if (!ctx) return -1;
    if (!bytes) return 0;
    if (!dst || !src) return nmx_fail(ctx, "nmx_copy_d2d: NULL pointer");
    if (nmx_overlap(dst, bytes, src, bytes)) return nmx_fail(ctx, "nmx_copy_d2d: overlap");
    NMX_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream));
    return 0;
}

int nmx_fill_zero(nmx_ctx *ctx, void *dst, size_t bytes) {
    if (!ctx) return -1;
    if (!bytes) return 0;
    if (!dst) return nmx_fail(ctx, "nmx_fill_zero: NULL pointer");
    if ((uintptr_t)dst % 4) return nmx_fail(ctx, "nmx_fill_zero: pointer not 4-byte aligned");
    const size_t words = bytes / 4, tail = bytes % 4;
    size_t blocks = (words + 255) / 256;
    if (blocks < 1) blocks = 1;
    if (blocks > 4096) blocks = 4096;
    nmx_fill_zero_k<<<(unsigned)blocks, 256, 0, ctx->stream>>>((uint32_t *)dst, words,
                                                               (uint8_t *)dst + words * 4, tail);
    NMX_LAUNCHED(ctx, "fill_zero");
    return 0;
}

int nmx_sync(nmx_ctx *ctx) {
    if (!ctx) return -1;
    NMX_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return 0;
}

nmx_event *nmx_event_create(nmx_ctx *ctx) {
    if (!ctx) return nullptr;
    nmx_event *ev = (nmx_event *)calloc(1, sizeof(nmx_event));
    if (!ev) return nullptr;
    if (hipEventCreate(&ev->ev) != hipSuccess) {
        free(ev);
        nmx_fail(ctx, "hipEventCreate failed");
        return nullptr;
    }
    return ev;
}

void nmx_event_destroy(nmx_event *ev) {
    if (!ev) return;
    (void)hipEventDestroy(ev->ev);
    free(ev);
}

int nmx_event_record(nmx_ctx *ctx, nmx_event *ev) {
    if (!ctx || !ev) return -1;
    NMX_HIP(ctx, hipEventRecord(ev->ev, ctx->stream));
    return 0;
}

int nmx_event_elapsed_ms(nmx_ctx *ctx, nmx_event *start, nmx_event *stop, float *ms) {
    if (!ctx || !start || !stop || !ms) return -1;
    NMX_HIP(ctx, hipEventSynchronize(stop->ev));
    NMX_HIP(ctx, hipEventElapsedTime(ms, start->ev, stop->ev));
    return 0;
}

int nmx_graph_begin(nmx_ctx *ctx) {
    if (!ctx) return -1;
    if (ctx->capturing) return nmx_fail(ctx, "nmx_graph_begin: already capturing");
    NMX_HIP(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    ctx->capturing = 1;
    return 0;
}

nmx_graph *nmx_graph_end(nmx_ctx *ctx) {
    if (!ctx || !ctx->capturing) return nullptr;
    ctx->capturing = 0;
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(ctx->stream, &g);
    if (e != hipSuccess || !g) {
        nmx_fail(ctx, "hipStreamEndCapture: %s", hipGetErrorString(e));
        return nullptr;
    }
    nmx_graph *out = (nmx_graph *)calloc(1, sizeof(nmx_graph));
    if (!out) {
        (void)hipGraphDestroy(g);
        nmx_fail(ctx, "out of host memory");
        return nullptr;
    }
    out->graph = g;
    e = hipGraphInstantiate(&out->exec, g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(g);
        free(out);
        nmx_fail(ctx, "hipGraphInstantiate: %s", hipGetErrorString(e));
        return nullptr;
    }
    return out;
}

int nmx_graph_launch(nmx_ctx *ctx, nmx_graph *g) {
    if (!ctx || !g) return -1;
    NMX_HIP(ctx, hipGraphLaunch(g->exec, ctx->stream));
    return 0;
}

void nmx_graph_destroy(nmx_graph *g) {
    if (!g) return;
    (void)hipGraphExecDestroy(g->exec);
    (void)hipGraphDestroy(g->graph);
    free(g);
}

} /* extern "C" */
