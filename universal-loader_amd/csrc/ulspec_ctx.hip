// ulspec_ctx.hip -- context, memory and error entry points of the C ABI.
#include "ulspec_internal.h"

#include <cstring>

using namespace ulspec;

extern "C" const char* ulspec_version(void)
{
    return "ulspec 0.1 gfx950";
}

extern "C" int ulspec_ggml_blck_size(uint32_t t)
{
    return t == ULSPEC_GGML_Q4_0 ? 32 : t == ULSPEC_GGML_Q4_K ? 256 : 0;
}

extern "C" int ulspec_ggml_type_size(uint32_t t)
{
    return t == ULSPEC_GGML_Q4_0 ? 18 : t == ULSPEC_GGML_Q4_K ? 144 : 0;
}

extern "C" const char* ulspec_status_str(ulspec_status s)
{
    switch (s) {
    case ULSPEC_OK: return "ok";
    case ULSPEC_EINVAL: return "invalid argument";
    case ULSPEC_ENOMEM: return "out of memory";
    case ULSPEC_EDEVICE: return "device error";
    case ULSPEC_EUNSUPPORTED: return "unsupported";
    }
    return "unknown status";
}

extern "C" ulspec_status ulspec_create(int hip_device, ulspec_ctx** out)
{
    if (!out) return ULSPEC_EINVAL;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return ULSPEC_EDEVICE;
    if (hip_device < 0 || hip_device >= n) return ULSPEC_EINVAL;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, hip_device) != hipSuccess) return ULSPEC_EDEVICE;
    // The kernels are built for gfx950 (CDNA4) only.
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) return ULSPEC_EDEVICE;
    if (hipSetDevice(hip_device) != hipSuccess) return ULSPEC_EDEVICE;
    ulspec_ctx* ctx = new ulspec_ctx();
    ctx->device = hip_device;
    ctx->n_cu = prop.multiProcessorCount;
    if (hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess) {
        delete ctx;
        return ULSPEC_EDEVICE;
    }
    if (gemm_init(ctx) != ULSPEC_OK) {
        (void)hipStreamDestroy(ctx->stream);
        delete ctx;
        return ULSPEC_EDEVICE;
    }
    *out = ctx;
    return ULSPEC_OK;
}

extern "C" void ulspec_destroy(ulspec_ctx* ctx)
{
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    for (auto& w : ctx->weights)
        if (w.dev) (void)hipFree(w.dev);
    for (auto& g : ctx->graphs)
        if (g) (void)hipGraphExecDestroy(g);
    for (auto& ev : ctx->events)
        if (ev) (void)hipEventDestroy(ev);
    if (ctx->ws) (void)hipFree(ctx->ws);
    if (ctx->staging) (void)hipHostFree(ctx->staging);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
}

extern "C" const char* ulspec_last_error(const ulspec_ctx* ctx)
{
    return ctx ? ctx->err.c_str() : "null context";
}

extern "C" ulspec_status ulspec_alloc(ulspec_ctx* ctx, size_t bytes, void** dev_ptr)
{
    ULSPEC_CHECK_CTX(ctx);
    if (!dev_ptr || bytes == 0) return fail(ctx, ULSPEC_EINVAL, "ulspec_alloc: null pointer or zero size");
    (void)hipSetDevice(ctx->device);
    hipError_t e = hipMalloc(dev_ptr, bytes);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipMalloc");
    return ULSPEC_OK;
}

extern "C" ulspec_status ulspec_free(ulspec_ctx* ctx, void* dev_ptr)
{
    ULSPEC_CHECK_CTX(ctx);
    if (!dev_ptr) return ULSPEC_OK;
    (void)hipSetDevice(ctx->device);
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e == hipSuccess) e = hipFree(dev_ptr);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipFree");
    return ULSPEC_OK;
}

extern "C" ulspec_status ulspec_memcpy(ulspec_ctx* ctx, void* dst, const void* src, size_t bytes, int kind)
{
    ULSPEC_CHECK_CTX(ctx);
    if (bytes == 0) return ULSPEC_OK;
    if (!dst || !src || kind < 0 || kind > 2) return fail(ctx, ULSPEC_EINVAL, "ulspec_memcpy: bad arguments");
    hipMemcpyKind k = kind == 0 ? hipMemcpyHostToDevice : kind == 1 ? hipMemcpyDeviceToHost : hipMemcpyDeviceToDevice;
    (void)hipSetDevice(ctx->device);
    hipError_t e = hipMemcpyAsync(dst, src, bytes, k, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipMemcpyAsync");
    return ULSPEC_OK;
}

extern "C" ulspec_status ulspec_sync(ulspec_ctx* ctx)
{
    ULSPEC_CHECK_CTX(ctx);
    (void)hipSetDevice(ctx->device);
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipStreamSynchronize");
    return ULSPEC_OK;
}

extern "C" ulspec_status ulspec_capture_begin(ulspec_ctx* ctx)
{
    ULSPEC_CHECK_CTX(ctx);
    if (ctx->capturing) return fail(ctx, ULSPEC_EINVAL, "capture_begin: already capturing");
    (void)hipSetDevice(ctx->device);
    hipError_t e = hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipStreamBeginCapture");
    ctx->capturing = true;
    return ULSPEC_OK;
}

extern "C" ulspec_status ulspec_capture_end(ulspec_ctx* ctx, uint32_t* graph_id)
{
    ULSPEC_CHECK_CTX(ctx);
    if (!ctx->capturing) return fail(ctx, ULSPEC_EINVAL, "capture_end: not capturing");
    if (!graph_id) return fail(ctx, ULSPEC_EINVAL, "capture_end: null graph_id");
    ctx->capturing = false;
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(ctx->stream, &g);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipStreamEndCapture");
    hipGraphExec_t ex = nullptr;
    e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipGraphInstantiate");
    *graph_id = (uint32_t)ctx->graphs.size();
    ctx->graphs.push_back(ex);
    return ULSPEC_OK;
}

extern "C" ulspec_status ulspec_graph_replay(ulspec_ctx* ctx, uint32_t graph_id, uint32_t times)
{
    ULSPEC_CHECK_CTX(ctx);
    if (graph_id >= ctx->graphs.size() || !ctx->graphs[graph_id])
        return fail(ctx, ULSPEC_EINVAL, "graph_replay: no graph %u", graph_id);
    (void)hipSetDevice(ctx->device);
    for (uint32_t i = 0; i < times; ++i) {
        hipError_t e = hipGraphLaunch(ctx->graphs[graph_id], ctx->stream);
        if (e != hipSuccess) return hip_fail(ctx, e, "hipGraphLaunch");
    }
    return ULSPEC_OK;
}

extern "C" ulspec_status ulspec_graph_destroy(ulspec_ctx* ctx, uint32_t graph_id)
{
    ULSPEC_CHECK_CTX(ctx);
    if (graph_id >= ctx->graphs.size() || !ctx->graphs[graph_id])
        return fail(ctx, ULSPEC_EINVAL, "graph_destroy: no graph %u", graph_id);
    (void)hipStreamSynchronize(ctx->stream);
    (void)hipGraphExecDestroy(ctx->graphs[graph_id]);
    ctx->graphs[graph_id] = nullptr;
    return ULSPEC_OK;
}

extern "C" ulspec_status ulspec_timer_mark(ulspec_ctx* ctx, uint32_t slot)
{
    ULSPEC_CHECK_CTX(ctx);
    if (slot >= 16) return fail(ctx, ULSPEC_EINVAL, "timer_mark: slot %u >= 16", slot);
    (void)hipSetDevice(ctx->device);
    if (!ctx->events[slot]) {
        hipError_t e = hipEventCreate(&ctx->events[slot]);
        if (e != hipSuccess) return hip_fail(ctx, e, "hipEventCreate");
    }
    hipError_t e = hipEventRecord(ctx->events[slot], ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipEventRecord");
    return ULSPEC_OK;
}

extern "C" ulspec_status ulspec_timer_elapsed_ms(ulspec_ctx* ctx, uint32_t a, uint32_t b, float* ms)
{
    ULSPEC_CHECK_CTX(ctx);
    if (a >= 16 || b >= 16 || !ms || !ctx->events[a] || !ctx->events[b])
        return fail(ctx, ULSPEC_EINVAL, "timer_elapsed_ms: bad slots or unmarked");
    hipError_t e = hipEventSynchronize(ctx->events[b]);
    if (e == hipSuccess) e = hipEventElapsedTime(ms, ctx->events[a], ctx->events[b]);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipEventElapsedTime");
    return ULSPEC_OK;
}

namespace ulspec {

ulspec_status workspace(ulspec_ctx* ctx, size_t bytes, void** out)
{
    if (bytes <= ctx->ws_bytes) {
        *out = ctx->ws;
        return ULSPEC_OK;
    }
    if (ctx->ws) {
        hipError_t e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) return hip_fail(ctx, e, "workspace sync");
        (void)hipFree(ctx->ws);
        ctx->ws = nullptr;
        ctx->ws_bytes = 0;
    }
    size_t want = bytes < (size_t(1) << 20) ? (size_t(1) << 20) : bytes;
    hipError_t e = hipMalloc(&ctx->ws, want);
    if (e != hipSuccess) return hip_fail(ctx, e, "workspace hipMalloc");
    ctx->ws_bytes = want;
    *out = ctx->ws;
    return ULSPEC_OK;
}

}  // namespace ulspec
