// ulspec_ctx.hip -- context, memory and error entry points of the C ABI.
#include "ulspec_internal.h"

#include <algorithm>
#include <cstring>

using namespace ulspec;

extern "C" const char* ulspec_version(void)
{
    return "ulspec 0.1 gfx950";
}

// Elements and bytes per block of every GGUF tensor type with a fixed block
// layout (the public ggml definitions; the reference's table,
// src/core/gguf_types.h:35-81, has wrong byte sizes for most of them).  0 for
// an unknown id.
namespace {
struct GgmlTypeInfo {
    uint16_t blck, bytes;
};
constexpr GgmlTypeInfo kGgmlTypes[] = {
    {1, 4},     // 0 F32
    {1, 2},     // 1 F16
    {32, 18},   // 2 Q4_0: fp16 d, 16 B of nibbles
    {32, 20},   // 3 Q4_1: fp16 d, m, 16 B
    {0, 0},     // 4 (removed Q4_2)
    {0, 0},     // 5 (removed Q4_3)
    {32, 22},   // 6 Q5_0: d, 4 B high bits, 16 B
    {32, 24},   // 7 Q5_1
    {32, 34},   // 8 Q8_0: d, 32 x int8
    {32, 36},   // 9 Q8_1
    {256, 84},  // 10 Q2_K
    {256, 110}, // 11 Q3_K
    {256, 144}, // 12 Q4_K: d, dmin, 12 B scales, 128 B nibbles
    {256, 176}, // 13 Q5_K
    {256, 210}, // 14 Q6_K
    {256, 292}, // 15 Q8_K
    {256, 66},  // 16 IQ2_XXS
    {256, 74},  // 17 IQ2_XS
    {256, 98},  // 18 IQ3_XXS
    {256, 50},  // 19 IQ1_S
    {32, 18},   // 20 IQ4_NL
    {256, 110}, // 21 IQ3_S
    {256, 82},  // 22 IQ2_S
    {256, 136}, // 23 IQ4_XS
    {1, 1},     // 24 I8
    {1, 2},     // 25 I16
    {1, 4},     // 26 I32
    {1, 8},     // 27 I64
    {1, 8},     // 28 F64
    {256, 56},  // 29 IQ1_M
    {1, 2},     // 30 BF16
};
}  // namespace

extern "C" int ulspec_ggml_blck_size(uint32_t t)
{
    return t < sizeof(kGgmlTypes) / sizeof(kGgmlTypes[0]) ? kGgmlTypes[t].blck : 0;
}

extern "C" int ulspec_ggml_type_size(uint32_t t)
{
    return t < sizeof(kGgmlTypes) / sizeof(kGgmlTypes[0]) ? kGgmlTypes[t].bytes : 0;
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
    if (gemm_init(ctx) != ULSPEC_OK || accept_init(ctx) != ULSPEC_OK) {
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

namespace {

// Streaming read: thread t of workgroup b reads units (b * 256 * U + t + 256 u),
// u < U, every load issued before the XOR that consumes them; NT: with the
// non-temporal cache policy (no last-level cache allocation), as the verify
// GEMMs read their weights.
template <int U, bool NT>
__global__ __launch_bounds__(256) void stream_read_kernel(const uint4* __restrict__ p, size_t n16,
                                                          uint32_t* __restrict__ sink)
{
    const size_t i = (size_t)blockIdx.x * 256 * U + threadIdx.x;
    uint4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const size_t k = i + (size_t)u * 256;
        if constexpr (NT) {
            typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
            v[u] = k < n16 ? __builtin_bit_cast(uint4, __builtin_nontemporal_load((const u32x4*)(p + k)))
                           : uint4{0u, 0u, 0u, 0u};
        } else {
            v[u] = k < n16 ? p[k] : uint4{0u, 0u, 0u, 0u};
        }
    }
    uint32_t acc = 0;
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    if (acc == 0x5eed5eedu) *sink = acc;
}

// Grid-wide barrier probe: `rounds` rounds of (each workgroup writes 256
// floats, barrier, reads another workgroup's) on co-resident workgroups.  The
// barrier: thread 0 of each workgroup stores the round number into its own
// flag; wave 0 polls all flags (64 lanes, agent-scope loads) until every one
// has reached it.  mode 0: plain data stores and loads, the flag stored with
// agent-scope release and the poll followed by an agent-scope acquire (the
// L2 write-back and invalidate of the memory model); mode 1: data through
// agent-scope relaxed stores and loads, the flag stored after s_waitcnt (no
// L2 write-back or invalidate).  Every wait is bounded: past `spin_limit`
// polls a workgroup raises ctl[0] and every workgroup skips all later rounds,
// so every wave exits.
template <int MODE>
__device__ __forceinline__ bool probe_barrier(uint32_t* flags, uint32_t* ctl, uint32_t G, uint32_t round,
                                              uint32_t spin_limit)
{
    __shared__ int ok_s;
    __syncthreads();
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        int ok = 1;
        if (lane == 0) {
            if (MODE == 0) {
                __hip_atomic_store(flags + blockIdx.x, round, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
            } else {
                __builtin_amdgcn_s_waitcnt(0);
                __hip_atomic_store(flags + blockIdx.x, round, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        for (uint32_t n = 0;; ++n) {
            bool mine = true;
            for (uint32_t g = lane; g < G; g += 64)
                mine &= __hip_atomic_load(flags + g, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= round;
            if (__ballot(!mine) == 0) break;
            if (__hip_atomic_load(ctl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) || n > spin_limit) {
                if (lane == 0) __hip_atomic_store(ctl, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                ok = 0;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        if (MODE == 0) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        if (lane == 0) ok_s = ok;
    }
    __syncthreads();
    return ok_s != 0;
}

template <int MODE>
__global__ void sync_probe_kernel(uint32_t* flags, uint32_t* ctl, float* data, uint32_t rounds, uint32_t spin_limit)
{
    const uint32_t G = gridDim.x;
    uint32_t bad = 0;
    for (uint32_t it = 0; it < rounds; ++it) {
        // rounds alternate two halves of data: a workgroup writing round it's
        // half has passed barrier it - 1, so nobody still reads it
        float* half = data + (size_t)(it & 1) * G * 256;
        for (uint32_t i = threadIdx.x; i < 256; i += blockDim.x) {
            const float v = (float)(it * 7 + blockIdx.x + i);
            if (MODE == 0) half[(size_t)blockIdx.x * 256 + i] = v;
            else __hip_atomic_store(half + (size_t)blockIdx.x * 256 + i, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (MODE == 1) __builtin_amdgcn_s_waitcnt(0);
        if (!probe_barrier<MODE>(flags, ctl, G, it + 1, spin_limit)) break;
        if (threadIdx.x < 256) {
            const uint32_t o = (blockIdx.x + 1 + it) % G, i = threadIdx.x;
            const float* src = half + (size_t)o * 256 + i;
            const float v = MODE == 0 ? *src : __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (v != (float)(it * 7 + o + i)) ++bad;
        }
    }
    if (bad) atomicAdd(ctl + 1, bad);
}

}  // namespace

extern "C" ulspec_status ulspec_sync_probe(ulspec_ctx* ctx, uint32_t mode, uint32_t workgroups, uint32_t threads,
                                           uint32_t rounds, float* us_per_round, uint32_t* errors)
{
    ULSPEC_CHECK_CTX(ctx);
    if (mode > 1 || workgroups == 0 || (threads != 256 && threads != 512 && threads != 1024) || rounds == 0 ||
        rounds > 100000 || !us_per_round || !errors)
        return fail(ctx, ULSPEC_EINVAL, "sync_probe: mode 0..1, threads 256/512/1024, 1..100000 rounds, outputs");
    (void)hipSetDevice(ctx->device);
    const void* fn = mode == 0 ? (const void*)sync_probe_kernel<0> : (const void*)sync_probe_kernel<1>;
    int per_cu = 0;
    hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, (int)threads, 0);
    if (e != hipSuccess) return hip_fail(ctx, e, "sync_probe occupancy");
    if ((uint64_t)per_cu * (uint64_t)std::max(1, ctx->n_cu) < workgroups)
        return fail(ctx, ULSPEC_EINVAL, "sync_probe: %u workgroups of %u threads are not co-resident", workgroups,
                    threads);
    uint32_t *flags = nullptr, *ctl = nullptr;
    float* data = nullptr;
    e = hipMalloc(&flags, (size_t)workgroups * 4);
    if (e == hipSuccess) e = hipMalloc(&ctl, 256);
    if (e == hipSuccess) e = hipMalloc(&data, (size_t)2 * workgroups * 256 * 4);
    if (e == hipSuccess) e = hipMemsetAsync(flags, 0, (size_t)workgroups * 4, ctx->stream);
    if (e == hipSuccess) e = hipMemsetAsync(ctl, 0, 256, ctx->stream);
    const uint32_t spin_limit = 400000;  // polls of ~1 us: far past any barrier, under a second
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (e == hipSuccess) e = hipEventCreate(&e0);
    if (e == hipSuccess) e = hipEventCreate(&e1);
    if (e == hipSuccess) e = hipEventRecord(e0, ctx->stream);
    if (e == hipSuccess) {
        void* args[] = {&flags, &ctl, &data, &rounds, (void*)&spin_limit};
        e = hipLaunchCooperativeKernel(fn, dim3(workgroups), dim3(threads), args, 0, ctx->stream);
    }
    if (e == hipSuccess) e = hipEventRecord(e1, ctx->stream);
    if (e == hipSuccess) e = hipEventSynchronize(e1);
    float ms = 0.f;
    uint32_t hc[2] = {0, 0};
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
    if (e == hipSuccess) e = hipMemcpy(hc, ctl, 8, hipMemcpyDeviceToHost);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    (void)hipFree(flags);
    (void)hipFree(ctl);
    (void)hipFree(data);
    if (e != hipSuccess) return hip_fail(ctx, e, "sync_probe");
    if (hc[0]) return fail(ctx, ULSPEC_EDEVICE, "sync_probe: a barrier wait passed its spin limit");
    *us_per_round = ms * 1e3f / (float)rounds;
    *errors = hc[1];
    return ULSPEC_OK;
}

extern "C" ulspec_status ulspec_device_info(ulspec_ctx* ctx, int* device, int* n_cu)
{
    ULSPEC_CHECK_CTX(ctx);
    if (device) *device = ctx->device;
    if (n_cu) *n_cu = ctx->n_cu;
    return ULSPEC_OK;
}

extern "C" ulspec_status ulspec_set_option(ulspec_ctx* ctx, uint32_t option, int64_t value)
{
    ULSPEC_CHECK_CTX(ctx);
    if (option == ULSPEC_OPT_TOPK_ROUTE) {
        if (value < 0 || value > 4) return fail(ctx, ULSPEC_EINVAL, "set_option: top-k route %lld (0 .. 4)", (long long)value);
        ctx->topk_route = (int)value;
        return ULSPEC_OK;
    }
    return fail(ctx, ULSPEC_EINVAL, "set_option: unknown option %u", option);
}

extern "C" ulspec_status ulspec_stream_read(ulspec_ctx* ctx, const void* buf, size_t bytes, uint32_t variant,
                                            uint32_t* sink)
{
    ULSPEC_CHECK_CTX(ctx);
    if (!buf || !sink || bytes == 0 || bytes % 16 || variant > 7)
        return fail(ctx, ULSPEC_EINVAL, "stream_read: buffer, sink, bytes %% 16 == 0 and variant 0..7 required");
    (void)hipSetDevice(ctx->device);
    const size_t n16 = bytes / 16;
    const int U = 4 << (variant & 3);
    const size_t grid = (n16 + 256 * (size_t)U - 1) / (256 * (size_t)U);
    if (grid > 0x7fffffffu) return fail(ctx, ULSPEC_EINVAL, "stream_read: %zu bytes is too large", bytes);
    const uint4* p = (const uint4*)buf;
    using Kern = void (*)(const uint4*, size_t, uint32_t*);
    static const Kern kern[8] = {stream_read_kernel<4, false>,  stream_read_kernel<8, false>,
                                 stream_read_kernel<16, false>, stream_read_kernel<32, false>,
                                 stream_read_kernel<4, true>,   stream_read_kernel<8, true>,
                                 stream_read_kernel<16, true>,  stream_read_kernel<32, true>};
    hipLaunchKernelGGL(kern[variant], dim3((unsigned)grid), dim3(256), 0, ctx->stream, p, n16, sink);
    return check_launch(ctx, "stream_read launch");
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
