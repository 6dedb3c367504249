// synth.hip -- synthetic random-init GGUF weights, generated on the device.
//
// Element (n, k) of an N x K weight is normal number i = n*K + k of the stream
// (seed, stream): pair p = i / 2 takes u1, u2 from splitmix64 counters 2p and
// 2p+1 of key mix64(seed ^ mix64(stream + c)); z = sqrt(-2 ln u1) cos / sin
// (2 pi u2) in double; value = (float)(0 + std * z).  The values are then
// quantized to GGUF blocks: Q4_0 with d = x_absmax / -8, q = min(15, (int)(x /
// d + 8.5)) (the ggml reference quantizer); Q4_K with per-32 affine scales and
// mins (scale = (max - min) / 15, min clamped to <= 0), both quantized to 6 bits
// against fp16 super-block factors max / 63.  The quantizer is plain IEEE fp32
// arithmetic; the normals come from the device's double log / cos / sin, so a
// value can differ from a host libm in its last bit.
#include "detmath.h"
#include "hip_common.h"
#include "ulspec_internal.h"

using namespace ulspec;

namespace {

constexpr uint64_t kNormalStreamSalt = 0x632be59bd9b4e019ull;

__device__ __forceinline__ uint64_t counter(uint64_t key, uint64_t idx)
{
    return mix64(key + (idx + 1u) * 0x9e3779b97f4a7c15ull);
}

// normals i0 .. i0 + n - 1 (i0 even, n even) of the keyed stream
__global__ void normals_kernel(uint64_t key, uint64_t i0, uint64_t n, double std_dev, float* __restrict__ out)
{
    const uint64_t p = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (2 * p >= n) return;
    const uint64_t gp = i0 / 2 + p;
    const uint64_t a = counter(key, 2 * gp), b = counter(key, 2 * gp + 1);
    const double u1 = (double)((a >> 11) + 1u) * 0x1.0p-53;  // (0, 1]
    const double u2 = (double)(b >> 11) * 0x1.0p-53;         // [0, 1)
    const double r = sqrt(-2.0 * log(u1));
    const double t = 6.283185307179586476925286766559 * u2;
    out[2 * p] = (float)(0.0 + std_dev * r * cos(t));
    out[2 * p + 1] = (float)(0.0 + std_dev * r * sin(t));
}

__device__ __forceinline__ void put16(uint8_t* p, _Float16 h)
{
    const uint16_t b = __builtin_bit_cast(uint16_t, h);
    p[0] = (uint8_t)(b & 255u);
    p[1] = (uint8_t)(b >> 8);
}

__global__ void quant_q4_0_kernel(const float* __restrict__ x, uint64_t n_blocks, uint8_t* __restrict__ out)
{
    const uint64_t b = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= n_blocks) return;
    const float* v = x + 32 * b;
    uint8_t* blk = out + 18 * b;
    float amax = 0.0f, vmax = 0.0f;
    for (int j = 0; j < 32; ++j) {
        const float a = fabsf(v[j]);
        if (a > amax) {
            amax = a;
            vmax = v[j];
        }
    }
    const float d = vmax / -8.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    put16(blk, (_Float16)d);
    for (int j = 0; j < 16; ++j) {
        int q0 = (int)(v[j] * id + 8.5f);
        int q1 = (int)(v[j + 16] * id + 8.5f);
        q0 = q0 > 15 ? 15 : (q0 < 0 ? 0 : q0);
        q1 = q1 > 15 ? 15 : (q1 < 0 ? 0 : q1);
        blk[2 + j] = (uint8_t)(q0 | (q1 << 4));
    }
}

__global__ void quant_q4_k_kernel(const float* __restrict__ x, uint64_t n_blocks, uint8_t* __restrict__ out)
{
    const uint64_t b = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= n_blocks) return;
    const float* v = x + 256 * b;
    uint8_t* blk = out + 144 * b;
    float scale[8], mins[8];
    float max_scale = 0.0f, max_min = 0.0f;
    for (int j = 0; j < 8; ++j) {
        float mn = 0.0f, mx = v[32 * j];
        for (int l = 0; l < 32; ++l) {
            const float t = v[32 * j + l];
            if (t < mn) mn = t;
            if (t > mx) mx = t;
        }
        if (mx < mn) mx = mn;
        scale[j] = (mx - mn) / 15.0f;
        mins[j] = -mn;
        if (scale[j] > max_scale) max_scale = scale[j];
        if (mins[j] > max_min) max_min = mins[j];
    }
    const _Float16 d16 = (_Float16)(max_scale / 63.0f), m16 = (_Float16)(max_min / 63.0f);
    const float dq = (float)d16, mq = (float)m16;
    int sc[8], mm[8];
    for (int j = 0; j < 8; ++j) {
        const int a = dq > 0.0f ? (int)(scale[j] / dq + 0.5f) : 0;
        const int c = mq > 0.0f ? (int)(mins[j] / mq + 0.5f) : 0;
        sc[j] = a > 63 ? 63 : a;
        mm[j] = c > 63 ? 63 : c;
    }
    put16(blk, d16);
    put16(blk + 2, m16);
    uint8_t* s = blk + 4;
    for (int j = 0; j < 4; ++j) {
        s[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        s[j + 4] = (uint8_t)((mm[j] & 63) | ((mm[j + 4] >> 4) << 6));
        s[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((mm[j + 4] & 15) << 4));
    }
    for (int c = 0; c < 4; ++c) {
        const float es0 = dq * (float)sc[2 * c], em0 = mq * (float)mm[2 * c];
        const float es1 = dq * (float)sc[2 * c + 1], em1 = mq * (float)mm[2 * c + 1];
        for (int l = 0; l < 32; ++l) {
            int q0 = es0 > 0.0f ? (int)((v[64 * c + l] + em0) / es0 + 0.5f) : 0;
            int q1 = es1 > 0.0f ? (int)((v[64 * c + 32 + l] + em1) / es1 + 0.5f) : 0;
            q0 = q0 < 0 ? 0 : (q0 > 15 ? 15 : q0);
            q1 = q1 < 0 ? 0 : (q1 > 15 ? 15 : q1);
            blk[16 + 32 * c + l] = (uint8_t)(q0 | (q1 << 4));
        }
    }
}

}  // namespace

extern "C" ulspec_status ulspec_synth_q4(ulspec_ctx* ctx, uint32_t type, uint64_t seed, uint64_t stream, uint32_t N,
                                         uint32_t K, float std_dev, void* out)
{
    ULSPEC_CHECK_CTX(ctx);
    if (type != ULSPEC_GGML_Q4_0 && type != ULSPEC_GGML_Q4_K)
        return fail(ctx, ULSPEC_EUNSUPPORTED, "synth_q4: ggml type %u not supported (Q4_0 / Q4_K)", type);
    const int bs = ulspec_ggml_blck_size(type), ts = ulspec_ggml_type_size(type);
    if (!out || N == 0 || K == 0 || K % bs) return fail(ctx, ULSPEC_EINVAL, "synth_q4: N=%u K=%u", N, K);
    if (!(std_dev >= 0.0f) || !(std_dev < __builtin_inff())) return fail(ctx, ULSPEC_EINVAL, "synth_q4: std");
    (void)hipSetDevice(ctx->device);
    const uint64_t key = mix64(seed ^ mix64(stream + kNormalStreamSalt));
    // rows in chunks of at most 8 Mi values of fp32 scratch
    const uint32_t rows = (uint32_t)std::max<uint64_t>(1, (8ull << 20) / K);
    void* ws = nullptr;
    ulspec_status st = workspace(ctx, (size_t)std::min<uint64_t>(rows, N) * K * sizeof(float), &ws);
    if (st != ULSPEC_OK) return st;
    const size_t row_bytes = (size_t)(K / bs) * ts;
    for (uint32_t r0 = 0; r0 < N; r0 += rows) {
        const uint32_t rc = std::min(rows, N - r0);
        const uint64_t n = (uint64_t)rc * K;
        hipLaunchKernelGGL(normals_kernel, dim3((unsigned)((n / 2 + 255) / 256)), dim3(256), 0, ctx->stream, key,
                           (uint64_t)r0 * K, n, (double)std_dev, (float*)ws);
        const uint64_t nb = n / bs;
        uint8_t* dst = (uint8_t*)out + (size_t)r0 * row_bytes;
        if (type == ULSPEC_GGML_Q4_0)
            hipLaunchKernelGGL(quant_q4_0_kernel, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, ctx->stream,
                               (const float*)ws, nb, dst);
        else
            hipLaunchKernelGGL(quant_q4_k_kernel, dim3((unsigned)((nb + 63) / 64)), dim3(64), 0, ctx->stream,
                               (const float*)ws, nb, dst);
    }
    return check_launch(ctx, "synth_q4 launch");
}
