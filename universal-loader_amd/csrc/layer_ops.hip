// layer_ops.hip -- the element-wise and row kernels around the three
// verification kernels in a Llama block, in the order of
// src/inference/inference_engine.cpp:602-682 (norm -> QKV -> RoPE ->
// attention -> O -> +residual -> norm -> gate/up -> SiLU * up -> down ->
// +residual).  The residual stream h stays fp32; every GEMM input is written
// as fp16 (round to nearest even).
#include "detmath.h"
#include "hip_common.h"
#include "layer_ops.h"

namespace ulspec {
namespace {

__device__ __forceinline__ float h2f_bits(uint32_t b) { return (float)__builtin_bit_cast(_Float16, (uint16_t)b); }

// ---- token embedding: dequantize rows of a raw GGUF [V][dim] tensor ----------
// Q4_0 element j of a block: low nibble of qs[j] (j < 16) / high nibble of
// qs[j-16], value (q - 8) * d.  Q4_K as in the GGUF definition (6-bit
// sub-scales / mins, chunk c of 64 elements uses qs[32c .. 32c+31]).
__global__ void embed_kernel(const uint8_t* __restrict__ w, uint32_t type, uint32_t dim,
                             const int32_t* __restrict__ tokens, uint32_t V, float* __restrict__ h)
{
    const uint32_t m = blockIdx.y;
    const uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= dim) return;
    int32_t tok = tokens[m];
    if (tok < 0 || (uint32_t)tok >= V) tok = 0;
    float v;
    if (type == 2) {
        const uint8_t* blk = w + ((size_t)tok * (dim / 32) + e / 32) * 18;
        const uint32_t j = e % 32;
        const uint32_t q = j < 16 ? (blk[2 + j] & 15u) : (blk[2 + j - 16] >> 4);
        v = (float)((int)q - 8) * h2f_bits(blk[0] | (blk[1] << 8));
    } else {
        const uint8_t* blk = w + ((size_t)tok * (dim / 256) + e / 256) * 144;
        const uint32_t i = e % 256, c = i / 64, l = i % 64, sb = 2 * c + (l >= 32);
        const uint8_t* s = blk + 4;
        uint32_t sc, mn;
        if (sb < 4) {
            sc = s[sb] & 63u;
            mn = s[sb + 4] & 63u;
        } else {
            sc = (s[sb + 4] & 15u) | ((s[sb - 4] >> 6) << 4);
            mn = (s[sb + 4] >> 4) | ((s[sb] >> 6) << 4);
        }
        const uint8_t byte = blk[16 + 32 * c + (l % 32)];
        const uint32_t q = l < 32 ? (byte & 15u) : (byte >> 4);
        const float d = h2f_bits(blk[0] | (blk[1] << 8)), dmin = h2f_bits(blk[2] | (blk[3] << 8));
        v = (d * (float)sc) * (float)q - dmin * (float)mn;
    }
    h[(size_t)m * dim + e] = v;
}

// ---- h += delta (optional); x = fp16(h * rsqrt(mean(h^2) + eps) * w) ---------
// RMSNorm as in src/shaders/ffn/ffn_fused.glsl:23-33.
constexpr int kNormThreads = 256;

__global__ __launch_bounds__(kNormThreads) void add_rmsnorm_kernel(float* __restrict__ h,
                                                                   const float* __restrict__ delta,
                                                                   const float* __restrict__ w, uint32_t dim,
                                                                   float eps, _Float16* __restrict__ x)
{
    __shared__ float part[kNormThreads / 64];
    const uint32_t m = blockIdx.x;
    float* hr = h + (size_t)m * dim;
    const float* dr = delta ? delta + (size_t)m * dim : nullptr;
    float ss = 0.0f;
    for (uint32_t i = threadIdx.x; i < dim; i += kNormThreads) {
        float v = hr[i];
        if (dr) {
            v = v + dr[i];
            hr[i] = v;
        }
        ss = __builtin_fmaf(v, v, ss);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int i = 0; i < kNormThreads / 64; ++i) tot += part[i];
    const float r = 1.0f / __builtin_sqrtf(tot / (float)dim + eps);
    for (uint32_t i = threadIdx.x; i < dim; i += kNormThreads) x[(size_t)m * dim + i] = (_Float16)((hr[i] * r) * w[i]);
}

// ---- RoPE on Q and K, write Q (fp16) and append K, V (fp16) to the cache -----
// Interleaved pairs (2i, 2i+1) rotated by theta = pos * base^(-2i / hd)
// (src/shaders/rope.glsl:50-73); cos / sin come from a host-built table.
__global__ void rope_append_kernel(const float* __restrict__ qkv, uint32_t M, uint32_t H, uint32_t Hkv, uint32_t D,
                                   const int32_t* __restrict__ pos_dev, int32_t pos_add,
                                   const float2* __restrict__ rope, _Float16* __restrict__ q16,
                                   _Float16* __restrict__ kc, _Float16* __restrict__ vc)
{
    const uint32_t pos0 = (uint32_t)(*pos_dev + pos_add);
    const uint32_t m = blockIdx.y;
    const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;  // pair index over Q, K, V
    const uint32_t qp = H * D / 2, kp = Hkv * D / 2;
    if (t >= qp + 2 * kp) return;
    const uint32_t width = (H + 2 * Hkv) * D;
    const float* row = qkv + (size_t)m * width;
    const uint32_t pos = pos0 + m;
    const float x0 = row[2 * t], x1 = row[2 * t + 1];
    if (t >= qp + kp) {  // V: no rotation
        const uint32_t u = t - qp - kp;
        _Float16* dst = vc + (size_t)pos * Hkv * D;
        dst[2 * u] = (_Float16)x0;
        dst[2 * u + 1] = (_Float16)x1;
        return;
    }
    const uint32_t u = t < qp ? t : t - qp;
    const float2 cs = rope[(size_t)pos * (D / 2) + (u % (D / 2))];
    const float a = x0 * cs.x, b = x1 * cs.y;
    const float y0 = a - b;
    const float c = x0 * cs.y, d = x1 * cs.x;
    const float y1 = c + d;
    _Float16* dst = t < qp ? q16 + (size_t)m * H * D : kc + (size_t)pos * Hkv * D;
    dst[2 * u] = (_Float16)y0;
    dst[2 * u + 1] = (_Float16)y1;
}

// ---- act = fp16(silu(gate) * up), gate = gu[:, :F], up = gu[:, F:] -----------
// SiLU x / (1 + e^-x) as in src/cpu_backend/activation_cpu.cpp:14-20.
__global__ void silu_mul_kernel(const float* __restrict__ gu, uint32_t F, _Float16* __restrict__ act)
{
    const uint32_t m = blockIdx.y;
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= F) return;
    const float g = gu[(size_t)m * 2 * F + i], u = gu[(size_t)m * 2 * F + F + i];
    const float s = g * (1.0f / (1.0f + det_expf(-g)));
    act[(size_t)m * F + i] = (_Float16)(s * u);
}

}  // namespace

void launch_embed(hipStream_t st, const uint8_t* w, uint32_t type, uint32_t dim, const int32_t* tokens, uint32_t M,
                  uint32_t V, float* h)
{
    hipLaunchKernelGGL(embed_kernel, dim3((dim + 255) / 256, M), dim3(256), 0, st, w, type, dim, tokens, V, h);
}

void launch_add_rmsnorm(hipStream_t st, float* h, const float* delta, const float* w, uint32_t M, uint32_t dim,
                        float eps, _Float16* x)
{
    hipLaunchKernelGGL(add_rmsnorm_kernel, dim3(M), dim3(kNormThreads), 0, st, h, delta, w, dim, eps, x);
}

void launch_rope_append(hipStream_t st, const float* qkv, uint32_t M, uint32_t H, uint32_t Hkv, uint32_t D,
                        const int32_t* pos_dev, int32_t pos_add, const float2* rope, _Float16* q16, _Float16* kc,
                        _Float16* vc)
{
    const uint32_t pairs = (H + 2 * Hkv) * D / 2;
    hipLaunchKernelGGL(rope_append_kernel, dim3((pairs + 255) / 256, M), dim3(256), 0, st, qkv, M, H, Hkv, D, pos_dev,
                       pos_add, rope, q16, kc, vc);
}

void launch_silu_mul(hipStream_t st, const float* gu, uint32_t M, uint32_t F, _Float16* act)
{
    hipLaunchKernelGGL(silu_mul_kernel, dim3((F + 255) / 256, M), dim3(256), 0, st, gu, F, act);
}

}  // namespace ulspec
