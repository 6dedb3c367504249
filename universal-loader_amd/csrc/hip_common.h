// hip_common.h -- vector types and small device helpers shared by the kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));

namespace ulspec {

__device__ __forceinline__ half2_t as_half2(uint32_t v) { return __builtin_bit_cast(half2_t, v); }
__device__ __forceinline__ uint32_t as_u32(half2_t h) { return __builtin_bit_cast(uint32_t, h); }

__device__ __forceinline__ float half_bits_to_float(uint32_t bits16)
{
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

__device__ __forceinline__ half8_t make_half8(half2_t a, half2_t b, half2_t c, half2_t d)
{
    half4_t lo = __builtin_shufflevector(a, b, 0, 1, 2, 3);
    half4_t hi = __builtin_shufflevector(c, d, 0, 1, 2, 3);
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

__device__ __forceinline__ half2_t splat2(float v)
{
    half2_t h = {(_Float16)v, (_Float16)v};
    return h;
}

// v from lane (lane ^ M) of the wave, M = 1, 2, 4, 8, 16 or 32: DPP moves
// (quad permutes, row shifts and rotates) and the gfx950 row and half swaps
// (v_permlane16_swap, v_permlane32_swap) instead of an LDS permute
// (ds_bpermute: a round trip through the LDS crossbar, ~100 cycles, where
// these take a few).  The values moved are the same, so a reduction written
// with them gives the same bits.  Every lane of the wave must be active.
template <int M>
__device__ __forceinline__ uint32_t xor_lane_u32(uint32_t v)
{
    const int x = (int)v;
    int r;
    if constexpr (M == 1) {
        r = __builtin_amdgcn_update_dpp(x, x, 0xb1, 0xf, 0xf, false);  // quad_perm [1, 0, 3, 2]
    } else if constexpr (M == 2) {
        r = __builtin_amdgcn_update_dpp(x, x, 0x4e, 0xf, 0xf, false);  // quad_perm [2, 3, 0, 1]
    } else if constexpr (M == 4) {
        r = __builtin_amdgcn_update_dpp(x, x, 0x104, 0xf, 0x5, false);  // row_shl:4 into lanes 0-3, 8-11 of each row
        r = __builtin_amdgcn_update_dpp(r, x, 0x114, 0xf, 0xa, false);  // row_shr:4 into lanes 4-7, 12-15
    } else if constexpr (M == 8) {
        r = __builtin_amdgcn_update_dpp(x, x, 0x128, 0xf, 0xf, false);  // row_ror:8
    } else if constexpr (M == 16) {
        // rows (0, 1, 2, 3) -> p[0] = rows (0, 0, 2, 2), p[1] = rows (1, 1, 3, 3)
        const auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        r = (int)((threadIdx.x & 16) ? p[0] : p[1]);
    } else {
        static_assert(M == 32, "xor_lane: M is 1, 2, 4, 8, 16 or 32");
        // halves (lo, hi) -> p[0] = (lo, lo), p[1] = (hi, hi)
        const auto p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        r = (int)((threadIdx.x & 32) ? p[0] : p[1]);
    }
    return (uint32_t)r;
}
template <int M>
__device__ __forceinline__ float xor_lane(float v)
{
    return __builtin_bit_cast(float, xor_lane_u32<M>(__builtin_bit_cast(uint32_t, v)));
}

// Split operand of an fp32 activation for the fp16 MFMAs: hi = fp16(x), lo =
// fp16((x - hi) * 2^11) (x - hi is exact in fp32), so x = hi + lo * 2^-11 to
// about 22 bits.  Products of either part with an fp16 weight are exact in
// fp32, so a GEMM over (hi, lo) accumulates x * w at fp32 precision.
constexpr float kLoScale = 2048.0f;
constexpr float kLoUnscale = 1.0f / 2048.0f;

__device__ __forceinline__ void split_hl(float x, _Float16& hi, _Float16& lo)
{
    hi = (_Float16)x;
    lo = (_Float16)((x - (float)hi) * kLoScale);
}

// 16x16x32 fp16 MFMA: C[i][j] += sum_k A[i][k] B[k][j].  Lane l supplies row
// i = l % 16 of A and column j = l % 16 of B (8 k values each, the same k
// slots in both), and holds C rows 4 * (l / 16) + 0..3 of column l % 16.
__device__ __forceinline__ float4_t mfma16x16x32(half8_t a, half8_t b, float4_t c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// 16x16x16 fp16 MFMA, 4 k values per lane, same row/column/C layout.
__device__ __forceinline__ float4_t mfma16x16x16(half4_t a, half4_t b, float4_t c)
{
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

}  // namespace ulspec
