// layer_ops.h -- launchers of the Llama-block kernels around the verification
// kernels (all asynchronous on the given stream).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace ulspec {

void launch_embed(hipStream_t st, const uint8_t* w, uint32_t type, uint32_t dim, const int32_t* tokens, uint32_t M,
                  uint32_t V, float* h);
void launch_add_rmsnorm(hipStream_t st, float* h, const float* delta, const float* w, uint32_t M, uint32_t dim,
                        float eps, _Float16* x);
// Positions pos0 .. pos0 + M - 1 with pos0 = *pos_dev + pos_add (device int).
void launch_rope_append(hipStream_t st, const float* qkv, uint32_t M, uint32_t H, uint32_t Hkv, uint32_t D,
                        const int32_t* pos_dev, int32_t pos_add, const float2* rope, _Float16* q16, _Float16* kc,
                        _Float16* vc);
void launch_silu_mul(hipStream_t st, const float* gu, uint32_t M, uint32_t F, _Float16* act);

}  // namespace ulspec
