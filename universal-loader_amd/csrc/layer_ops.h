// layer_ops.h -- launcher of the token-embedding kernel (asynchronous on the
// given stream).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace ulspec {

// h[m][:] = dequantized row tokens[m] of the raw GGUF [V][dim] tensor (ids
// out of range read row 0); pss[m][b] = sum of squares of h[m][256 b ..
// 256 b + 255], b < embed_partials(dim); with xn, the split fp16 pairs of
// h * xn_w (rows m, then rows M + m).
uint32_t embed_partials(uint32_t dim);
void launch_embed(hipStream_t st, const uint8_t* w, uint32_t type, uint32_t dim, const int32_t* tokens, uint32_t M,
                  uint32_t V, float* h, float* pss, const float* xn_w, _Float16* xn);

// The last n of every group of r rows (nseq groups, M = nseq r rows): split
// X rows (xn: hi rows 0 .. M-1, lo rows M ..; dim halves each) and their P
// row-scale partials (pss [M][P]) -> xg (hi rows 0 .. nseq n - 1, lo rows
// nseq n ..) and pg [nseq n][P].
void launch_gather_rows(hipStream_t st, const _Float16* xn, const float* pss, uint32_t M, uint32_t dim, uint32_t P,
                        uint32_t r, uint32_t n, uint32_t nseq, _Float16* xg, float* pg);

}  // namespace ulspec
