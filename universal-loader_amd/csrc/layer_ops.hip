// layer_ops.hip -- token embedding of the model forward: dequantized rows of
// the raw GGUF token_embd tensor start the fp32 residual stream, with the
// per-block sums of squares its first RMSNorm consumes and the split X of the
// first GEMM (h times the norm's weights; the GEMM applies the norm's row
// factor to its outputs).  (The other Llama block steps of
// src/inference/inference_engine.cpp:602-682 -- RMSNorm, RoPE and the KV
// append, SiLU * up, the residual adds -- run fused into the dequant-GEMM's
// row scale and epilogues.)
#include "detmath.h"
#include "hip_common.h"
#include "layer_ops.h"

namespace ulspec {
namespace {

__device__ __forceinline__ float h2f_bits(uint32_t b) { return (float)__builtin_bit_cast(_Float16, (uint16_t)b); }

// Q4_0 element j of a block: low nibble of qs[j] (j < 16) / high nibble of
// qs[j-16], value (q - 8) * d.  Q4_K as in the GGUF definition (6-bit
// sub-scales / mins, chunk c of 64 elements uses qs[32c .. 32c+31]).  F16,
// Q8_0 and Q6_K as ggml defines them (the types Q4_K_M files mix in).
// Grid (ceil(dim / 256), M); block b of row m also writes pss[m][b], the sum
// of its 256 values squared (xor tree in each wave, the 4 waves in order).
// With xn, also the first GEMM's split X: rows m (hi) and xn_lo + m (lo) of h * xn_w.
__global__ __launch_bounds__(256) void embed_kernel(const uint8_t* __restrict__ w, uint32_t type, uint32_t dim,
                                                    const int32_t* __restrict__ tokens, uint32_t V,
                                                    float* __restrict__ h, float* __restrict__ pss,
                                                    const float* __restrict__ xn_w, _Float16* __restrict__ xn,
                                                    uint32_t xn_lo)
{
    __shared__ float part[4];
    const uint32_t m = blockIdx.y;
    const uint32_t e = blockIdx.x * 256 + threadIdx.x;
    int32_t tok = tokens[m];
    if (tok < 0 || (uint32_t)tok >= V) tok = 0;
    float v = 0.0f;
    if (e < dim) {
        if (type == 1) {  // F16
            v = h2f_bits(((const uint16_t*)w)[(size_t)tok * dim + e]);
        } else if (type == 8) {  // Q8_0: d * q
            const uint8_t* blk = w + ((size_t)tok * (dim / 32) + e / 32) * 34;
            v = h2f_bits(blk[0] | (blk[1] << 8)) * (float)(int8_t)blk[2 + e % 32];
        } else if (type == 14) {  // Q6_K: (d * scale) * q, ggml's block_q6_K layout
            const uint8_t* blk = w + ((size_t)tok * (dim / 256) + e / 256) * 210;
            const uint32_t i = e % 256, hh = i / 128, p = i % 128, quarter = p / 32, l = p % 32;
            const uint8_t lo = blk[64 * hh + l + (quarter & 1 ? 32 : 0)];
            const uint32_t nib = quarter < 2 ? (lo & 15u) : (lo >> 4);
            const uint32_t hb = (blk[128 + 32 * hh + l] >> (2 * quarter)) & 3u;
            const int q = (int)(nib | (hb << 4)) - 32;
            const int sc = (int8_t)blk[192 + 8 * hh + l / 16 + 2 * quarter];
            v = h2f_bits(blk[208] | (blk[209] << 8)) * (float)sc * (float)q;
        } else if (type == 2) {
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
        if (xn) {
            _Float16 hi, lo;
            split_hl(v * xn_w[e], hi, lo);
            xn[(size_t)m * dim + e] = hi;
            xn[(size_t)(xn_lo + m) * dim + e] = lo;
        }
    }
    float sq = v * v;
    sq += xor_lane<32>(sq);
    sq += xor_lane<16>(sq);
    sq += xor_lane<8>(sq);
    sq += xor_lane<4>(sq);
    sq += xor_lane<2>(sq);
    sq += xor_lane<1>(sq);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = sq;
    __syncthreads();
    if (threadIdx.x == 0) pss[(size_t)m * gridDim.x + blockIdx.x] = ((part[0] + part[1]) + part[2]) + part[3];
}

// One workgroup per gathered row i (blockIdx.x < nseq n): source row
// (i / n) r + r - n + i % n.
__global__ __launch_bounds__(256) void gather_rows_kernel(const _Float16* __restrict__ xn,
                                                          const float* __restrict__ pss, uint32_t M, uint32_t dim,
                                                          uint32_t P, uint32_t r, uint32_t n, uint32_t G,
                                                          _Float16* __restrict__ xg, float* __restrict__ pg)
{
    const uint32_t i = blockIdx.x;
    const uint32_t src = (i / n) * r + (r - n) + i % n;
    for (uint32_t c = threadIdx.x; c < dim; c += 256) {
        xg[(size_t)i * dim + c] = xn[(size_t)src * dim + c];
        xg[(size_t)(G + i) * dim + c] = xn[(size_t)(M + src) * dim + c];
    }
    for (uint32_t c = threadIdx.x; c < P; c += 256) pg[(size_t)i * P + c] = pss[(size_t)src * P + c];
}

}  // namespace

uint32_t embed_partials(uint32_t dim) { return (dim + 255) / 256; }

void launch_gather_rows(hipStream_t st, const _Float16* xn, const float* pss, uint32_t M, uint32_t dim, uint32_t P,
                        uint32_t r, uint32_t n, uint32_t nseq, _Float16* xg, float* pg)
{
    hipLaunchKernelGGL(gather_rows_kernel, dim3(nseq * n), dim3(256), 0, st, xn, pss, M, dim, P, r, n, nseq * n, xg,
                       pg);
}

void launch_embed(hipStream_t st, const uint8_t* w, uint32_t type, uint32_t dim, const int32_t* tokens, uint32_t M,
                  uint32_t V, float* h, float* pss, const float* xn_w, _Float16* xn)
{
    hipLaunchKernelGGL(embed_kernel, dim3(embed_partials(dim), M), dim3(256), 0, st, w, type, dim, tokens, V, h, pss,
                       xn_w, xn, M);
}

}  // namespace ulspec
