// q4_gemm.hip -- K1, the verify dequant-GEMM: Y[M][N] = X[M][K] . W[N][K]^T
// with W in GGUF Q4_0 / Q4_K blocks and X fp16, fp32 accumulation.
//
// The reference runs this as a separate fp32 dequantize pass plus a naive
// GEMM (src/inference/inference_engine.cpp:532-570, orientation of
// src/shaders/gemm/gemm_transposed_b_v2.glsl:23-29).  Here the weights are
// read once, dequantized in registers and fed to 16x16x32 fp16 MFMAs.
//
// Device weight layout (re-tiled at upload, same 18 / 144 bytes per block):
//   Tiles of 16 rows.  Lane l of a wave handles row r = l % 16 of the tile and
//   k-group g = l / 16 (8 consecutive elements of each 32-element block or
//   sub-block), so one 16-byte load per lane covers a 1 KB contiguous piece.
//   Within each 32-bit word the eight 4-bit values of elements e0..e7 sit at
//   nibble positions (e0,e2,e4,e6,e1,e3,e5,e7), so that masking with
//   0x000F000F / 0x00F000F0 before and after one 8-bit shift yields fp16 pairs
//   (e0,e1) (e2,e3) (e4,e5) (e6,e7) via the 0x6400 exponent trick.
//   Q4_0 chunk (tile t, block quad c) = 1152 B:
//     [0,1024)    lane l: 4 words (blocks 4c..4c+3) at l*16
//     [1024,1152) fp16 d of row r, block 4c+j at r*8 + j*2
//   Q4_K chunk (tile t, super-block s) = 2304 B:
//     [0,2048)    step j (0..7) of lane l at (j/4)*1024 + l*16 + (j%4)*4; lane
//                 group g covers qs bytes 32g..32g+31 (sub-blocks 2g, 2g+1);
//                 steps 0-3 are sub-block 2g, 4-7 sub-block 2g+1
//     [2048,2304) row r's 16-byte header at r*16: d | dmin << 16, then the
//                 eight 6-bit scales and mins re-packed per lane group: bits
//                 24g .. 24g+23 of the next 96 bits are sc[2g], sc[2g+1],
//                 m[2g], m[2g+1] (6 bits each), the same values as GGUF's
//                 12-byte packing, placed for a two-word funnel shift
//   Q6_K chunk (tile t, super-block s) = 3360 B (16 x 210, ggml's block_q6_K
//   with the 6-bit values split and re-tiled):
//     [0,2048)    low 4 bits, placed as the Q4_K nibbles (step j of lane l at
//                 (j/4)*1024 + l*16 + (j%4)*4; lane group g covers elements
//                 64g..64g+63 of the super-block, step j elements 64g+8j..+7)
//     [2048,3072) high 2 bits, word w of lane l at 2048 + l*16 + w*4 for steps
//                 2w (bit pairs at 4,20 8,24 12,28 0,16 for e0,e1 e2,e3 e4,e5
//                 e6,e7) and 2w+1 (the same positions + 2), so that masking
//                 before / after an 8-bit shift lines them up with the nibbles
//     [3072,3328) the int8 scales (one per 16 elements) of row r at r*16
//     [3328,3360) fp16 d of row r at r*2
#include <type_traits>
#include <utility>
#include <vector>

#include "detmath.h"
#include "hip_common.h"
#include "ulspec_internal.h"

#include <algorithm>

using namespace ulspec;

namespace {

constexpr int kQ40Chunk = 1152;
// Q8_0: one 16-row tile x 4 blocks (128 K): lane l holds the 8 int8 values
// k = 32 j + 8 (l >> 4) .. +7 of row l & 15 for blocks j = 0, 1 at l * 16 and
// j = 2, 3 at 1024 + l * 16 (two 1 KB coalesced loads per wave), then the
// 16 rows' 4 fp16 block scales at 2048 + row * 8.  1.0625 B per weight, as
// in GGUF.
constexpr int kQ80Chunk = 2176;
constexpr int kQ4KChunk = 2304;
constexpr int kQ6KChunk = 3360;
// fp16 weights (GGUF F16, and Q6_K or mixed-type fused weights converted at
// upload): a chunk is
// one 16-row tile x 128 K, 4 KB; lane l reads 16 contiguous bytes at
// 1024 j + 16 l for MFMA j (rows l & 15, K 32 j + 8 (l >> 4) ..).
constexpr int kF16Chunk = 4096;
// Types whose chunk is one 256-element super-block (lane group g takes
// elements 64 g .. 64 g + 63 of it); the others take 128 K per chunk.
template <int TYPE>
constexpr bool kSuperBlock = TYPE == ULSPEC_GGML_Q4_K || TYPE == ULSPEC_GGML_Q6_K;
// 16-byte X units (8 halves) per weight chunk: 128 K for Q4_0, Q8_0 and F16,
// 256 for Q4_K and Q6_K
template <int TYPE>
constexpr int kUnitsPerChunk = kSuperBlock<TYPE> ? 32 : 16;

__device__ __forceinline__ uint32_t perm_nibbles(const uint32_t q[8])
{
    // nibble position p holds element (0,2,4,6,1,3,5,7)[p]
    return q[0] | (q[2] << 4) | (q[4] << 8) | (q[6] << 12) | (q[1] << 16) | (q[3] << 20) | (q[5] << 24) |
           (q[7] << 28);
}

__global__ void repack_q4_0_kernel(const uint8_t* __restrict__ raw, uint8_t* __restrict__ out, uint32_t N,
                                   uint32_t nb, uint32_t nquads, uint64_t total)
{
    uint64_t id = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= total) return;
    const uint32_t j = id & 3;
    const uint32_t L = (id >> 2) & 63;
    const uint64_t tc = id >> 8;  // t * nquads + c
    const uint32_t c = (uint32_t)(tc % nquads);
    const uint32_t t = (uint32_t)(tc / nquads);
    const uint32_t r = L & 15, g = L >> 4;
    const uint32_t n = 16 * t + r, b = 4 * c + j;
    uint8_t* chunk = out + tc * kQ40Chunk;
    uint32_t word = 0;
    uint16_t d = 0;
    if (n < N && b < nb) {
        const uint8_t* blk = raw + ((uint64_t)n * nb + b) * 18;
        uint32_t q[8];
        for (int e = 0; e < 8; ++e) {
            uint32_t el = 8 * g + e;
            q[e] = el < 16 ? (blk[2 + el] & 15u) : (blk[2 + el - 16] >> 4);
        }
        word = perm_nibbles(q);
        d = (uint16_t)(blk[0] | (blk[1] << 8));
    }
    *(uint32_t*)(chunk + L * 16 + j * 4) = word;
    if (g == 0) *(uint16_t*)(chunk + 1024 + r * 8 + j * 2) = d;
}

// One thread per (tile, chunk, lane, block j): the lane's 8 values of block
// 4 c + j and, for lanes 0-15, the row's scale of that block; zeros past N
// and past the last block.
__global__ void repack_q8_0_kernel(const uint8_t* __restrict__ raw, uint8_t* __restrict__ out, uint32_t N,
                                   uint32_t nb, uint32_t nquads, uint64_t total)
{
    const uint64_t id = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= total) return;
    const uint32_t j = id & 3;
    const uint32_t L = (id >> 2) & 63;
    const uint64_t tc = id >> 8;  // t * nquads + c
    const uint32_t c = (uint32_t)(tc % nquads);
    const uint32_t t = (uint32_t)(tc / nquads);
    const uint32_t r = L & 15, g = L >> 4;
    const uint32_t n = 16 * t + r, b = 4 * c + j;
    uint8_t* chunk = out + tc * kQ80Chunk;
    uint32_t w0 = 0, w1 = 0;
    uint16_t d = 0;
    if (n < N && b < nb) {
        const uint8_t* blk = raw + ((uint64_t)n * nb + b) * 34;
        const uint8_t* q = blk + 2 + 8 * g;
        w0 = q[0] | (q[1] << 8) | (q[2] << 16) | ((uint32_t)q[3] << 24);
        w1 = q[4] | (q[5] << 8) | (q[6] << 16) | ((uint32_t)q[7] << 24);
        d = (uint16_t)(blk[0] | (blk[1] << 8));
    }
    uint32_t* dst = (uint32_t*)(chunk + (j >> 1) * 1024 + L * 16 + (j & 1) * 8);
    dst[0] = w0;
    dst[1] = w1;
    if (g == 0) *(uint16_t*)(chunk + 2048 + r * 8 + j * 2) = d;
}

// 6-bit scale / min of sub-block j (0..7) from the 12 packed bytes held in
// words y (bytes 0-3), z (4-7), w (8-11); branch-free in j.
__device__ __forceinline__ void q4k_scale_min(uint32_t y, uint32_t z, uint32_t w, int j, uint32_t& sc, uint32_t& m)
{
    const uint32_t sh = 8u * (uint32_t)(j & 3);
    const uint32_t by = (y >> sh) & 255u, bz = (z >> sh) & 255u, bw = (w >> sh) & 255u;
    const uint32_t sc_lo = by & 63u, m_lo = bz & 63u;
    const uint32_t sc_hi = (bw & 15u) | ((by >> 6) << 4), m_hi = (bw >> 4) | ((bz >> 6) << 4);
    const bool lo = j < 4;
    sc = lo ? sc_lo : sc_hi;
    m = lo ? m_lo : m_hi;
}

__global__ void repack_q4_k_kernel(const uint8_t* __restrict__ raw, uint8_t* __restrict__ out, uint32_t N,
                                   uint32_t nsb, uint64_t total)
{
    uint64_t id = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= total) return;
    const uint32_t j = id & 7;
    const uint32_t L = (id >> 3) & 63;
    const uint64_t ts = id >> 9;  // t * nsb + s
    const uint32_t s = (uint32_t)(ts % nsb);
    const uint32_t t = (uint32_t)(ts / nsb);
    const uint32_t r = L & 15, g = L >> 4;
    const uint32_t n = 16 * t + r;
    uint8_t* chunk = out + ts * kQ4KChunk;
    uint32_t word = 0;
    const uint8_t* blk = n < N ? raw + ((uint64_t)n * nsb + s) * 144 : nullptr;
    if (blk) {
        const uint8_t* qs = blk + 16 + 32 * g + 8 * (j & 3);
        uint32_t q[8];
        for (int e = 0; e < 8; ++e) q[e] = j < 4 ? (qs[e] & 15u) : (qs[e] >> 4);
        word = perm_nibbles(q);
    }
    *(uint32_t*)(chunk + (j >> 2) * 1024 + L * 16 + (j & 3) * 4) = word;
    if (g == 0 && j == 0) {
        uint32_t* dst = (uint32_t*)(chunk + 2048 + r * 16);
        uint32_t hw[4] = {0, 0, 0, 0};
        if (blk)
            for (int w = 0; w < 4; ++w)
                hw[w] = blk[4 * w] | (blk[4 * w + 1] << 8) | (blk[4 * w + 2] << 16) | ((uint32_t)blk[4 * w + 3] << 24);
        uint64_t lo = 0, hi = 0;  // the 96 re-packed bits
        for (int gg = 0; gg < 4; ++gg) {
            uint32_t s0, m0, s1, m1;
            q4k_scale_min(hw[1], hw[2], hw[3], 2 * gg, s0, m0);
            q4k_scale_min(hw[1], hw[2], hw[3], 2 * gg + 1, s1, m1);
            const uint64_t bits = s0 | (s1 << 6) | (m0 << 12) | (m1 << 18);
            const int at = 24 * gg;
            if (at < 64) lo |= bits << at;
            if (at + 24 > 64) hi |= at >= 64 ? bits << (at - 64) : bits >> (64 - at);
        }
        dst[0] = hw[0];
        dst[1] = (uint32_t)lo;
        dst[2] = (uint32_t)(lo >> 32);
        dst[3] = (uint32_t)hi;
    }
}

// Element i (0..255) of a ggml block_q6_K (ql[128] low nibbles, qh[64] 2-bit
// pairs, int8 scales[16], fp16 d): its 4 low bits, 2 high bits and scale.
__device__ __forceinline__ void q6k_element(const uint8_t* blk, uint32_t i, uint32_t& lo, uint32_t& hb, int& sc)
{
    const uint32_t h = i / 128, p = i % 128, quarter = p / 32, l = p % 32;
    const uint8_t byte = blk[64 * h + l + (quarter & 1 ? 32 : 0)];
    lo = quarter < 2 ? (byte & 15u) : (byte >> 4);
    hb = (blk[128 + 32 * h + l] >> (2 * quarter)) & 3u;
    sc = (int8_t)blk[192 + i / 16];
}

// One thread per (tile, super-block, lane, step j): the lane's low-nibble
// word of step j, for even j the high-bit word of steps j and j + 1, and for
// lane 0-15 / step 0 the row's scales and d; zeros past N.
__global__ void repack_q6_k_kernel(const uint8_t* __restrict__ raw, uint8_t* __restrict__ out, uint32_t N,
                                   uint32_t nsb, uint64_t total)
{
    const uint64_t id = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= total) return;
    const uint32_t j = id & 7;
    const uint32_t L = (id >> 3) & 63;
    const uint64_t ts = id >> 9;  // t * nsb + s
    const uint32_t s = (uint32_t)(ts % nsb), t = (uint32_t)(ts / nsb);
    const uint32_t r = L & 15, g = L >> 4, n = 16 * t + r;
    uint8_t* chunk = out + ts * kQ6KChunk;
    const uint8_t* blk = n < N ? raw + ((uint64_t)n * nsb + s) * 210 : nullptr;
    // bit position of the high pair of element e in its step's 16-bit pattern
    constexpr uint32_t kHPos[8] = {4, 20, 8, 24, 12, 28, 0, 16};
    uint32_t word = 0, hword = 0;
    if (blk) {
        uint32_t q[8];
        for (uint32_t e = 0; e < 8; ++e) {
            uint32_t hb;
            int sc;
            q6k_element(blk, 64 * g + 8 * j + e, q[e], hb, sc);
        }
        word = perm_nibbles(q);
        for (uint32_t st = 0; st < 2 && (j & 1) == 0; ++st)
            for (uint32_t e = 0; e < 8; ++e) {
                uint32_t lo, hb;
                int sc;
                q6k_element(blk, 64 * g + 8 * (j + st) + e, lo, hb, sc);
                hword |= hb << (kHPos[e] + 2 * st);
            }
    }
    *(uint32_t*)(chunk + (j >> 2) * 1024 + L * 16 + (j & 3) * 4) = word;
    if ((j & 1) == 0) *(uint32_t*)(chunk + 2048 + L * 16 + (j >> 1) * 4) = hword;
    if (g == 0 && j == 0) {
        uint32_t* dst = (uint32_t*)(chunk + 3072 + r * 16);
        for (int w = 0; w < 4; ++w) {
            uint32_t v = 0;
            if (blk)
                v = blk[192 + 4 * w] | (blk[193 + 4 * w] << 8) | (blk[194 + 4 * w] << 16) |
                    ((uint32_t)blk[195 + 4 * w] << 24);
            dst[w] = v;
        }
        *(uint16_t*)(chunk + 3328 + r * 2) = blk ? (uint16_t)(blk[208] | (blk[209] << 8)) : (uint16_t)0;
    }
}

// GGUF rows -> fp16 rows (row r to out row out_row0 + r * out_row_step).
// Q8_0: d * q; Q6_K: d * scale * q with the 6-bit q of ggml's block_q6_K (ql
// low nibbles, qh 2-bit pairs, int8 scales per 16 elements, fp16 d last);
// Q4_0 / Q4_K (only for fused weights whose parts mix types) as in their own
// kernels.  Evaluated in fp32 and rounded once to fp16 (the only inexact step).
__global__ void dequant_rows_f16_kernel(const uint8_t* __restrict__ raw, _Float16* __restrict__ out, uint32_t type,
                                        uint32_t K, uint64_t row_bytes, uint64_t total, uint32_t out_row0,
                                        uint32_t out_row_step)
{
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const uint64_t row = i / K;
    const uint32_t k = (uint32_t)(i - row * K);
    const uint8_t* r = raw + row * row_bytes;
    float v;
    if (type == ULSPEC_GGML_Q4_0) {  // (q - 8) * d
        const uint8_t* blk = r + (uint64_t)(k / 32) * 18;
        const uint32_t j = k % 32, q = j < 16 ? (blk[2 + j] & 15u) : (blk[2 + j - 16] >> 4);
        v = (float)((int)q - 8) * half_bits_to_float(blk[0] | (blk[1] << 8));
    } else if (type == ULSPEC_GGML_Q4_K) {  // (d * sc) * q - dmin * m
        const uint8_t* blk = r + (uint64_t)(k / 256) * 144;
        const uint32_t e = k % 256, c = e / 64, l = e % 64, sb = 2 * c + (l >= 32);
        const uint8_t* sx = blk + 4;
        const uint32_t sc = sb < 4 ? (sx[sb] & 63u) : ((sx[sb + 4] & 15u) | ((sx[sb - 4] >> 6) << 4));
        const uint32_t mn = sb < 4 ? (sx[sb + 4] & 63u) : ((sx[sb + 4] >> 4) | ((sx[sb] >> 6) << 4));
        const uint8_t byte = blk[16 + 32 * c + l % 32];
        const uint32_t q = l < 32 ? (byte & 15u) : (byte >> 4);
        v = (half_bits_to_float(blk[0] | (blk[1] << 8)) * (float)sc) * (float)q -
            half_bits_to_float(blk[2] | (blk[3] << 8)) * (float)mn;
    } else if (type == ULSPEC_GGML_F16) {
        v = (float)((const _Float16*)r)[k];
    } else if (type == ULSPEC_GGML_Q8_0) {
        const uint8_t* blk = r + (uint64_t)(k / 32) * 34;
        v = half_bits_to_float(blk[0] | (blk[1] << 8)) * (float)(int8_t)blk[2 + k % 32];
    } else {  // Q6_K
        const uint8_t* blk = r + (uint64_t)(k / 256) * 210;
        uint32_t nib, hb;
        int sc;
        q6k_element(blk, k % 256, nib, hb, sc);
        const int q = (int)(nib | (hb << 4)) - 32;
        v = half_bits_to_float(blk[208] | (blk[209] << 8)) * (float)sc * (float)q;
    }
    out[((uint64_t)out_row0 + row * out_row_step) * K + k] = (_Float16)v;
}

// fp16 rows [N][K] -> kF16Chunk tiles; one 16-byte lane slot per thread,
// zero past N or K.
__global__ void repack_f16_kernel(const _Float16* __restrict__ src, uint8_t* __restrict__ out, uint32_t N,
                                  uint32_t K, uint32_t n_chunks, uint64_t total)
{
    const uint64_t id = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= total) return;
    const uint32_t l = (uint32_t)(id & 63), j = (uint32_t)((id >> 6) & 3);
    const uint64_t tc = id >> 8;  // t * n_chunks + c
    const uint32_t c = (uint32_t)(tc % n_chunks), t = (uint32_t)(tc / n_chunks);
    const uint32_t n = 16 * t + (l & 15), k0 = 128 * c + 32 * j + 8 * (l >> 4);
    half8_t v = {};
    if (n < N)
        for (int e = 0; e < 8; ++e)
            if (k0 + e < K) v[e] = src[(uint64_t)n * K + k0 + e];
    *(half8_t*)(out + tc * kF16Chunk + j * 1024 + l * 16) = v;
}

// Compiler-only barrier: loads issued before it stay before it (they are not
// sunk to their first use), so all of a batch's loads are in flight together.
// The hardware still overlaps them; s_waitcnt is placed at each first use.
__device__ __forceinline__ void pin_loads() { asm volatile("" ::: "memory"); }

// Workgroup barrier after this wave's LDS accesses have completed; no memory
// fence, so vector loads in flight stay in flight across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Wait until every vector-memory operation but the N youngest has completed;
// no barrier.  After this wave's own buffer->LDS copies followed by N register
// loads, the wave may read what it copied.
template <int N>
__device__ __forceinline__ void vm_wait()
{
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

#define ULSPEC_VM_CASE(n) \
    case n: vm_wait<n>(); break;
#define ULSPEC_VM_CASE8(n) \
    ULSPEC_VM_CASE(n) ULSPEC_VM_CASE(n + 1) ULSPEC_VM_CASE(n + 2) ULSPEC_VM_CASE(n + 3) \
    ULSPEC_VM_CASE(n + 4) ULSPEC_VM_CASE(n + 5) ULSPEC_VM_CASE(n + 6) ULSPEC_VM_CASE(n + 7)

// vm_wait with a wave-uniform count n known only at run time (a jump table);
// counts outside 0..63 wait for everything.
__device__ __forceinline__ void vm_wait_dyn(int n)
{
    switch (n) {
        ULSPEC_VM_CASE8(0) ULSPEC_VM_CASE8(8) ULSPEC_VM_CASE8(16) ULSPEC_VM_CASE8(24)
        ULSPEC_VM_CASE8(32) ULSPEC_VM_CASE8(40) ULSPEC_VM_CASE8(48) ULSPEC_VM_CASE8(56)
    default: vm_wait<0>();
    }
}
#undef ULSPEC_VM_CASE8
#undef ULSPEC_VM_CASE

// Raw buffer loads: 32-bit offsets from a base held in scalar registers, and
// the hardware returns 0 for offsets at or past num_records instead of
// faulting (such a load still occupies the texture unit like any other).  0x00020000 is the gfx9-family dword-3 of the resource.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off)
{
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// Weight loads are non-temporal: a weight is read once per call, and the
// step streams gigabytes of other weights and K / V before it comes back, so
// allocating it in the last-level cache only evicts the activations the next
// kernel reads.  (A plain streaming read of 2 GB: 5.47 TB/s plain, 5.78 TB/s
// non-temporal, and a 160 MB buffer read before it stays cache-resident; the
// 7B target's verify GEMMs as the step runs them 13.15 -> 12.90 us per call.)
constexpr int kWeightCache = 2;  // the nt bit of the buffer instructions' cache policy

__device__ __forceinline__ uint4 wt_load16(__amdgpu_buffer_rsrc_t r, uint32_t off)
{
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kWeightCache));
}

__device__ __forceinline__ uint2 wt_load8(__amdgpu_buffer_rsrc_t r, uint32_t off)
{
    return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, kWeightCache));
}

__device__ __forceinline__ half8_t buf_load_h8(__amdgpu_buffer_rsrc_t r, uint32_t off)
{
    return __builtin_bit_cast(half8_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// (v & mask) | magic as one v_and_or_b32 (gfx9 VOP3 takes no two literals,
// so the compiler would otherwise split it).
__device__ __forceinline__ uint32_t and_or(uint32_t v, uint32_t mask, uint32_t magic)
{
    uint32_t o;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(o) : "v"(v), "v"(mask), "v"(magic));
    return o;
}

// Masks and the fp16 exponent magic, kept in VGPRs.
struct NibbleConsts {
    uint32_t lo, hi, magic;
};

__device__ __forceinline__ NibbleConsts nibble_consts()
{
    NibbleConsts k;
    k.lo = 0x000F000Fu;
    k.hi = 0x00F000F0u;
    k.magic = 0x64006400u;
    // keep them in registers across the loop
    asm volatile("" : "+v"(k.lo), "+v"(k.hi), "+v"(k.magic));
    return k;
}

// 8 nibbles in the tiled order -> fp16 (1024+q, 1024+16q, 1024+q, 1024+16q) pairs
struct MagicPairs {
    half2_t a, b, c, d;  // (e0,e1) q, (e2,e3) 16q, (e4,e5) q, (e6,e7) 16q
};

__device__ __forceinline__ MagicPairs magic_pairs(uint32_t v, const NibbleConsts& k)
{
    const uint32_t v8 = v >> 8;
    MagicPairs m;
    m.a = as_half2(and_or(v, k.lo, k.magic));
    m.b = as_half2(and_or(v, k.hi, k.magic));
    m.c = as_half2(and_or(v8, k.lo, k.magic));
    m.d = as_half2(and_or(v8, k.hi, k.magic));
    return m;
}

// Q4_0: (q - 8) exactly, elements e0..e7.
__device__ __forceinline__ half8_t dequant_q4_0(uint32_t v, const NibbleConsts& k)
{
    MagicPairs m = magic_pairs(v, k);
    const half2_t c1032 = splat2(-1032.0f), s16 = splat2(0.0625f), c72 = splat2(-72.0f);
    half2_t a = m.a + c1032;
    half2_t b = __builtin_elementwise_fma(m.b, s16, c72);
    half2_t c = m.c + c1032;
    half2_t d = __builtin_elementwise_fma(m.d, s16, c72);
    return make_half8(a, b, c, d);
}

// Q4_K: q * sc exactly (q <= 15, sc <= 63 -> <= 945).
struct SubScale {
    half2_t sc, nsc1024, sc16, nsc64;
};

__device__ __forceinline__ half8_t dequant_q4_k(uint32_t v, const SubScale& s, const NibbleConsts& k)
{
    MagicPairs m = magic_pairs(v, k);
    half2_t a = __builtin_elementwise_fma(m.a, s.sc, s.nsc1024);
    half2_t b = __builtin_elementwise_fma(m.b, s.sc16, s.nsc64);
    half2_t c = __builtin_elementwise_fma(m.c, s.sc, s.nsc1024);
    half2_t d = __builtin_elementwise_fma(m.d, s.sc16, s.nsc64);
    return make_half8(a, b, c, d);
}


// ---- X operand and common pieces -------------------------------------------
// X is fp16 rows [M][K] (hl = 0), or split fp32 activations (hl = 1): the
// high parts (split_hl) of rows 0..M-1, and the low part of row m at row
// lo_rows + m.  In split mode an MFMA covers 8 output rows: A-operand slots
// 0-7 take the high parts of 8 rows, slots 8-15 the low parts of the same
// rows, and the two halves of the result are added in the epilogue (hi + lo *
// 2^-11), so M <= 8 per 16-column tile.
constexpr int kWaves = 16;
constexpr uint32_t kOOB = 0x80000000u;  // >= any buffer's num_records

struct GemmArgs {
    const uint8_t* w;
    uint32_t w_bytes;
    const _Float16* x;
    float* out;  // Y, or the slice partials [ks_count][M][N] of the split-K kernel
    int M, N, K, n_tiles, n_chunks, ks_count;
    int ks_q, ks_r;  // n_chunks = ks_q * ks_count + ks_r; slice s starts at s * ks_q + min(s, ks_r)
    int hl;          // split X (see above)
    int lo_rows;     // split X: row of X holding the low part of row 0
    int xrows;       // rows of X staged: M, or 2M when split
    GemmFuse f;      // row scale and epilogue
};

// X row behind staged row rho (0 .. xrows-1).
__device__ __forceinline__ int x_row(const GemmArgs& a, int rho)
{
    return a.hl && rho >= a.M ? a.lo_rows + rho - a.M : rho;
}

// Bytes of X the kernels may read.
__device__ __forceinline__ uint32_t x_bytes(const GemmArgs& a)
{
    return (uint32_t)(a.hl ? a.lo_rows + a.M : a.M) * (uint32_t)a.K * 2u;
}

// Staged row that A-operand slot r (0..15) of column tile mt reads; slots past
// the last row repeat it (their outputs are never stored).
__device__ __forceinline__ int xslot_row(const GemmArgs& a, int mt, int r)
{
    if (!a.hl) return min(16 * mt + r, a.M - 1);
    const int m = min(8 * mt + (r & 7), a.M - 1);
    return r < 8 ? m : a.M + m;
}

// Output row of accumulator element i of lane `lane` in column tile mt, or
// -1 where the element is a low-part slot of split X.
__device__ __forceinline__ int acc_row(const GemmArgs& a, int mt, int lane, int i)
{
    if (!a.hl) return 16 * mt + 4 * (lane >> 4) + i;
    return lane < 32 ? 8 * mt + 4 * (lane >> 4) + i : -1;
}

__device__ __forceinline__ void slice_range(const GemmArgs& a, int ks, int& lo, int& hi)
{
    lo = ks * a.ks_q + min(ks, a.ks_r);
    hi = lo + a.ks_q + (ks < a.ks_r ? 1 : 0);
}

// ---- weights: one batch of up to CMAX chunks of one tile, in registers ------
template <int TYPE, int CMAX>
struct WBatch;
template <int CMAX>
struct WBatch<ULSPEC_GGML_Q4_0, CMAX> {
    static constexpr int kLoadsPerChunk = 2;
    uint4 wq[CMAX];
    uint2 sc[CMAX];
};
template <int CMAX>
struct WBatch<ULSPEC_GGML_Q4_K, CMAX> {
    static constexpr int kLoadsPerChunk = 3;
    uint4 w0[CMAX], w1[CMAX], hd[CMAX];
};
template <int CMAX>
struct WBatch<ULSPEC_GGML_Q6_K, CMAX> {
    static constexpr int kLoadsPerChunk = 5;
    uint4 w0[CMAX], w1[CMAX], hb[CMAX];
    uint32_t sc[CMAX], d[CMAX];
};
template <int CMAX>
struct WBatch<ULSPEC_GGML_Q8_0, CMAX> {
    static constexpr int kLoadsPerChunk = 3;
    uint4 w0[CMAX], w1[CMAX];
    uint2 sc[CMAX];
};
template <int CMAX>
struct WBatch<ULSPEC_GGML_F16, CMAX> {
    static constexpr int kLoadsPerChunk = 4;
    uint4 w[CMAX][4];
};

// Chunk c of tile t into slot i of b.  Every slot's loads are issued (out of
// range when !ok or t is past the last tile: the load returns 0 and moves no
// data), so the loads in flight are a compile-time count and each chunk
// waits for exactly its own.
template <int TYPE, int CMAX>
__device__ __forceinline__ void load_slot(const GemmArgs& a, __amdgpu_buffer_rsrc_t wr, int t, int c, bool ok, int i,
                                          WBatch<TYPE, CMAX>& b)
{
    const int lane = threadIdx.x & 63, r = lane & 15;
    ok = ok && t < a.n_tiles;
    const uint32_t ch = (uint32_t)(t < a.n_tiles ? t : 0) * (uint32_t)a.n_chunks + (uint32_t)c;
    if constexpr (TYPE == ULSPEC_GGML_F16) {
        const uint32_t o = ch * kF16Chunk + lane * 16;
#pragma unroll
        for (int j = 0; j < 4; ++j) b.w[i][j] = wt_load16(wr, ok ? o + 1024u * j : kOOB);
    } else if constexpr (TYPE == ULSPEC_GGML_Q8_0) {
        const uint32_t o = ch * kQ80Chunk;
        b.w0[i] = wt_load16(wr, ok ? o + lane * 16 : kOOB);
        b.w1[i] = wt_load16(wr, ok ? o + 1024 + lane * 16 : kOOB);
        b.sc[i] = wt_load8(wr, ok ? o + 2048 + r * 8 : kOOB);
    } else if constexpr (TYPE == ULSPEC_GGML_Q4_0) {
        const uint32_t o = ch * kQ40Chunk;
        b.wq[i] = wt_load16(wr, ok ? o + lane * 16 : kOOB);
        b.sc[i] = wt_load8(wr, ok ? o + 1024 + r * 8 : kOOB);
    } else if constexpr (TYPE == ULSPEC_GGML_Q6_K) {
        const uint32_t o = ch * kQ6KChunk;
        b.w0[i] = wt_load16(wr, ok ? o + lane * 16 : kOOB);
        b.w1[i] = wt_load16(wr, ok ? o + 1024 + lane * 16 : kOOB);
        b.hb[i] = wt_load16(wr, ok ? o + 2048 + lane * 16 : kOOB);
        b.sc[i] = __builtin_amdgcn_raw_buffer_load_b32(wr, ok ? o + 3072 + r * 16 + (lane >> 4) * 4 : kOOB, 0, kWeightCache);
        b.d[i] = __builtin_amdgcn_raw_buffer_load_b16(wr, ok ? o + 3328 + r * 2 : kOOB, 0, kWeightCache);
    } else {
        const uint32_t o = ch * kQ4KChunk;
        b.w0[i] = wt_load16(wr, ok ? o + lane * 16 : kOOB);
        b.w1[i] = wt_load16(wr, ok ? o + 1024 + lane * 16 : kOOB);
        b.hd[i] = wt_load16(wr, ok ? o + 2048 + r * 16 : kOOB);
    }
}

// Chunks c0 .. c0 + nc - 1 of tile t into slots 0 .. nc - 1 (the rest out of range).
template <int TYPE, int CMAX>
__device__ __forceinline__ void stream_load(const GemmArgs& a, __amdgpu_buffer_rsrc_t wr, int t, int c0, int nc,
                                            WBatch<TYPE, CMAX>& b)
{
#pragma unroll
    for (int i = 0; i < CMAX; ++i) load_slot<TYPE, CMAX>(a, wr, t, c0 + i, i < nc, i, b);
}

// ---- dequantize + MFMA -------------------------------------------------------
// acc[mt] += slots i0 <= i < min(i1, nc) of the batch, chunk c0 + i.  The A
// operand of slot i, K step j comes from LDS unit xrow[mt] + cs * (c0 + i) + 4 j
// (Q4_0 / Q8_0 / F16: 32-element blocks of 4 units) or + j (Q4_K: 8 steps of
// one unit in each lane group's 64-element run); cs = units per chunk stride.
template <int CMAX, int MT>
__device__ __forceinline__ void q4_0_mma(const uint4* xs, const int (&xrow)[MT], int cs, int c0, int nc, int i0,
                                         int i1, const WBatch<ULSPEC_GGML_Q4_0, CMAX>& b, const NibbleConsts& nk,
                                         float4_t (&acc)[MT])
{
    const float4_t zero4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = i0; i < i1; ++i) {
        if (i < nc) {
            const uint32_t words[4] = {b.wq[i].x, b.wq[i].y, b.wq[i].z, b.wq[i].w};
            const uint32_t sw[2] = {b.sc[i].x, b.sc[i].y};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const half8_t B = dequant_q4_0(words[j], nk);
                const float d = half_bits_to_float((sw[j >> 1] >> (16 * (j & 1))) & 0xffffu);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const half8_t A = __builtin_bit_cast(half8_t, xs[xrow[mt] + cs * (c0 + i) + 4 * j]);
                    const float4_t pr = mfma16x16x32(A, B, zero4);
                    acc[mt] = __builtin_elementwise_fma((float4_t)d, pr, acc[mt]);
                }
            }
        }
    }
}

// Eight int8 values (two words) -> fp16, exactly: each biased byte b ^ 0x80
// under exponent 0x64 is 1024 + (b + 128); subtracting 1152 leaves b.
__device__ __forceinline__ half8_t dequant_q8_0(uint32_t lo, uint32_t hi)
{
    const uint32_t x0 = lo ^ 0x80808080u, x1 = hi ^ 0x80808080u;
    const uint4 u = {(x0 & 0xffu) | ((x0 & 0xff00u) << 8) | 0x64006400u,
                     ((x0 >> 16) & 0xffu) | ((x0 >> 8) & 0xff0000u) | 0x64006400u,
                     (x1 & 0xffu) | ((x1 & 0xff00u) << 8) | 0x64006400u,
                     ((x1 >> 16) & 0xffu) | ((x1 >> 8) & 0xff0000u) | 0x64006400u};
    return __builtin_bit_cast(half8_t, u) - (half8_t)(_Float16)1152.0f;
}

// acc[mt] += d_block * (A . q) per block, as for Q4_0.
template <int CMAX, int MT>
__device__ __forceinline__ void q8_0_mma(const uint4* xs, const int (&xrow)[MT], int cs, int c0, int nc, int i0,
                                         int i1, const WBatch<ULSPEC_GGML_Q8_0, CMAX>& b, float4_t (&acc)[MT])
{
    const float4_t zero4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = i0; i < i1; ++i) {
        if (i < nc) {
            const uint32_t words[8] = {b.w0[i].x, b.w0[i].y, b.w0[i].z, b.w0[i].w,
                                       b.w1[i].x, b.w1[i].y, b.w1[i].z, b.w1[i].w};
            const uint32_t sw[2] = {b.sc[i].x, b.sc[i].y};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const half8_t B = dequant_q8_0(words[2 * j], words[2 * j + 1]);
                const float d = half_bits_to_float((sw[j >> 1] >> (16 * (j & 1))) & 0xffffu);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const half8_t A = __builtin_bit_cast(half8_t, xs[xrow[mt] + cs * (c0 + i) + 4 * j]);
                    const float4_t pr = mfma16x16x32(A, B, zero4);
                    acc[mt] = __builtin_elementwise_fma((float4_t)d, pr, acc[mt]);
                }
            }
        }
    }
}

// Q4_K chunk header of lane group g: d, dmin, the sub-scales of sub-blocks
// 2g and 2g + 1 (fp16 products for dequant_q4_k, exact) and their 6-bit mins
// (bits 0-5 and 6-11 of mn).
struct Q4KHead {
    float d, dmin;
    SubScale ss[2];
    uint32_t mn;
};

__device__ __forceinline__ Q4KHead q4k_head(uint4 h, int g)
{
    Q4KHead q;
    q.d = half_bits_to_float(h.x & 0xffffu);
    q.dmin = half_bits_to_float(h.x >> 16);
    // this lane group's 24 bits: (z:y) >> 24g for g < 2, (w:z) >> (24g - 32) beyond
    const uint64_t pair = g < 2 ? ((uint64_t)h.z << 32 | h.y) : ((uint64_t)h.w << 32 | h.z);
    const uint32_t bits = (uint32_t)(pair >> (g < 2 ? 24 * g : 24 * g - 32));
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const uint32_t scv = (bits >> (6 * e)) & 63u;
        const _Float16 hs = (_Float16)(uint16_t)scv;  // exact, as are the products below
        q.ss[e].sc = half2_t{hs, hs};
        q.ss[e].nsc1024 = q.ss[e].sc * splat2(-1024.0f);
        q.ss[e].sc16 = q.ss[e].sc * splat2(0.0625f);
        q.ss[e].nsc64 = q.ss[e].sc * splat2(-64.0f);
    }
    q.mn = (bits >> 12) & 4095u;
    return q;
}

// Q4_K: B = q * sc exactly, one MFMA chain per super-block scaled by d, and the
// min term as a second chain with the 6-bit mins as the B operand, scaled by
// -dmin.
template <int CMAX, int MT>
__device__ __forceinline__ void q4_k_mma(const uint4* xs, const int (&xrow)[MT], int cs, int c0, int nc, int i0,
                                         int i1, const WBatch<ULSPEC_GGML_Q4_K, CMAX>& b, int g,
                                         const NibbleConsts& nk, float4_t (&acc)[MT])
{
    const float4_t zero4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = i0; i < i1; ++i) {
        if (i < nc) {
            const uint32_t words[8] = {b.w0[i].x, b.w0[i].y, b.w0[i].z, b.w0[i].w,
                                       b.w1[i].x, b.w1[i].y, b.w1[i].z, b.w1[i].w};
            const Q4KHead hd = q4k_head(b.hd[i], g);
            half8_t mins[2];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const _Float16 hm = (_Float16)(uint16_t)((hd.mn >> (6 * e)) & 63u);
                mins[e] = half8_t{hm, hm, hm, hm, hm, hm, hm, hm};
            }
            float4_t P1[MT], P2[MT];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                P1[mt] = zero4;
                P2[mt] = zero4;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const half8_t B = dequant_q4_k(words[j], hd.ss[j >> 2], nk);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const half8_t A = __builtin_bit_cast(half8_t, xs[xrow[mt] + cs * (c0 + i) + j]);
                    P1[mt] = mfma16x16x32(A, B, P1[mt]);
                    P2[mt] = mfma16x16x32(A, mins[j >> 2], P2[mt]);
                }
            }
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                acc[mt] = __builtin_elementwise_fma((float4_t)hd.d, P1[mt], acc[mt]);
                acc[mt] = __builtin_elementwise_fma((float4_t)(-hd.dmin), P2[mt], acc[mt]);
            }
        }
    }
}

// Q4_K with the min term from sub-block sums of X (the split-K kernel, which
// stages X through registers and sums it on the way): xsum holds, per staged
// row and chunk, the 8 sub-blocks' (hi, lo) fp16 pairs of s / 32 (lo scaled
// by 2^11, so hi + lo 2^-11 keeps 22 bits of the fp32 sum s); slot
// srow[mt] + 4 i is lane group g's pairs of sub-blocks 2g, 2g + 1.  One
// 16x16x16 MFMA per chunk and column tile against B = the row's mins times 32
// (high slots) and 2^-6 (low slots) -- exact fp16 -- gives sum_sb min * s,
// in place of a second 16x16x32 chain of 8.
template <int CMAX, int MT>
__device__ __forceinline__ void q4_k_mma_xs(const uint4* xs, const uint2* xsum, const int (&xrow)[MT],
                                            const int (&srow)[MT], int nc, const WBatch<ULSPEC_GGML_Q4_K, CMAX>& b,
                                            int g, const NibbleConsts& nk, float4_t (&acc)[MT])
{
    constexpr int UPC = kUnitsPerChunk<ULSPEC_GGML_Q4_K>;
    const float4_t zero4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < CMAX; ++i) {
        if (i < nc) {
            const uint32_t words[8] = {b.w0[i].x, b.w0[i].y, b.w0[i].z, b.w0[i].w,
                                       b.w1[i].x, b.w1[i].y, b.w1[i].z, b.w1[i].w};
            const Q4KHead hd = q4k_head(b.hd[i], g);
            const _Float16 m0 = (_Float16)(uint16_t)(hd.mn & 63u), m1 = (_Float16)(uint16_t)(hd.mn >> 6);
            const half4_t B2 = {m0 * (_Float16)32.0f, m0 * (_Float16)0.015625f, m1 * (_Float16)32.0f,
                                m1 * (_Float16)0.015625f};
            float4_t P1[MT];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) P1[mt] = zero4;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const half8_t B = dequant_q4_k(words[j], hd.ss[j >> 2], nk);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const half8_t A = __builtin_bit_cast(half8_t, xs[xrow[mt] + UPC * i + j]);
                    P1[mt] = mfma16x16x32(A, B, P1[mt]);
                }
            }
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const float4_t P2 = mfma16x16x16(__builtin_bit_cast(half4_t, xsum[srow[mt] + 4 * i]), B2, zero4);
                acc[mt] = __builtin_elementwise_fma((float4_t)hd.d, P1[mt], acc[mt]);
                acc[mt] = __builtin_elementwise_fma((float4_t)(-hd.dmin), P2, acc[mt]);
            }
        }
    }
}

// Q6_K: 8 values -> fp16 (q - 32) * sc, q = low nibble | high pair << 4.  The
// magic 0x6400 pairs are 1024 + q (pairs a, c) or 1024 + 16 q (b, d), the
// high pairs ORed in under the magic first; subtracting 1056 / 1536 leaves
// q - 32 / 16 (q - 32) exactly, and one multiply by sc / sc/16 rounds only
// where |(q - 32) sc| > 2048 (2^-12 relative, as an fp16 copy of the
// weight).  hx: the step's high-bit word (shifted right by 2 for odd steps).
struct Q6Consts {
    uint32_t m30, m300;  // 0x00300030, 0x03000300
};

__device__ __forceinline__ Q6Consts q6_consts()
{
    Q6Consts k;
    k.m30 = 0x00300030u;
    k.m300 = 0x03000300u;
    asm volatile("" : "+v"(k.m30), "+v"(k.m300));
    return k;
}

struct Q6Scale {
    half2_t s1, s16;  // sc, sc / 16
};

__device__ __forceinline__ Q6Scale q6_scale(int sc)
{
    const float f = (float)sc;
    return Q6Scale{splat2(f), splat2(f * 0.0625f)};
}

__device__ __forceinline__ half8_t dequant_q6_k(uint32_t v, uint32_t hx, const Q6Scale& s, const NibbleConsts& k,
                                                const Q6Consts& k6)
{
    const uint32_t v8 = v >> 8;
    const uint32_t ta = and_or(hx, k6.m30, k.magic), tb = and_or(hx, k6.m300, k.magic);
    const uint32_t tc = and_or(hx >> 8, k6.m30, k.magic), td = and_or(hx << 8, k6.m300, k.magic);
    const half2_t c1056 = splat2(-1056.0f), c1536 = splat2(-1536.0f);
    const half2_t a = as_half2(and_or(v, k.lo, ta)) + c1056, b = as_half2(and_or(v, k.hi, tb)) + c1536;
    const half2_t c = as_half2(and_or(v8, k.lo, tc)) + c1056, d = as_half2(and_or(v8, k.hi, td)) + c1536;
    return make_half8(a * s.s1, b * s.s16, c * s.s1, d * s.s16);
}

// acc += d * (X . B) per chunk; lane group g's steps 2q, 2q + 1 share scale
// byte q of its scale word (elements 64 g + 16 q ..).
template <int CMAX, int MT>
__device__ __forceinline__ void q6_k_mma(const uint4* xs, const int (&xrow)[MT], int cs, int c0, int nc, int i0,
                                         int i1, const WBatch<ULSPEC_GGML_Q6_K, CMAX>& b, const NibbleConsts& nk,
                                         float4_t (&acc)[MT])
{
    const float4_t zero4 = {0.f, 0.f, 0.f, 0.f};
    const Q6Consts k6 = q6_consts();
#pragma unroll
    for (int i = i0; i < i1; ++i) {
        if (i < nc) {
            const uint32_t words[8] = {b.w0[i].x, b.w0[i].y, b.w0[i].z, b.w0[i].w,
                                       b.w1[i].x, b.w1[i].y, b.w1[i].z, b.w1[i].w};
            const uint32_t hw[4] = {b.hb[i].x, b.hb[i].y, b.hb[i].z, b.hb[i].w};
            const float dd = half_bits_to_float(b.d[i] & 0xffffu);
            float4_t P[MT];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) P[mt] = zero4;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const Q6Scale sc = q6_scale((int)(int8_t)(b.sc[i] >> (8 * q)));
#pragma unroll
                for (int st = 0; st < 2; ++st) {
                    const int j = 2 * q + st;
                    const half8_t B = dequant_q6_k(words[j], st ? hw[q] >> 2 : hw[q], sc, nk, k6);
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) {
                        const half8_t A = __builtin_bit_cast(half8_t, xs[xrow[mt] + cs * (c0 + i) + j]);
                        P[mt] = mfma16x16x32(A, B, P[mt]);
                    }
                }
            }
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) acc[mt] = __builtin_elementwise_fma((float4_t)dd, P[mt], acc[mt]);
        }
    }
}

// F16: four MFMAs of 32 K per chunk, no dequantization.
template <int CMAX, int MT>
__device__ __forceinline__ void f16_mma(const uint4* xs, const int (&xrow)[MT], int cs, int c0, int nc, int i0,
                                        int i1, const WBatch<ULSPEC_GGML_F16, CMAX>& b, float4_t (&acc)[MT])
{
#pragma unroll
    for (int i = i0; i < i1; ++i)
        if (i < nc)
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
                    acc[mt] = mfma16x16x32(__builtin_bit_cast(half8_t, xs[xrow[mt] + cs * (c0 + i) + 4 * j]),
                                           __builtin_bit_cast(half8_t, b.w[i][j]), acc[mt]);
}

template <int TYPE, int CMAX, int MT>
__device__ __forceinline__ void stream_mma(const uint4* xs, const int (&xrow)[MT], int cs, int c0, int nc, int i0,
                                           int i1, const WBatch<TYPE, CMAX>& b, const NibbleConsts& nk,
                                           float4_t (&acc)[MT])
{
    if constexpr (TYPE == ULSPEC_GGML_F16)
        f16_mma<CMAX, MT>(xs, xrow, cs, c0, nc, i0, i1, b, acc);
    else if constexpr (TYPE == ULSPEC_GGML_Q8_0)
        q8_0_mma<CMAX, MT>(xs, xrow, cs, c0, nc, i0, i1, b, acc);
    else if constexpr (TYPE == ULSPEC_GGML_Q4_0)
        q4_0_mma<CMAX, MT>(xs, xrow, cs, c0, nc, i0, i1, b, nk, acc);
    else if constexpr (TYPE == ULSPEC_GGML_Q6_K)
        q6_k_mma<CMAX, MT>(xs, xrow, cs, c0, nc, i0, i1, b, nk, acc);
    else
        q4_k_mma<CMAX, MT>(xs, xrow, cs, c0, nc, i0, i1, b, (threadIdx.x & 63) >> 4, nk, acc);
}

// ---- row scale and epilogue --------------------------------------------------
// Row scale r_m = 1 / sqrt(sum_p pss[m][p] / K + eps) (RMSNorm,
// src/shaders/ffn/ffn_fused.glsl:23-33).  The GEMMs that follow a norm take X
// = split(h * w) from the producer of h and apply r_m to each output, which
// is x * W^T for x = (h * r) * w.  Lane l holds partials 4 l .. 4 l + 3 of the
// row (P <= 256); rs_reduce sums them ((a + b) + (c + d), then an xor tree).
constexpr int kMaxPartials = 256;

__device__ __forceinline__ float4 rs_load(const GemmArgs& a, int m)
{
    const GemmFuse& f = a.f;
    const __amdgpu_buffer_rsrc_t pr = make_rsrc(f.rs_pss, (uint32_t)a.M * (uint32_t)f.rs_P * 4u);
    const int p0 = 4 * (threadIdx.x & 63);
    return __builtin_bit_cast(float4, buf_load16(pr, m < a.M && p0 < f.rs_P ? (uint32_t)(m * f.rs_P + p0) * 4u : kOOB));
}

__device__ __forceinline__ float rs_reduce(const GemmArgs& a, float4 v)
{
    const int p0 = 4 * (threadIdx.x & 63), P = a.f.rs_P;
    float ss = ((p0 < P ? v.x : 0.0f) + (p0 + 1 < P ? v.y : 0.0f)) + ((p0 + 2 < P ? v.z : 0.0f) + (p0 + 3 < P ? v.w : 0.0f));
    ss += xor_lane<32>(ss);
    ss += xor_lane<16>(ss);
    ss += xor_lane<8>(ss);
    ss += xor_lane<4>(ss);
    ss += xor_lane<2>(ss);
    ss += xor_lane<1>(ss);
    return 1.0f / __builtin_sqrtf(ss / (float)a.K + a.f.rs_eps);
}

// First position of each sequence's rows for the RoPE epilogue: scalar
// loads through the constant address space (the values are fixed for the
// whole kernel), so they never wait behind the vector loads in flight.
// (Named fields, not an array: the positions stay in registers.)
static_assert(kMaxSeqs == 8, "EpiPos holds 8 sequences");
struct EpiPos {
    int p0, p1, p2, p3, p4, p5, p6, p7;
};

__device__ __forceinline__ EpiPos epi_pos0(const GemmArgs& a)
{
    EpiPos r{0, 0, 0, 0, 0, 0, 0, 0};
    if (a.f.epi != kEpiRope) return r;
    const __attribute__((address_space(4))) int32_t* p = (const __attribute__((address_space(4))) int32_t*)a.f.pos_dev;
    const int n = a.f.nseq, add = a.f.pos_add;
    r.p0 = p[0] + add;
    if (n > 1) {
        r.p1 = p[1] + add;
        r.p2 = n > 2 ? p[2] + add : 0;
        r.p3 = n > 3 ? p[3] + add : 0;
        r.p4 = n > 4 ? p[4] + add : 0;
        r.p5 = n > 5 ? p[5] + add : 0;
        r.p6 = n > 6 ? p[6] + add : 0;
        r.p7 = n > 7 ? p[7] + add : 0;
    }
    return r;
}

// Sequence of row m (rows are grouped by sequence, seq_rows each) and the
// row's index j within it.
__device__ __forceinline__ int row_seq(const GemmFuse& f, int m, int& j)
{
    const int b = f.nseq > 1 ? m / f.seq_rows : 0;
    j = m - b * f.seq_rows;
    return b;
}

__device__ __forceinline__ int seq_pos0(EpiPos ps, int b)
{
    int v = ps.p0;
    v = b == 1 ? ps.p1 : v;
    v = b == 2 ? ps.p2 : v;
    v = b == 3 ? ps.p3 : v;
    v = b == 4 ? ps.p4 : v;
    v = b == 5 ? ps.p5 : v;
    v = b == 6 ? ps.p6 : v;
    v = b == 7 ? ps.p7 : v;
    return v;
}

// RoPE position of row m: its sequence's first position plus j, or plus the
// row's tree depth.
__device__ __forceinline__ int rope_pos(const GemmFuse& f, EpiPos ps, int m)
{
    int j;
    const int b = row_seq(f, m, j);
    return seq_pos0(ps, b) + (f.tree ? (int)((f.row_depth >> (4 * (j & 15))) & 15u) : j);
}

// K / V cache row of row m: slot first position + j of its sequence's cache.
__device__ __forceinline__ size_t kv_row(const GemmFuse& f, EpiPos ps, int m)
{
    int j;
    const int b = row_seq(f, m, j);
    return (size_t)(f.seq0 + b) * f.seq_slots + (size_t)(seq_pos0(ps, b) + j);
}

// The memory operands of the epilogue of output (m, n), loaded ahead of it
// with the weights so that the epilogue reads no memory (vmcnt retires in
// issue order: a load issued in the epilogue would wait for every weight load
// in flight).  Two 4-byte loads for the resid and rope epilogues (out of range
// where a thread has no output), none otherwise:
//   resid: (h[m][n], xn_w[n])   rope: (cos, sin) of the pair at the row's
//                               RoPE position (rope_pos)
// Split in two: epi_addr (the buffer descriptors and the offsets, most of the
// address arithmetic) and epi_issue (the loads), so that a wave without an
// output slot skips the arithmetic while every wave still issues the same
// number of loads (the vmcnt waits count them).
struct EpiAddr {
    __amdgpu_buffer_rsrc_t r0, r1;
    uint32_t o0, o1;
};

// Descriptors of the epilogue's operands, offsets out of range (no output).
__device__ __forceinline__ EpiAddr epi_none(const GemmArgs& a)
{
    const GemmFuse& f = a.f;
    EpiAddr e;
    if (f.epi == kEpiResid) {
        e.r0 = make_rsrc(f.h, (uint32_t)a.M * (uint32_t)a.N * 4u);
        e.r1 = make_rsrc(f.xn_w, f.xn ? (uint32_t)a.N * 4u : 0u);
    } else if (f.epi == kEpiRope) {
        e.r0 = make_rsrc(f.rope, (uint32_t)min((uint64_t)f.rope_rows * (uint64_t)(f.hd / 2) * 8u, (uint64_t)0xffffffffu));
        e.r1 = e.r0;
    } else {
        e.r0 = e.r1 = make_rsrc(a.out, 0u);
    }
    e.o0 = e.o1 = kOOB;
    return e;
}

// The offsets of output (m, n)'s operands into e (out of range where the
// thread has no output).
__device__ __forceinline__ void epi_offsets(const GemmArgs& a, int m, int n, EpiPos pos0, EpiAddr& e)
{
    const GemmFuse& f = a.f;
    const bool ok = m < a.M && n < a.N;
    if (!ok) return;
    if (f.epi == kEpiResid) {
        e.o0 = (uint32_t)(m * a.N + n) * 4u;
        e.o1 = (uint32_t)n * 4u;
    } else if (f.epi == kEpiRope && n < f.qdim + f.kvdim) {
        const int nn = n < f.qdim ? n : n - f.qdim;
        e.o0 = (uint32_t)(rope_pos(f, pos0, m) * (f.hd / 2) + (nn % f.hd) / 2) * 8u;
        e.o1 = e.o0 + 4u;
    }
}

__device__ __forceinline__ float2 epi_issue(const GemmArgs& a, const EpiAddr& e)
{
    float2 v = {0.f, 0.f};
    if (a.f.epi == kEpiResid || a.f.epi == kEpiRope) {
        v.x = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(e.r0, e.o0, 0, 0));
        v.y = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(e.r1, e.o1, 0, 0));
    }
    return v;
}

__device__ __forceinline__ float2 epi_load(const GemmArgs& a, int m, int n, EpiPos pos0)
{
    EpiAddr e = epi_none(a);
    epi_offsets(a, m, n, pos0, e);
    return epi_issue(a, e);
}

// epi_load for the threads of tile slot j (wave-uniform): slots past the
// iteration's tiles skip the address arithmetic and issue out-of-range loads.
__device__ __forceinline__ float2 epi_load_slot(const GemmArgs& a, int j, int tpi, int m, int n, EpiPos pos0)
{
    EpiAddr e = epi_none(a);
    if (__builtin_amdgcn_readfirstlane(j) < tpi) epi_offsets(a, m, n, pos0, e);
    return epi_issue(a, e);
}

// Vector loads epi_load issues (wave-uniform).
__device__ __forceinline__ int epi_nloads(const GemmArgs& a)
{
    return a.f.epi == kEpiResid || a.f.epi == kEpiRope ? 2 : 0;
}

// Epilogue of output (m, n) of tile t, value s (already row-scaled); pre from
// epi_load, pos0 from epi_pos0.  Lanes l and l ^ 1 hold columns n and n ^ 1
// of the same row m, and 16-lane groups one row of one tile (whole waves call
// this).
//   store: Y[m][n] = s
//   rope:  RoPE pair (n, n+1) at the row's position (rope_pos: its sequence's
//          first position + j, or + depth(j) for a tree; Q and K rows, angles
//          from epi_load), then fp16 Q -> q16[m][n], K -> kc[row][n - qdim],
//          V -> vc[row][n - qdim - kvdim], row = kv_row(m)
//          (y0 = x0 c - x1 s, y1 = x0 s + x1 c; src/shaders/rope.glsl:50-73)
//   silu:  rows interleaved (2i = gate i, 2i+1 = up i): a = g * (1 / (1 +
//          e^-g)) * u, split: act[m][i] = hi, act[M + m][i] = lo
//   resid: h[m][n] += s (in place); pss[m][t] = sum over the tile's 16 columns
//          of h^2 (xor tree over the 16 lanes), the RMSNorm partial of row m;
//          with xn, the next GEMM's split X: xn[m][n] = hi, xn[xn_lo + m][n] =
//          lo of h * xn_w[n] (the next norm's weights)
__device__ __forceinline__ void epilogue(const GemmArgs& a, float s, int m, int n, int t, int l, float2 pre,
                                         EpiPos pos0)
{
    const bool ok = m < a.M && n < a.N;
    const GemmFuse& f = a.f;
    switch (f.epi) {
    case kEpiRope: {
        const float other = xor_lane<1>(s);
        if (!ok) break;
        const bool odd = n & 1;
        const size_t pos = kv_row(f, pos0, m);
        if (n < f.qdim + f.kvdim) {
            const int nn = n < f.qdim ? n : n - f.qdim;
            const float2 cs = pre;
            const float x0 = odd ? other : s, x1 = odd ? s : other;
            float y;
            if (!odd) {
                const float p0 = x0 * cs.x, p1 = x1 * cs.y;
                y = p0 - p1;
            } else {
                const float p0 = x0 * cs.y, p1 = x1 * cs.x;
                y = p0 + p1;
            }
            if (n < f.qdim) f.q16[(size_t)m * f.qdim + nn] = (_Float16)y;
            else f.kc[(size_t)pos * f.kvdim + nn] = (_Float16)y;
        } else {
            f.vc[(size_t)pos * f.kvdim + (n - f.qdim - f.kvdim)] = (_Float16)s;
        }
        break;
    }
    case kEpiSilu: {
        const float u = xor_lane<1>(s);
        if (ok && !(n & 1)) {
            const float sg = s * (1.0f / (1.0f + det_expf(-s)));
            _Float16 hi, lo;
            split_hl(sg * u, hi, lo);
            f.act[(size_t)m * (a.N / 2) + n / 2] = hi;
            f.act[(size_t)(a.M + m) * (a.N / 2) + n / 2] = lo;
        }
        break;
    }
    case kEpiResid: {
        float v = 0.0f;
        if (ok) {
            v = pre.x + s;
            f.h[(size_t)m * a.N + n] = v;
            if (f.xn) {
                _Float16 hi, lo;
                split_hl(v * pre.y, hi, lo);
                f.xn[(size_t)m * a.N + n] = hi;
                f.xn[(size_t)(f.xn_lo + m) * a.N + n] = lo;
            }
        }
        float sq = v * v;
        sq += xor_lane<1>(sq);
        sq += xor_lane<2>(sq);
        sq += xor_lane<4>(sq);
        sq += xor_lane<8>(sq);
        if (m < a.M && t < a.n_tiles && (l & 15) == 0) f.pss_out[(size_t)m * a.n_tiles + t] = sq;
        break;
    }
    default:
        if (ok) a.out[(size_t)m * a.N + n] = s;
    }
}

// ---- split-K kernels (any M) --------------------------------------------------
// Grid (row groups of kWaves 16-row tiles, K slices).  Wave w of a workgroup
// owns tile blockIdx.x * kWaves + w over the slice's chunks.  Per batch of
// CMAX chunks: the batch's X from registers to LDS (XStage rows; Q4_K also
// the sub-block sums of X), barrier, dequantize + MFMA for the MT column
// tiles.  Double-buffered (slice_db): two LDS buffers, and the next batch's
// X and weight loads are issued before the multiply, so they fly behind it;
// otherwise a batch's loads are issued at its start.  Each wave accumulates
// its chunks in K order and stores the slice's partial Y (high plus 2^-11
// low part for split X) to out[ks][M][N]; gemm_reduce_kernel sums the slices
// in slice order, so every output row is bitwise independent of M.
constexpr int kMaxSlices = 32;

// X slice of one batch in LDS: 16 MT rows of UB units (16 bytes = 8 halves)
// plus one pad unit (bank spread); UB is a power of two <= 128.  Thread tid
// stages unit tid % UB of rows tid / UB + pass * (1024 / UB).
template <int MT, int UB>
struct XStage {
    static constexpr int kUnitsPerRow = UB + 1;
    static constexpr int kRowsPerPass = kWaves * 64 / UB;
    static constexpr int kXU = (16 * MT + kRowsPerPass - 1) / kRowsPerPass;  // passes = units per thread
};

// Load this batch's X slice (staged rows < xrows, units [0, U) starting at
// element k0, U <= UB) into registers.  Units past K load 0.
template <int MT, int UB>
__device__ __forceinline__ void x_stage_load(const GemmArgs& a, __amdgpu_buffer_rsrc_t xr,
                                             uint4 (&xv)[XStage<MT, UB>::kXU], int k0, int U)
{
    using XS = XStage<MT, UB>;
    const int uu = threadIdx.x & (UB - 1), m0 = threadIdx.x / UB;
    const int k = k0 + 8 * uu;
#pragma unroll
    for (int u = 0; u < XS::kXU; ++u) {
        const int rho = m0 + u * XS::kRowsPerPass;
        const bool ok = rho < a.xrows && uu < U && k < a.K;
        xv[u] = buf_load16(xr, ok ? (uint32_t)(x_row(a, rho) * a.K + k) * 2u : kOOB);
    }
}

// lo_pad: units added to the LDS position of rows >= a.M (the low parts of
// split X; see slice_lo_pad).
template <int MT, int UB>
__device__ __forceinline__ void x_stage_store(const GemmArgs& a, uint4* xs, const uint4 (&xv)[XStage<MT, UB>::kXU],
                                              int U, int lo_pad)
{
    using XS = XStage<MT, UB>;
    const int uu = threadIdx.x & (UB - 1), m0 = threadIdx.x / UB;
#pragma unroll
    for (int u = 0; u < XS::kXU; ++u) {
        const int rho = m0 + u * XS::kRowsPerPass;
        if (rho < a.xrows && uu < U) xs[rho * XS::kUnitsPerRow + uu + (rho >= a.M ? lo_pad : 0)] = xv[u];
    }
}

// Q4_K staging: also each staged row's sub-block sums (32 elements = the 4
// lanes holding its units; rows and units past the data hold 0): s = the fp32
// sum, as fp16 hi = s / 32 and lo = (s / 32 - hi) 2^11 at half
// ((rho CMAX + chunk) 16 + 2 sub-block) of xsum (q4_k_mma_xs).
template <int MT, int CMAX>
__device__ __forceinline__ void x_stage_sums(_Float16* xsum, const uint4 (&xv)[XStage<MT, 32 * CMAX>::kXU])
{
    constexpr int UB = 32 * CMAX;
    using XS = XStage<MT, UB>;
    const int uu = threadIdx.x & (UB - 1), m0 = threadIdx.x / UB;
#pragma unroll
    for (int u = 0; u < XS::kXU; ++u) {
        const int rho = m0 + u * XS::kRowsPerPass;
        // the unit's 8 halves by dot products with (1, 1) (exact products,
        // fp32 sums), then the quad's 4 units by DPP lane swaps (xor 1, xor 2)
        const half2_t one2 = {(_Float16)1.0f, (_Float16)1.0f};
        float v = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, xv[u].x), one2, 0.0f, false);
        v = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, xv[u].y), one2, v, false);
        v = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, xv[u].z), one2, v, false);
        v = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, xv[u].w), one2, v, false);
        v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xb1, 0xf, 0xf, true));
        v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4e, 0xf, 0xf, true));
        if ((uu & 3) == 0 && rho < 16 * MT) {
            v *= 0.03125f;
            const _Float16 hi = (_Float16)v;
            const _Float16 lo = (_Float16)((v - (float)hi) * 2048.0f);
            const half2_t pr = {hi, lo};
            *(half2_t*)(xsum + (rho * CMAX + (uu >> 5)) * 16 + ((uu & 31) >> 2) * 2) = pr;
        }
    }
}

// The split-K kernel's LDS, in 16-byte units: the X buffer(s) (XStage rows,
// plus up to 15 units of lo_pad), then for Q4_K the sub-block sum buffer(s)
// (16 MT rows x CMAX chunks x 32 B).  Double-buffered (DB): two of each,
// batches alternating.
template <int TYPE, int MT, int CMAX>
constexpr int slice_buf_units()
{
    return 16 * MT * XStage<MT, kUnitsPerChunk<TYPE> * CMAX>::kUnitsPerRow + 16;
}

template <int TYPE, int MT, int CMAX>
constexpr int slice_sum_units()
{
    return TYPE == ULSPEC_GGML_Q4_K ? 16 * MT * CMAX * 2 : 0;
}

// Split X: the LDS rows of the low parts start lo_pad units later, so that
// low-part row M + i and high-part row i sit 32 banks apart (of 64 x 4 B)
// and the 16 A-operand slots of an MFMA (8 high, 8 low rows) read
// distinct banks: row rho starts at bank 4 RS rho mod 64, RS = 1 mod 16.
__device__ __forceinline__ int slice_lo_pad(const GemmArgs& a)
{
    return a.hl ? (8 - a.M % 16 + 16) % 16 : 0;
}

template <int TYPE, int MT, int CMAX, bool DB, bool HL>
__global__ __launch_bounds__(kWaves * 64) void gemm_slice_kernel(GemmArgs a)
{
    constexpr int UPC = kUnitsPerChunk<TYPE>;
    constexpr int UB = UPC * CMAX;
    constexpr bool kSums = TYPE == ULSPEC_GGML_Q4_K;
    using XS = XStage<MT, UB>;
    constexpr int XSZ = slice_buf_units<TYPE, MT, CMAX>(), SSZ = slice_sum_units<TYPE, MT, CMAX>();
    constexpr int NBUF = DB ? 2 : 1;
    extern __shared__ uint4 xsd[];  // [NBUF][XSZ] X, then [NBUF][SSZ] sums
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, g = lane >> 4;
    const int t = blockIdx.x * kWaves + wave;
    const bool live = t < a.n_tiles;
    const int tl = live ? t : a.n_tiles;  // past the last tile: loads move nothing
    const int ks = blockIdx.y;
    int ca, cb;
    slice_range(a, ks, ca, cb);
    const int nb = (cb - ca + CMAX - 1) / CMAX;
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.w, a.w_bytes);
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, x_bytes(a));
    // A-operand slot r of column tile mt reads staged row rho0 + step mt
    // (HL == a.hl): unclamped, so the tiles' LDS addresses differ by
    // constants; slots past the last row read rows of other slots, or stale
    // ones past a.xrows, and their outputs are never stored
    constexpr int kStep = HL ? 8 : 16;
    const int lo_pad = slice_lo_pad(a);
    const int rho0 = HL ? (r & 7) + (r < 8 ? 0 : a.M) : r;
    const int pad0 = HL && r >= 8 ? lo_pad : 0;
    int xrow[MT], srow[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        xrow[mt] = (rho0 + kStep * mt) * XS::kUnitsPerRow + pad0 + (kSuperBlock<TYPE> ? 8 * g : g);
        srow[mt] = (rho0 + kStep * mt) * CMAX * 4 + g;
    }
    const NibbleConsts nk = nibble_consts();
    float4_t acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = float4_t{0.f, 0.f, 0.f, 0.f};
    auto nc_of = [&](int bi) { return min(CMAX, cb - (ca + bi * CMAX)); };
    // batch bi's X from registers into buffer buf
    auto stage = [&](const uint4 (&xv)[XS::kXU], int bi, int buf) {
        x_stage_store<MT, UB>(a, xsd + buf * XSZ, xv, UPC * nc_of(bi), lo_pad);
        if constexpr (kSums) x_stage_sums<MT, CMAX>((_Float16*)(xsd + NBUF * XSZ + buf * SSZ), xv);
    };
    auto load = [&](uint4 (&xv)[XS::kXU], WBatch<TYPE, CMAX>& w, int bi) {
        const int c0 = ca + bi * CMAX, nc = nc_of(bi);
        x_stage_load<MT, UB>(a, xr, xv, c0 * UPC * 8, UPC * nc);
        pin_loads();
        stream_load<TYPE, CMAX>(a, wr, tl, c0, nc, w);
        pin_loads();
    };
    auto mma = [&](const WBatch<TYPE, CMAX>& w, int bi, int buf) {
        const int nc = live ? nc_of(bi) : 0;
        if constexpr (kSums)
            q4_k_mma_xs<CMAX, MT>(xsd + buf * XSZ, (const uint2*)(xsd + NBUF * XSZ + buf * SSZ), xrow, srow, nc, w,
                                  g, nk, acc);
        else
            stream_mma<TYPE, CMAX, MT>(xsd + buf * XSZ, xrow, UPC, 0, nc, 0, CMAX, w, nk, acc);
    };
    uint4 xv[XS::kXU];
    if constexpr (DB) {
        // batch bi: its X (registers) to buffer bi & 1, barrier (every wave is
        // past the multiply of batch bi - 2, which read that buffer), batch
        // bi + 1's loads issued, batch bi multiplied -- two batches per pass,
        // so the weight registers alternate statically
        WBatch<TYPE, CMAX> w0, w1;
        if (nb > 0) load(xv, w0, 0);
        for (int bi = 0; bi < nb; bi += 2) {
            stage(xv, bi, 0);
            __syncthreads();
            if (bi + 1 < nb) load(xv, w1, bi + 1);
            mma(w0, bi, 0);
            if (bi + 1 < nb) {
                stage(xv, bi + 1, 1);
                __syncthreads();
                if (bi + 2 < nb) load(xv, w0, bi + 2);
                mma(w1, bi + 1, 1);
            }
        }
    } else {
        // per batch: X and weight loads, barrier (the previous batch is done
        // reading the buffer), X to LDS, barrier, multiply
        for (int bi = 0; bi < nb; ++bi) {
            WBatch<TYPE, CMAX> w;
            load(xv, w, bi);
            if (bi) __syncthreads();
            stage(xv, bi, 0);
            __syncthreads();
            mma(w, bi, 0);
        }
    }
    if (!live) return;  // wave-uniform
    float* out = a.out + (size_t)ks * a.M * a.N;
    const int n = 16 * t + r;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float v = acc[mt][i];
            if (a.hl) v = v + xor_lane<32>(v) * kLoUnscale;  // lanes 0-31: + their low-part slot
            const int m = acc_row(a, mt, lane, i);
            if (m >= 0 && m < a.M && n < a.N) out[(size_t)m * a.N + n] = v;
        }
}

// Y[m][n] = the sum of the ks_count (<= KB) slices of part in slice order,
// times the row scale (if any), then the epilogue of output (m, n) (a.out is
// Y for the store epilogue).  Grid (16 n_tiles / 256, M / RPT): thread tid
// of workgroup (bx, by) takes padded column n = 256 bx + tid of rows RPT by
// .. RPT by + RPT - 1, all their slice loads issued at once; a 16-lane group
// is one row of one tile (the epilogue's lane pairs and xor tree); wave w
// computes the scale of the workgroup's row w.  RPT = 4 for large outputs
// (fewer workgroups, each with more loads in flight), 1 where that would
// leave too few workgroups.
template <int KB, int RPT>
__global__ __launch_bounds__(256) void gemm_reduce_kernel(GemmArgs a, const float* __restrict__ part)
{
    static_assert(RPT <= 256 / 64, "one wave per row scale");
    __shared__ float rs[RPT];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = blockIdx.x * 256 + threadIdx.x;
    const int m0 = blockIdx.y * RPT;
    const EpiPos pos0 = epi_pos0(a);
    const size_t MN = (size_t)a.M * a.N;
    float v[RPT][KB];
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
        const int m = m0 + j;
        const bool ok = m < a.M && n < a.N;
#pragma unroll
        for (int k = 0; k < KB; ++k) v[j][k] = ok && k < a.ks_count ? part[k * MN + (size_t)m * a.N + n] : 0.0f;
    }
    float2 pre[RPT];
#pragma unroll
    for (int j = 0; j < RPT; ++j) pre[j] = epi_load(a, m0 + j < a.M ? m0 + j : a.M, n, pos0);
    if (a.f.rs_pss) {
        if (wave < RPT && m0 + wave < a.M) {  // wave-uniform
            const float r = rs_reduce(a, rs_load(a, m0 + wave));
            if (lane == 0) rs[wave] = r;
        }
        __syncthreads();
    }
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
        const int m = m0 + j;
        float s = v[j][0];
#pragma unroll
        for (int k = 1; k < KB; ++k)
            if (k < a.ks_count) s += v[j][k];
        if (a.f.rs_pss && m < a.M) s *= rs[j];
        epilogue(a, s, m, n, n >> 4, lane, pre[j], pos0);
    }
}

// ---- whole-X kernels (small M) ------------------------------------------------
// The whole X sits in LDS for the workgroup's lifetime.  Per iteration the NW
// waves cover tpi = NW / P tiles x P parts of K (P a power of two, at most NW
// and at most the chunks per row); wave p owns chunks [ca, cb) of its tiles
// and the X of those chunks, which only it reads.  Each wave copies the X of
// its own chunks with direct buffer->LDS loads (the LDS side of one is 64
// consecutive units) before its weight loads and waits for those copies only
// (loads complete in issue order): no barrier before the first multiply.
// Parts are summed in part order in LDS, then the row scale and the epilogue
// run.  Two LDS layouts (XLayout), chosen per kernel by the length of a part:
//   chunk-major (parts of one chunk or short rows): unit c * CS + rho * RS + j
//     holds X[x_row(rho)][8 (UPC c + j) .. + 7], RS = UPC + 1 units per staged
//     row and chunk (the pad unit spreads the rows over the banks), CS =
//     xrows * RS per chunk -- a wave's X is one contiguous run, copied in full
//     64-unit loads whose sources each lane finds by dividing by CS and RS;
//   row-major (parts of at least 64 units per row): unit rho * RSTR + u holds
//     X[x_row(rho)][8 u .. 8 u + 7], RSTR = n_chunks UPC + 1 (odd: the 16 rows
//     of an A operand start in distinct bank groups) -- a wave's X is one run
//     per staged row on both sides, no division.
// Units past K read as 0.  The chunk-major size bounds both (the launch's LDS).
constexpr int kWideWaves = 16;

template <int TYPE>
constexpr int kRowStride = kUnitsPerChunk<TYPE> + 1;

struct XLayout {
    int row;    // units from one staged row to the next
    int chunk;  // units from one chunk of a row to the next
};

template <int TYPE, bool RM>
__device__ __forceinline__ XLayout x_layout(const GemmArgs& a)
{
    constexpr int UPC = kUnitsPerChunk<TYPE>;
    if constexpr (RM) return XLayout{a.n_chunks * UPC + 1, UPC};
    else return XLayout{kRowStride<TYPE>, a.xrows * kRowStride<TYPE>};
}

// Row-major for parts of CMAX chunks that fill a 64-unit load per row.
template <int TYPE, int CMAX>
constexpr bool kXRowMajor = CMAX * kUnitsPerChunk<TYPE> >= 64;

// This wave's X: chunks [ca, cb) of every staged row into their LDS places.
template <int TYPE, bool RM>
__device__ __forceinline__ void x_copy_region(const GemmArgs& a, __amdgpu_buffer_rsrc_t xr, uint8_t* xs_bytes, int ca,
                                              int cb, XLayout L)
{
    constexpr int UPC = kUnitsPerChunk<TYPE>, RS = kRowStride<TYPE>;
    const int lane = threadIdx.x & 63;
    const int KU = a.K / 8;
    if constexpr (RM) {  // one run of (cb - ca) UPC units per staged row
        const int k0 = ca * UPC, k1 = cb * UPC;
        for (int rho = 0; rho < a.xrows; ++rho) {
            const uint32_t grow = (uint32_t)x_row(a, rho) * (uint32_t)KU;
            for (int q = k0; q < k1; q += 64) {
                const int ku = q + lane;
                const uint32_t off = ku < KU ? (grow + (uint32_t)ku) * 16u : kOOB;
                if (ku < k1)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(
                        xr, (__attribute__((address_space(3))) void*)(xs_bytes + (size_t)(rho * L.row + q) * 16), 16,
                        off, 0, 0, 0);
            }
        }
    } else {  // one contiguous run of (cb - ca) CS units (the pad units load nothing)
        const int CS = L.chunk;
        const int u0 = ca * CS, u1 = cb * CS;
        const float inv_cs = 1.0f / (float)CS;
        for (int q = u0; q < u1; q += 64) {
            const int u = q + lane;
            int c = (int)((float)u * inv_cs);  // u / CS, corrected below (u < 2^22)
            if (c * CS > u) --c;
            if ((c + 1) * CS <= u) ++c;
            const int rem = u - c * CS;
            const int rho = rem / RS, j = rem - rho * RS;
            const int ku = c * UPC + j;
            const uint32_t off =
                j < UPC && ku < KU && rho < a.xrows ? (uint32_t)(x_row(a, rho) * KU + ku) * 16u : kOOB;
            if (u < u1)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    xr, (__attribute__((address_space(3))) void*)(xs_bytes + (size_t)q * 16), 16, off, 0, 0, 0);
        }
    }
}

// Output row the epilogue thread (lane l, accumulator row `row`) of a
// whole-X kernel handles: 4 (l / 16) + row; with split X the lanes 32-63 (the
// low-part slots) handle none (M).
__device__ __forceinline__ int epi_row(const GemmArgs& a, int l, int row)
{
    return a.hl && l >= 32 ? a.M : 4 * (l >> 4) + row;
}

// Sum of the P part sums of tile slot j in LDS, in part order; with split X
// the high-part sum (lane l) plus 2^-11 times the low-part sum (lane l ^ 32).
// All 2P reads are issued before the first add (one LDS round trip; a loop
// over a run-time P waited on each read).
template <int P>
__device__ __forceinline__ float red_sum(const GemmArgs& a, const float* red, int j, int row, int l)
{
    const float* b = red + (j * P * 4 + row) * 64;
    float hv[P], lv[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
        hv[p] = b[p * 256 + l];
        lv[p] = b[p * 256 + (l ^ 32)];
    }
    float s = hv[0], t = lv[0];
#pragma unroll
    for (int p = 1; p < P; ++p) {
        s += hv[p];
        t += lv[p];
    }
    return a.hl ? s + t * kLoUnscale : s;
}

// Row scales of rows wave, wave + NW, ... (every row of a whole-X kernel, at
// most 16) into rs (LDS), from loads issued by the same wave before its X and
// weights.
template <int NW>
constexpr int kRsIters = (16 + NW - 1) / NW;

template <int NW>
__device__ __forceinline__ void rs_finish(const GemmArgs& a, const float4 (&ps)[kRsIters<NW>], float* rs)
{
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < kRsIters<NW>; ++i) {
        const int m = wave + NW * i;
        if (m < a.M) {  // wave-uniform
            const float r = rs_reduce(a, ps[i]);
            if (lane == 0) rs[m] = r;
        }
    }
}

template <int NW>
__device__ __forceinline__ void rs_issue(const GemmArgs& a, float4 (&ps)[kRsIters<NW>])
{
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
    for (int i = 0; i < kRsIters<NW>; ++i)
        if (wave + NW * i < a.M) ps[i] = rs_load(a, wave + NW * i);
}

// One iteration per workgroup (tiles <= what the grid holds at once).
template <int TYPE, int CMAX, int NW>
__global__ __launch_bounds__(NW * 64) void gemm_stream_kernel(GemmArgs a)
{
    static_assert(NW >= 4 && NW % 4 == 0, "the reduction and epilogue take 256-thread tile slots");
    extern __shared__ uint4 xs[];
    __shared__ float red[NW * 4 * 64];
    __shared__ float rs[16];
    constexpr int NWL = WBatch<TYPE, CMAX>::kLoadsPerChunk;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, g = lane >> 4;
    // every launch splits K into NW parts (ks_count == NW): one tile per
    // workgroup, part p = wave
    constexpr int P = NW, tpi = 1;
    const int tw = 0, p = wave;
    const int ca = p * a.ks_q + min(p, a.ks_r);
    const int cb = ca + a.ks_q + (p < a.ks_r ? 1 : 0);
    const int nc0 = max(0, min(CMAX, cb - ca));
    constexpr bool RM = kXRowMajor<TYPE, CMAX>;
    const XLayout L = x_layout<TYPE, RM>(a);
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.w, a.w_bytes);
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, x_bytes(a));
    const int xrow[1] = {xslot_row(a, 0, r) * L.row + (kSuperBlock<TYPE> ? 8 * g : g)};
    const NibbleConsts nk = nibble_consts();
    const EpiPos pos0 = epi_pos0(a);
    const int it = blockIdx.x, t = it * tpi + tw;

    // issue order: row-scale partials, this wave's X (its whole part), the
    // first batch of weights, the epilogue operands
    float4 ps[kRsIters<NW>];
    if (a.f.rs_pss) rs_issue<NW>(a, ps);
    x_copy_region<TYPE, RM>(a, xr, (uint8_t*)xs, ca, cb, L);
    pin_loads();
    WBatch<TYPE, CMAX> A;
    stream_load<TYPE, CMAX>(a, wr, t, ca, nc0, A);
    // the epilogue operands of this thread's output (tile slot j = tid / 256)
    const int j_epi = threadIdx.x >> 8;
    const float2 pre = epi_load_slot(a, j_epi, tpi, epi_row(a, lane, (threadIdx.x >> 6) & 3),
                                     16 * (it * tpi + j_epi) + (lane & 15), pos0);
    pin_loads();
    if (a.f.rs_pss) rs_finish<NW>(a, ps, rs);
    vm_wait_dyn(CMAX * NWL + epi_nloads(a));  // this wave's X copies, issued before its weights
    float4_t acc[1] = {{0.f, 0.f, 0.f, 0.f}};
    stream_mma<TYPE, CMAX, 1>(xs, xrow, L.chunk, ca, t < a.n_tiles ? nc0 : 0, 0, CMAX, A, nk, acc);
    for (int c0 = ca + CMAX; c0 < cb; c0 += CMAX) {  // the rest of a long part (not prefetched)
        const int nc = min(CMAX, cb - c0);
        stream_load<TYPE, CMAX>(a, wr, t, c0, nc, A);
        pin_loads();
        stream_mma<TYPE, CMAX, 1>(xs, xrow, L.chunk, c0, t < a.n_tiles ? nc : 0, 0, CMAX, A, nk, acc);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) red[(wave * 4 + i) * 64 + lane] = acc[0][i];
    __syncthreads();
    // 256 threads per tile slot, NW / 4 slots per pass
    const int row = (threadIdx.x >> 6) & 3, l = lane;
    for (int j = j_epi; j < tpi; j += NW / 4) {
        const int m = epi_row(a, l, row);
        const float rsm = rs[min(m, 15)];  // read beside the part sums (m <= 16)
        float s = red_sum<P>(a, red, j, row, l);
        const int tt = it * tpi + j;
        const int n = 16 * tt + (l & 15);
        if (a.f.rs_pss && m < a.M) s *= rsm;
        epilogue(a, s, m, n, tt, l, j == j_epi ? pre : epi_load(a, m, n, pos0), pos0);
    }
}

// ---- ring kernel (more tiles than CUs) ----------------------------------------
// One 16-wave workgroup per CU walks its iterations (tpi = 16 / P tiles x P
// parts each, as above) in groups of G: a ring of G register batches holds
// the weights of one group, the first group's issued (after the wave's X
// copies) before the first multiply, and each multiply refills its batch with
// the weights of the same slot of the next group, so a group of weight loads
// stays in flight behind the arithmetic.  Each iteration of a group writes its
// part sums to its own LDS buffer; after the group's G multiplies one barrier,
// and 256-thread slots sum and run the epilogue of all G tpi tiles together
// (a wave reaches its next multiply without waiting on each tile's
// reduction; a second barrier keeps the next group's part sums off the
// buffers until they have been read).
constexpr int kRingWaves = 16;

// The epilogue slots of a group: thread t takes slot t / 256 + 4 q of pass q;
// slot j is tile j % TPI of the group's iteration j / TPI.
template <int G, int TPI>
constexpr int kRingPasses = (G * TPI + 3) / 4;

// epi_load of this thread's output in pass q of the group starting at local
// iteration base (nothing when its slot is past the group's tiles).
template <int G, int TPI>
__device__ __forceinline__ float2 ring_epi_load(const GemmArgs& a, int base, int n_loc, int q, EpiPos pos0)
{
    const int l = threadIdx.x & 63, row = (threadIdx.x >> 6) & 3, j = (threadIdx.x >> 8) + 4 * q;
    const int g = j / TPI, jj = j - g * TPI, li = base + g;
    const int live = __builtin_amdgcn_readfirstlane(j < G * TPI && li < n_loc ? 1 : 0);
    const int it = (int)blockIdx.x + li * (int)gridDim.x;
    return epi_load_slot(a, live ? jj : TPI, TPI, epi_row(a, l, row), 16 * (it * TPI + jj) + (l & 15), pos0);
}

template <int TYPE, int C, int G, int TPI>
__global__ __launch_bounds__(kRingWaves * 64) void gemm_ring_kernel(GemmArgs a)
{
    extern __shared__ uint4 xs[];
    constexpr int NW = kRingWaves, P = NW / TPI, NP = kRingPasses<G, TPI>;
    __shared__ float red[G][NW * 4 * 64];
    __shared__ float rs[16];
    constexpr int NWL = WBatch<TYPE, C>::kLoadsPerChunk;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, g = lane >> 4;
    const int tw = wave / P, p = wave % P;
    const int ca = p * a.ks_q + min(p, a.ks_r);
    const int nc = a.ks_q + (p < a.ks_r ? 1 : 0);  // <= C (checked by the host)
    const int n_iter = (a.n_tiles + TPI - 1) / TPI;
    const int n_loc = (n_iter - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;
    constexpr bool RM = kXRowMajor<TYPE, C>;
    const XLayout L = x_layout<TYPE, RM>(a);
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.w, a.w_bytes);
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, x_bytes(a));
    const int xrow[1] = {xslot_row(a, 0, r) * L.row + (kSuperBlock<TYPE> ? 8 * g : g)};
    const NibbleConsts nk = nibble_consts();
    // tile of local iteration li for this wave (>= n_tiles: nothing to load or multiply)
    auto tile_of = [&](int li) { return li < n_loc ? ((int)blockIdx.x + li * (int)gridDim.x) * TPI + tw : a.n_tiles; };
    const EpiPos pos0 = epi_pos0(a);

    // issue order: row-scale partials, this wave's X, the first group's
    // weights, then its epilogue operands; a workgroup with more than one
    // group issues its first iteration's weights ahead of X (the first
    // multiply waits for both; the 7B gate/up at M = 6, 5-6 iterations per
    // workgroup: 17.8 -> 17.1 us, where the QKV's single group of 3 was
    // 0.2 us slower that way)
    float4 ps[kRsIters<NW>];
    if (a.f.rs_pss) rs_issue<NW>(a, ps);
    WBatch<TYPE, C> ring[G];
    const bool wfirst = n_loc > G;  // uniform over the workgroup
    if (wfirst) {
        stream_load<TYPE, C>(a, wr, tile_of(0), ca, nc, ring[0]);
        pin_loads();
    }
    x_copy_region<TYPE, RM>(a, xr, (uint8_t*)xs, ca, ca + nc, L);
    pin_loads();
    if (!wfirst) stream_load<TYPE, C>(a, wr, tile_of(0), ca, nc, ring[0]);
#pragma unroll
    for (int k = 1; k < G; ++k) stream_load<TYPE, C>(a, wr, tile_of(k), ca, nc, ring[k]);
    float2 pre[NP];
#pragma unroll
    for (int q = 0; q < NP; ++q) pre[q] = ring_epi_load<G, TPI>(a, 0, n_loc, q, pos0);
    pin_loads();
    if (a.f.rs_pss) rs_finish<NW>(a, ps, rs);
    vm_wait_dyn((wfirst ? G - 1 : G) * C * NWL + NP * epi_nloads(a));  // this wave's X copies
    const int row = (threadIdx.x >> 6) & 3;
    for (int base = 0; base < n_loc; base += G) {
#pragma unroll
        for (int k = 0; k < G; ++k) {
            const int t = tile_of(base + k);
            float4_t acc[1] = {{0.f, 0.f, 0.f, 0.f}};
            stream_mma<TYPE, C, 1>(xs, xrow, L.chunk, ca, t < a.n_tiles ? nc : 0, 0, C, ring[k], nk, acc);
            stream_load<TYPE, C>(a, wr, tile_of(base + G + k), ca, nc, ring[k]);
            pin_loads();
#pragma unroll
            for (int i = 0; i < 4; ++i) red[k][(wave * 4 + i) * 64 + lane] = acc[0][i];
        }
        lds_barrier();
#pragma unroll
        for (int q = 0; q < NP; ++q) {
            const int j = (threadIdx.x >> 8) + 4 * q;
            if (j < G * TPI) {
                const int gk = j / TPI, jj = j - gk * TPI, li = base + gk;
                if (li < n_loc) {
                    const int m = epi_row(a, lane, row);
                    const float rsm = rs[min(m, 15)];  // read beside the part sums (m <= 16)
                    float s = red_sum<P>(a, red[gk], jj, row, lane);
                    const int tt = ((int)blockIdx.x + li * (int)gridDim.x) * TPI + jj;
                    if (a.f.rs_pss && m < a.M) s *= rsm;
                    epilogue(a, s, m, 16 * tt + (lane & 15), tt, lane, pre[q], pos0);
                }
            }
        }
        if (base + G < n_loc) {
            // the next group's epilogue operands (behind its weights), then
            // the barrier before its part sums reuse red
#pragma unroll
            for (int q = 0; q < NP; ++q) pre[q] = ring_epi_load<G, TPI>(a, base + G, n_loc, q, pos0);
            pin_loads();
            lds_barrier();
        }
    }
}

// Double-buffered split-K kernel (the next batch's weights and X in flight
// during a multiply) where it fits the 128 registers of 4 waves per SIMD: not
// for the super-block types past 4 (Q4_K) or 2 (Q6_K) column tiles.
template <int TYPE, int MT>
constexpr bool slice_db()
{
    return TYPE == ULSPEC_GGML_Q6_K ? MT <= 2 : TYPE == ULSPEC_GGML_Q4_K ? MT <= 4 : true;
}

// Chunks per batch of the split-K kernel: weight registers per lane (Q4_0 6
// per chunk, Q4_K 12, Q6_K 14, Q8_0 10, F16 16) times the batches in flight
// (two when double-buffered) at about 32-48 up to two column tiles, fewer
// beyond; a batch covers at most 1024 K (128 X units).
template <int TYPE, int MT>
constexpr int slice_cmax()
{
    return TYPE == ULSPEC_GGML_Q4_0 ? (MT <= 2 ? 4 : 2)
           : TYPE == ULSPEC_GGML_Q4_K ? (MT <= 2 ? 2 : 1)
           : TYPE == ULSPEC_GGML_Q6_K ? (MT <= 4 ? 2 : 1)
           : TYPE == ULSPEC_GGML_Q8_0 ? (MT <= 2 ? 4 : MT <= 4 ? 2 : 1)
                                       : (MT <= 2 ? 2 : 1);
}

template <int TYPE, int MT>
constexpr size_t slice_lds_bytes()
{
    constexpr int C = slice_cmax<TYPE, MT>();
    return (slice_db<TYPE, MT>() ? 2 : 1) *
           (size_t)(slice_buf_units<TYPE, MT, C>() + slice_sum_units<TYPE, MT, C>()) * sizeof(uint4);
}

template <int TYPE, int MT, bool HL>
constexpr const void* slice_fn()
{
    return (const void*)gemm_slice_kernel<TYPE, MT, slice_cmax<TYPE, MT>(), slice_db<TYPE, MT>(), HL>;
}

template <int TYPE, int MT>
void slice_launch_mt(const GemmArgs& a, hipStream_t st)
{
    static_assert(slice_lds_bytes<TYPE, MT>() <= 160 * 1024, "split-K LDS");
    const dim3 grid((a.n_tiles + kWaves - 1) / kWaves, a.ks_count);
    constexpr size_t lds = slice_lds_bytes<TYPE, MT>();
    constexpr int C = slice_cmax<TYPE, MT>();
    constexpr bool DB = slice_db<TYPE, MT>();
    if (a.hl) hipLaunchKernelGGL((gemm_slice_kernel<TYPE, MT, C, DB, true>), grid, dim3(kWaves * 64), lds, st, a);
    else hipLaunchKernelGGL((gemm_slice_kernel<TYPE, MT, C, DB, false>), grid, dim3(kWaves * 64), lds, st, a);
}

template <int TYPE>
void slice_launch_t(const GemmArgs& a, int mt, hipStream_t st)
{
    switch (mt) {
    case 1: slice_launch_mt<TYPE, 1>(a, st); break;
    case 2: slice_launch_mt<TYPE, 2>(a, st); break;
    case 3: slice_launch_mt<TYPE, 3>(a, st); break;
    case 4: slice_launch_mt<TYPE, 4>(a, st); break;
    default: slice_launch_mt<TYPE, 6>(a, st); break;
    }
}

}  // namespace

namespace ulspec {

// LDS available to one workgroup on gfx950, and what each whole-X kernel
// keeps besides X (part sums and row scales).
constexpr size_t kWideLdsMax = 160 * 1024;
constexpr size_t stream_static(int nw) { return (size_t)nw * 4 * 64 * sizeof(float) + 16 * sizeof(float); }
constexpr size_t kStaticWide = stream_static(kWideWaves);
constexpr size_t kStaticSmall = stream_static(4);
constexpr size_t ring_static(int G)
{
    return (size_t)G * kRingWaves * 4 * 64 * sizeof(float) + 16 * sizeof(float);
}

// LDS bytes of the whole X of `rows` staged rows (the chunk-major layout, which
// bounds the row-major one).
size_t x_lds_bytes(const Weight& w, int rows)
{
    const size_t rs = (w.type == ULSPEC_GGML_Q4_K || w.type == ULSPEC_GGML_Q6_K ? 32 : 16) + 1;
    return (size_t)w.n_chunks * rows * rs * 16;
}

bool wide_fits(const Weight& w, int rows)
{
    return rows <= 16 && x_lds_bytes(w, rows) + kStaticWide <= kWideLdsMax;
}

// Batch sizes (chunks per wave) the one-tile-per-workgroup kernel is built
// for: a launch takes the smallest that holds a whole part, so no load slot
// is wasted on chunks past the part (longer parts loop over batches).
template <int... C>
struct CList {};
using WideQ40 = CList<1, 2, 3, 4, 6, 8>;
using WideQ4K = CList<1, 2, 3, 4>;
using WideQ6K = CList<1, 2, 3>;  // 14 VGPRs of weights per chunk
using WideF16 = CList<1, 2>;  // 16 VGPRs of weights per chunk
using WideQ80 = CList<1, 2, 3, 4, 6>;  // 10 VGPRs of weights per chunk

template <int TYPE>
struct GemmCfg;
template <>
struct GemmCfg<ULSPEC_GGML_Q4_0> {
    using Wide = WideQ40;
};
template <>
struct GemmCfg<ULSPEC_GGML_Q4_K> {
    using Wide = WideQ4K;
};
template <>
struct GemmCfg<ULSPEC_GGML_Q6_K> {
    using Wide = WideQ6K;
};
template <>
struct GemmCfg<ULSPEC_GGML_Q8_0> {
    using Wide = WideQ80;
};
template <>
struct GemmCfg<ULSPEC_GGML_F16> {
    using Wide = WideF16;
};

template <int TYPE, int... C>
void wide_kernels(CList<C...>, std::vector<const void*>& out)
{
    (out.push_back((const void*)gemm_stream_kernel<TYPE, C, kWideWaves>), ...);
}

// One tile per 4-wave workgroup, two chunks per wave: weights of at most 8
// chunks per row (Q4_K K <= 2048) with up to 4 tiles per CU, and with fewer
// tiles than CUs too.  The workgroups of one launch are all resident at
// once, so every CU works, where the ring kernel's 16-wave workgroups would
// leave CUs idle (384 tiles of 8 chunks: 192 of them).  With more tiles per
// CU the ring kernel, which copies X once per CU instead of once per tile, is
// faster.  (8 waves of one chunk each, and the 16-wave kernel, half of whose
// waves idle, below one tile per CU: the draft's O projection at M = 1 5.28
// -> 4.63 us, gate/up 7.47 -> 6.92 us, the 7B step 1.7 % faster.)
constexpr int kSmallWaves = 4;
constexpr int kSmallChunks = 2;  // per wave
constexpr int kSmallTilesPerCu = 4;

// Launch the one-tile kernel with the smallest batch >= cpp (the largest when none is).
template <int TYPE, int... C>
void wide_launch(CList<C...>, int cpp, dim3 grid, dim3 block, size_t lds, hipStream_t st, GemmArgs& a)
{
    constexpr int cs[] = {C...};
    int pick = cs[sizeof...(C) - 1];
    for (int c : cs)
        if (c >= cpp) {
            pick = c;
            break;
        }
    bool done = false;
    auto one = [&](auto cmax) {
        constexpr int CM = decltype(cmax)::value;
        if (done || CM != pick) return;
        done = true;
        hipLaunchKernelGGL((gemm_stream_kernel<TYPE, CM, kWideWaves>), grid, block, lds, st, a);
    };
    (one(std::integral_constant<int, C>{}), ...);
}

template <int TYPE, int C, int G>
void ring_kernels(std::vector<const void*>& out)
{
    out.push_back((const void*)gemm_ring_kernel<TYPE, C, G, 1>);
    out.push_back((const void*)gemm_ring_kernel<TYPE, C, G, 2>);
    out.push_back((const void*)gemm_ring_kernel<TYPE, C, G, 4>);
}

// The ring kernel for C chunks per part, groups of G, TPI = 16 / P tiles per
// iteration.
template <int TYPE, int C, int G>
void ring_launch(int tpi, dim3 grid, dim3 block, size_t lds, hipStream_t st, const GemmArgs& a)
{
    if (tpi == 1) hipLaunchKernelGGL((gemm_ring_kernel<TYPE, C, G, 1>), grid, block, lds, st, a);
    else if (tpi == 2) hipLaunchKernelGGL((gemm_ring_kernel<TYPE, C, G, 2>), grid, block, lds, st, a);
    else hipLaunchKernelGGL((gemm_ring_kernel<TYPE, C, G, 4>), grid, block, lds, st, a);
}

template <int TYPE, int... MT>
void slice_kernels(std::integer_sequence<int, MT...>, std::vector<const void*>& out)
{
    (out.push_back(slice_fn<TYPE, MT, true>()), ...);
    (out.push_back(slice_fn<TYPE, MT, false>()), ...);
}

template <int TYPE>
void type_kernels(std::vector<const void*>& wide, std::vector<const void*>& small, std::vector<const void*>& rings,
                  std::vector<const void*>& rings3, std::vector<const void*>& slices, std::vector<const void*>& mid8,
                  std::vector<const void*>& mid12)
{
    slice_kernels<TYPE>(std::integer_sequence<int, 1, 2, 3, 4, 6>{}, slices);
    wide_kernels<TYPE>(typename GemmCfg<TYPE>::Wide{}, wide);
    small.push_back((const void*)gemm_stream_kernel<TYPE, kSmallChunks, kSmallWaves>);
    mid8.push_back((const void*)gemm_stream_kernel<TYPE, 2, 8>);
    mid12.push_back((const void*)gemm_stream_kernel<TYPE, 2, 12>);
    ring_kernels<TYPE, 1, 2>(rings);
    ring_kernels<TYPE, 2, 2>(rings);
    rings3.push_back((const void*)gemm_ring_kernel<TYPE, 1, 3, 1>);
}

ulspec_status gemm_init(ulspec_ctx* ctx)
{
    std::vector<const void*> wide, small, rings, rings3, slices, mid8, mid12;
    type_kernels<ULSPEC_GGML_Q4_0>(wide, small, rings, rings3, slices, mid8, mid12);
    type_kernels<ULSPEC_GGML_Q4_K>(wide, small, rings, rings3, slices, mid8, mid12);
    type_kernels<ULSPEC_GGML_F16>(wide, small, rings, rings3, slices, mid8, mid12);
    type_kernels<ULSPEC_GGML_Q8_0>(wide, small, rings, rings3, slices, mid8, mid12);
    type_kernels<ULSPEC_GGML_Q6_K>(wide, small, rings, rings3, slices, mid8, mid12);
    const struct {
        const std::vector<const void*>* fns;
        size_t fixed;
    } groups[] = {{&wide, kStaticWide},       {&small, kStaticSmall},    {&rings, ring_static(2)},
                  {&rings3, ring_static(3)},    {&slices, 0},              {&mid8, stream_static(8)},
                  {&mid12, stream_static(12)}};
    // The launch checks add each group's static LDS to the dynamic size; the
    // opt-in must not let static + dynamic exceed the CU's 160 KB, so both
    // come from the compiled kernel's own static size.
    for (const auto& gr : groups)
        for (const void* f : *gr.fns) {
            hipFuncAttributes at{};
            hipError_t e = hipFuncGetAttributes(&at, f);
            if (e != hipSuccess) return hip_fail(ctx, e, "hipFuncGetAttributes(GEMM kernel)");
            if (at.sharedSizeBytes != gr.fixed)
                return fail(ctx, ULSPEC_EDEVICE, "GEMM kernel static LDS %zu B, launch checks assume %zu B",
                            (size_t)at.sharedSizeBytes, gr.fixed);
            e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    (int)(kWideLdsMax - at.sharedSizeBytes));
            if (e != hipSuccess) return hip_fail(ctx, e, "hipFuncSetAttribute(max dynamic LDS)");
        }
    return ULSPEC_OK;
}

// Launch a whole-X kernel if one fits; false when the split-K path must run.
// At most 8 chunks per row and up to 4 tiles per CU: the 4-wave one-tile
// kernel (below 8 staged rows, or while the ring would leave CUs idle).
// More tiles than CUs and at most two chunks per part: the ring kernel, one
// 16-wave workgroup per CU, P parts per tile (the largest power of two <=
// min(16, chunks per row), P >= 4), 16 / P tiles per iteration.  Otherwise,
// at most one tile per CU: one workgroup per tile, 8 or 12 waves of at most
// two chunks up to 24 chunks per row, else 16 waves (a wave with an empty
// part idles).
template <int TYPE>
bool stream_launch_t(ulspec_ctx* ctx, const Weight& w, GemmArgs& a)
{
    const int n_cu = std::max(1, ctx->n_cu);
    const bool pipe = (int)w.n_tiles > n_cu;
    const size_t lds = x_lds_bytes(w, a.xrows);
    hipStream_t st = ctx->stream;
    if (a.xrows > 16) return false;
    auto split = [&](int P) {
        a.ks_count = P;
        a.ks_q = (int)(w.n_chunks / P);
        a.ks_r = (int)(w.n_chunks % P);
    };
    // the ring: P parts per tile, 16 / P tiles per iteration
    int P = kRingWaves;
    while (P > 1 && (uint32_t)P > w.n_chunks) P >>= 1;
    const int cpp = (int)((w.n_chunks + P - 1) / P);
    const int ring_iters = ((int)w.n_tiles + kRingWaves / P - 1) / (kRingWaves / P);
    const bool ring_ok = pipe && P >= 4 && cpp <= 2 && lds + ring_static(2) <= kWideLdsMax;
    const bool small_ok = w.n_chunks <= (uint32_t)(kSmallWaves * kSmallChunks) &&
                          (int)w.n_tiles <= kSmallTilesPerCu * n_cu && lds + kStaticSmall <= kWideLdsMax;
    // the one-tile kernel stages the whole X per tile: from 8 staged rows on,
    // the ring (X once per CU) where its iterations cover every CU
    const bool small_x = a.xrows < 8 || ring_iters < n_cu;
    if (small_ok && (small_x || !ring_ok)) {
        split(kSmallWaves);  // at most kSmallChunks chunks per wave
        hipLaunchKernelGGL((gemm_stream_kernel<TYPE, kSmallChunks, kSmallWaves>), dim3(w.n_tiles),
                           dim3(kSmallWaves * 64), lds, st, a);
        return true;
    }
    if (pipe) {
        if (!ring_ok) return false;
        split(P);
        const int tpi = kRingWaves / P, n_iter = ((int)w.n_tiles + tpi - 1) / tpi;
        const dim3 grid(std::min(n_iter, n_cu)), block(kRingWaves * 64);
        // groups of 3 iterations for one-chunk parts of one tile per
        // iteration where their part sums fit beside X (the other shapes run
        // out of registers at 3), else groups of 2
        if (cpp <= 1 && tpi == 1 && lds + ring_static(3) <= kWideLdsMax)
            hipLaunchKernelGGL((gemm_ring_kernel<TYPE, 1, 3, 1>), grid, block, lds, st, a);
        else if (cpp <= 1) ring_launch<TYPE, 1, 2>(tpi, grid, block, lds, st, a);
        else ring_launch<TYPE, 2, 2>(tpi, grid, block, lds, st, a);
        return true;
    }
    if (lds + kStaticWide > kWideLdsMax) return false;
    // one tile per workgroup: up to 24 chunks 8 or 12 waves of at most two
    // (fewer idle waves than 16: the 7B O projection 7.58 -> 7.24 us, the
    // draft's down 6.74 -> 6.41 us at M = 2), past that 16 waves
    if (w.n_chunks <= 16) {
        split(8);
        hipLaunchKernelGGL((gemm_stream_kernel<TYPE, 2, 8>), dim3(w.n_tiles), dim3(8 * 64), lds, st, a);
        return true;
    }
    if (w.n_chunks <= 24) {
        split(12);
        hipLaunchKernelGGL((gemm_stream_kernel<TYPE, 2, 12>), dim3(w.n_tiles), dim3(12 * 64), lds, st, a);
        return true;
    }
    split(kWideWaves);
    wide_launch<TYPE>(typename GemmCfg<TYPE>::Wide{}, a.ks_q + (a.ks_r ? 1 : 0), dim3(w.n_tiles),
                      dim3(kWideWaves * 64), lds, st, a);
    return true;
}

bool stream_launch(ulspec_ctx* ctx, const Weight& w, GemmArgs& a)
{
    if (w.type == ULSPEC_GGML_Q4_0) return stream_launch_t<ULSPEC_GGML_Q4_0>(ctx, w, a);
    if (w.type == ULSPEC_GGML_Q4_K) return stream_launch_t<ULSPEC_GGML_Q4_K>(ctx, w, a);
    if (w.type == ULSPEC_GGML_Q6_K) return stream_launch_t<ULSPEC_GGML_Q6_K>(ctx, w, a);
    if (w.type == ULSPEC_GGML_Q8_0) return stream_launch_t<ULSPEC_GGML_Q8_0>(ctx, w, a);
    return stream_launch_t<ULSPEC_GGML_F16>(ctx, w, a);
}

// K slices per weight.  The split-K kernel runs one workgroup per CU at a
// time, so its time goes as (rounds of n_cu workgroups) x (a workgroup's
// start-up and partial store, about kSliceFixed chunks' worth, + the chunks
// of the longest slice); the fewest slices that minimise that (a round that
// spills a few workgroups over n_cu doubles the time).
constexpr uint32_t kSliceFixed = 3;

uint32_t choose_ksplit(uint32_t n_tiles, uint32_t n_chunks, int n_cu)
{
    const uint32_t groups = (n_tiles + kWaves - 1) / kWaves;
    const uint32_t cu = n_cu > 0 ? (uint32_t)n_cu : 1u;
    uint32_t best = 1;
    uint64_t best_cost = ~0ull;
    for (uint32_t ks = 1; ks <= n_chunks && ks <= (uint32_t)kMaxSlices; ++ks) {
        const uint64_t rounds = ((uint64_t)groups * ks + cu - 1) / cu;
        const uint64_t cost = rounds * (kSliceFixed + (n_chunks + ks - 1) / ks);
        if (cost < best_cost) {
            best = ks;
            best_cost = cost;
        }
    }
    return best;
}

size_t gemm_workspace_bytes(const Weight& w)
{
    return w.ksplit > 1 ? (size_t)w.ksplit * kGemmRowsH16 * w.n * sizeof(float) : 0;
}

namespace {

GemmArgs make_args(const Weight& w, const _Float16* x, uint32_t M, bool hl, uint32_t lo_rows, float* out)
{
    GemmArgs a;
    a.w = w.dev;
    a.w_bytes = (uint32_t)w.bytes;
    a.x = x;
    a.out = out;
    a.M = (int)M;
    a.N = (int)w.n;
    a.K = (int)w.k;
    a.n_tiles = (int)w.n_tiles;
    a.n_chunks = (int)w.n_chunks;
    a.ks_count = 1;
    a.ks_q = (int)w.n_chunks;
    a.ks_r = 0;
    a.hl = hl ? 1 : 0;
    a.lo_rows = hl ? (int)lo_rows : 0;
    a.xrows = hl ? 2 * (int)M : (int)M;
    a.f = GemmFuse();
    return a;
}

template <int KB>
void reduce_launch(const GemmArgs& a, const float* part, int cols, bool four_rows, hipStream_t st)
{
    if (four_rows)
        hipLaunchKernelGGL((gemm_reduce_kernel<KB, 4>), dim3(cols, (a.M + 3) / 4), dim3(256), 0, st, a, part);
    else
        hipLaunchKernelGGL((gemm_reduce_kernel<KB, 1>), dim3(cols, a.M), dim3(256), 0, st, a, part);
}

// The split-K kernel over a.M rows into part[ks][M][N], then the slice sum, row
// scale and a.f's epilogue into y (one slice, no row scale and a plain store:
// straight into y).
void split_launch(ulspec_ctx* ctx, const Weight& w, GemmArgs a, float* part, float* y)
{
    a.ks_count = (int)w.ksplit;
    a.ks_q = (int)(w.n_chunks / w.ksplit);
    a.ks_r = (int)(w.n_chunks % w.ksplit);
    const bool direct = w.ksplit == 1 && a.f.epi == kEpiStore && !a.f.rs_pss;
    a.out = direct ? y : part;
    const int mt = a.hl ? (a.M + 7) / 8 : (a.M + 15) / 16;
    if (w.type == ULSPEC_GGML_Q4_0) slice_launch_t<ULSPEC_GGML_Q4_0>(a, mt, ctx->stream);
    else if (w.type == ULSPEC_GGML_Q4_K) slice_launch_t<ULSPEC_GGML_Q4_K>(a, mt, ctx->stream);
    else if (w.type == ULSPEC_GGML_Q6_K) slice_launch_t<ULSPEC_GGML_Q6_K>(a, mt, ctx->stream);
    else if (w.type == ULSPEC_GGML_Q8_0) slice_launch_t<ULSPEC_GGML_Q8_0>(a, mt, ctx->stream);
    else slice_launch_t<ULSPEC_GGML_F16>(a, mt, ctx->stream);
    if (direct) return;
    a.out = y;
    const int cols = (16 * a.n_tiles + 255) / 256;
    const bool wide = cols * ((a.M + 3) / 4) >= 2 * std::max(1, ctx->n_cu);
    if (a.ks_count <= 2) reduce_launch<2>(a, part, cols, wide, ctx->stream);
    else if (a.ks_count <= 4) reduce_launch<4>(a, part, cols, wide, ctx->stream);
    else if (a.ks_count <= 8) reduce_launch<8>(a, part, cols, wide, ctx->stream);
    else if (a.ks_count <= 16) reduce_launch<16>(a, part, cols, wide, ctx->stream);
    else reduce_launch<kMaxSlices>(a, part, cols, wide, ctx->stream);
}

}  // namespace

// Launch the GEMM for one weight (fp16 X); rows beyond kGemmRowsH16 go in
// further launches.  Never allocates (the slice workspace is sized at upload).
ulspec_status gemm_launch(ulspec_ctx* ctx, const Weight& w, const uint16_t* x, uint32_t M, float* y)
{
    const _Float16* X = reinterpret_cast<const _Float16*>(x);
    if (gemm_workspace_bytes(w) > ctx->ws_bytes)
        return fail(ctx, ULSPEC_EINVAL, "verify_gemm: workspace smaller than the weight needs");
    for (uint32_t m0 = 0; m0 < M; m0 += kGemmRowsH16) {
        const uint32_t mc = std::min<uint32_t>(kGemmRowsH16, M - m0);
        GemmArgs a = make_args(w, X + (size_t)m0 * w.k, mc, false, 0, y + (size_t)m0 * w.n);
        if (stream_launch(ctx, w, a)) continue;  // whole X in LDS, parts summed in the kernel
        split_launch(ctx, w, a, (float*)ctx->ws, y + (size_t)m0 * w.n);
    }
    return check_launch(ctx, "verify_gemm launch");
}

size_t gemm_split_part_bytes(const Weight& w, uint32_t M)
{
    return (size_t)w.ksplit * M * w.n * sizeof(float);
}

ulspec_status gemm_fused(ulspec_ctx* ctx, const Weight& w, const GemmFuse& f, const uint16_t* x, uint32_t M,
                         uint32_t lo_rows, float* y)
{
    if (M == 0 || M > (uint32_t)kGemmRowsSplit || lo_rows < M)
        return fail(ctx, ULSPEC_EINVAL, "fused gemm: %u rows (1..%d), low parts at row %u", M, kGemmRowsSplit,
                    lo_rows);
    if (f.rs_pss && (f.rs_P < 1 || f.rs_P > kMaxPartials))
        return fail(ctx, ULSPEC_EINVAL, "fused gemm: the row scale needs 1..%d partial sums", kMaxPartials);
    GemmArgs a = make_args(w, reinterpret_cast<const _Float16*>(x), M, true, lo_rows, y);
    a.f = f;
    if (M <= 8 && stream_launch(ctx, w, a)) return check_launch(ctx, "fused gemm launch");
    float* part = f.part ? f.part : (float*)ctx->ws;
    const size_t room = f.part ? f.part_bytes : ctx->ws_bytes;
    if (gemm_split_part_bytes(w, M) > room)
        return fail(ctx, ULSPEC_EINVAL, "fused gemm: %zu bytes of slice partials, %zu available",
                    gemm_split_part_bytes(w, M), room);
    split_launch(ctx, w, a, part, y);
    return check_launch(ctx, "fused gemm launch");
}

}  // namespace ulspec

namespace ulspec {

// Rows of GGUF blocks (device memory) to fp16 rows out[out_row0 + r * step]
// (asynchronous on the context stream).
ulspec_status rows_to_f16(ulspec_ctx* ctx, uint32_t type, const void* raw, uint32_t rows, uint32_t K,
                          _Float16* out, uint32_t out_row0, uint32_t out_row_step)
{
    const int bs = ulspec_ggml_blck_size(type), ts = ulspec_ggml_type_size(type);
    const bool ok = type == ULSPEC_GGML_Q4_0 || type == ULSPEC_GGML_Q4_K || type == ULSPEC_GGML_F16 ||
                    type == ULSPEC_GGML_Q8_0 || type == ULSPEC_GGML_Q6_K;
    if (!ok || bs <= 0 || K % bs) return fail(ctx, ULSPEC_EUNSUPPORTED, "rows_to_f16: type %u, K=%u", type, K);
    const uint64_t elems = (uint64_t)rows * K;
    hipLaunchKernelGGL(dequant_rows_f16_kernel, dim3((unsigned)((elems + 255) / 256)), dim3(256), 0, ctx->stream,
                       (const uint8_t*)raw, out, type, K, (uint64_t)(K / bs) * ts, elems, out_row0, out_row_step);
    return check_launch(ctx, "rows_to_f16 launch");
}

// Re-tile raw GGUF blocks (host or device memory) into a new device weight.
ulspec_status weight_create(ulspec_ctx* ctx, uint32_t type, const void* blocks, size_t nbytes, uint32_t N, uint32_t K,
                            bool on_device, uint32_t* out_id)
{
    if (!blocks || !out_id) return fail(ctx, ULSPEC_EINVAL, "weight_upload: null pointer");
    const bool f16 = type == ULSPEC_GGML_F16;
    const bool q80 = type == ULSPEC_GGML_Q8_0;
    const bool sb = type == ULSPEC_GGML_Q4_K || type == ULSPEC_GGML_Q6_K;  // 256-element super-blocks
    if (type != ULSPEC_GGML_Q4_0 && !sb && !f16 && !q80)
        return fail(ctx, ULSPEC_EUNSUPPORTED, "weight_upload: ggml type %u not supported (Q4_0, Q4_K, Q6_K, Q8_0, F16)",
                    type);
    const int bs = ulspec_ggml_blck_size(type), ts = ulspec_ggml_type_size(type);
    // F16 rows too are taken in multiples of 32 (activation rows stay 64-byte aligned)
    const int k_mult = std::max(bs, 32);
    if (N == 0 || K == 0 || K % k_mult)
        return fail(ctx, ULSPEC_EINVAL, "weight_upload: K=%u must be a positive multiple of %d", K, k_mult);
    const size_t expect = (size_t)N * (K / bs) * ts;
    if (nbytes != expect) return fail(ctx, ULSPEC_EINVAL, "weight_upload: %zu bytes given, %zu expected", nbytes, expect);
    Weight w;
    w.type = type;
    w.src_type = type;
    w.n = N;
    w.k = K;
    w.n_tiles = (N + 15) / 16;
    w.n_chunks = sb ? K / 256 : (K + 127) / 128;
    w.bytes = (size_t)w.n_tiles * w.n_chunks *
              (f16 ? kF16Chunk : q80 ? kQ80Chunk : type == ULSPEC_GGML_Q4_0 ? kQ40Chunk
                                              : type == ULSPEC_GGML_Q6_K ? kQ6KChunk : kQ4KChunk);
    if (w.bytes >= kOOB) return fail(ctx, ULSPEC_EINVAL, "weight_upload: %zu bytes exceeds the 2 GiB per-weight limit", w.bytes);
    w.ksplit = choose_ksplit(w.n_tiles, w.n_chunks, ctx->n_cu);
    (void)hipSetDevice(ctx->device);
    hipError_t e = hipMalloc(&w.dev, w.bytes);
    if (e != hipSuccess) return hip_fail(ctx, e, "weight_upload hipMalloc");
    void* raw = nullptr;
    // workspace: the host blocks (when not on the device), then for the fp16
    // formats the fp16 rows
    const size_t raw_room = on_device ? 0 : (nbytes + 255) / 256 * 256;
    const size_t need = f16 ? raw_room + (size_t)N * K * 2 : std::max(raw_room, gemm_workspace_bytes(w));
    ulspec_status st = workspace(ctx, need, &raw);
    if (st != ULSPEC_OK) {
        (void)hipFree(w.dev);
        return st;
    }
    if (on_device) {
        raw = const_cast<void*>(blocks);
    } else {
        e = hipMemcpyAsync(raw, blocks, nbytes, hipMemcpyHostToDevice, ctx->stream);
        if (e != hipSuccess) {
            (void)hipFree(w.dev);
            return hip_fail(ctx, e, "weight_upload copy");
        }
    }
    if (f16) {
        // to fp16 rows (after the blocks in the workspace), then re-tiled
        _Float16* half_rows = (_Float16*)((uint8_t*)ctx->ws + raw_room);
        const uint64_t elems = (uint64_t)N * K;
        hipLaunchKernelGGL(dequant_rows_f16_kernel, dim3((unsigned)((elems + 255) / 256)), dim3(256), 0, ctx->stream,
                           (const uint8_t*)raw, half_rows, type, K, (uint64_t)(K / bs) * ts, elems, 0u, 1u);
        const uint64_t total = (uint64_t)w.n_tiles * w.n_chunks * 256;
        hipLaunchKernelGGL(repack_f16_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, ctx->stream,
                           (const _Float16*)half_rows, w.dev, N, K, w.n_chunks, total);
    } else if (q80) {
        const uint64_t total = (uint64_t)w.n_tiles * w.n_chunks * 256;
        hipLaunchKernelGGL(repack_q8_0_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, ctx->stream,
                           (const uint8_t*)raw, w.dev, N, K / 32, w.n_chunks, total);
    } else if (type == ULSPEC_GGML_Q4_0) {
        const uint64_t total = (uint64_t)w.n_tiles * w.n_chunks * 256;
        hipLaunchKernelGGL(repack_q4_0_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, ctx->stream,
                           (const uint8_t*)raw, w.dev, N, K / 32, w.n_chunks, total);
    } else {
        const uint64_t total = (uint64_t)w.n_tiles * w.n_chunks * 512;
        hipLaunchKernelGGL(type == ULSPEC_GGML_Q6_K ? repack_q6_k_kernel : repack_q4_k_kernel,
                           dim3((unsigned)((total + 255) / 256)), dim3(256), 0, ctx->stream, (const uint8_t*)raw,
                           w.dev, N, w.n_chunks, total);
    }
    st = check_launch(ctx, "weight repack launch");
    if (st == ULSPEC_OK) {
        e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) st = hip_fail(ctx, e, "weight_upload sync");
    }
    if (st != ULSPEC_OK) {
        (void)hipFree(w.dev);
        return st;
    }
    *out_id = (uint32_t)ctx->weights.size();
    ctx->weights.push_back(w);
    return ULSPEC_OK;
}

}  // namespace ulspec

extern "C" ulspec_status ulspec_weight_upload(ulspec_ctx* ctx, uint32_t type, const void* blocks, size_t nbytes,
                                              uint32_t N, uint32_t K, uint32_t* out_id)
{
    ULSPEC_CHECK_CTX(ctx);
    return weight_create(ctx, type, blocks, nbytes, N, K, false, out_id);
}

extern "C" ulspec_status ulspec_weight_info(ulspec_ctx* ctx, uint32_t id, uint32_t* type, uint32_t* n, uint32_t* k,
                                            size_t* bytes)
{
    ULSPEC_CHECK_CTX(ctx);
    if (id >= ctx->weights.size()) return fail(ctx, ULSPEC_EINVAL, "weight_info: no weight %u", id);
    const Weight& w = ctx->weights[id];
    if (type) *type = w.src_type;
    if (n) *n = w.n;
    if (k) *k = w.k;
    if (bytes) *bytes = w.bytes;
    return ULSPEC_OK;
}

extern "C" ulspec_status ulspec_verify_gemm(ulspec_ctx* ctx, uint32_t id, const uint16_t* x, uint32_t M, float* y)
{
    ULSPEC_CHECK_CTX(ctx);
    if (id >= ctx->weights.size()) return fail(ctx, ULSPEC_EINVAL, "verify_gemm: no weight %u", id);
    if (!x || !y) return fail(ctx, ULSPEC_EINVAL, "verify_gemm: null pointer");
    if (M == 0) return fail(ctx, ULSPEC_EINVAL, "verify_gemm: M must be >= 1");
    if (((uintptr_t)x & 15) != 0) return fail(ctx, ULSPEC_EINVAL, "verify_gemm: x must be 16-byte aligned");
    (void)hipSetDevice(ctx->device);
    return gemm_launch(ctx, ctx->weights[id], x, M, y);
}
