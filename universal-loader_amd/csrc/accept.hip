// accept.hip -- K3, acceptance sampling of k drafted tokens, and sampling of
// one token per row.
//
// Replaces SpeculativeDecoder::verify_speculation (first-match of token ids,
// src/inference/speculative_decoder.cpp:89-110) with the speculative-sampling
// rule (Leviathan, Kalman & Matias, ICML 2023, Alg. 1), and
// InferenceEngine::sample_token (src/inference/inference_engine.cpp:340-367)
// with seeded uniforms; its inverse-CDF convention (strict "<" on the running
// sum, fall back to the last index) is kept.
//
// Every decision uses exact arithmetic so that any reduction order gives the
// same tokens:
//   warp of a row: lmax = max l; e_i = det_expf((l_i - lmax) * invT) for the
//   kept tokens (all, or the top_k by (logit desc, index asc)); fixed point
//   E_i = trunc(e_i * 2^S), S = 63 - bitlen(V); Z = sum E_i in uint64 (exact,
//   order-free); top_p keeps the shortest (logit desc, index asc) prefix with
//   (double)cum >= (double)top_p * (double)Z.
//   accept x iff ((double)u * Q_x) * Zp < (double)P_x * Zq  (u q(x) < p(x)).
//   residual R_j = trunc(ldexp(max(0, P_j Zq - Q_j Zp), 62 - bitlen(Zp) -
//   bitlen(Zq))) in double; draw T = trunc(u * Z), first j with T < cumsum.
//
// Every logit row is split over up to 64 chunk workgroups (one workgroup
// reading a whole row is bound by what a single CU keeps in flight); integer
// weights make chunked sums and draws equal to a scan of the whole row.
//   full vocabulary / greedy: chunk maxima, chunk sums of E (and the last
//   nonzero index), a one-wave accept walk per sequence on the row totals,
//   the residual's chunk sums for a sequence that rejected, and a final draw
//   that scans only the chunk holding T;
//   top-k / top-p: per-chunk thread maxima, a radix-selected lower bound of
//   the k-th largest logit, candidate collection by the chunks, one
//   workgroup per row for the candidate sort and the kept list (sorted by
//   index), then decide (one workgroup per sequence, lists staged in LDS).
// Tree acceptance keeps one workgroup per row (row_stats) and per tree.
#include <type_traits>

#include "detmath.h"
#include "hip_common.h"
#include "ulspec_internal.h"

using namespace ulspec;

namespace {

constexpr int kKMax = 256;       // largest supported top_k
constexpr int kCandMax = 2048;   // candidate buffer of the fast top-k path
constexpr int kRankMax = 512;    // candidates ranked by counting (more: a bitonic sort)
constexpr int kMaxK = 16;        // draft tokens per sequence of one acceptance call
// decide_kernel's dynamic LDS: 2k + 1 lists of up to K entries (u64 weight, i32 token)
inline size_t decide_lds_bytes(uint32_t k, uint32_t K) { return (size_t)(2 * k + 1) * K * 12; }
constexpr int kRowThreads = 1024;
constexpr int kSeqThreads = 1024;
constexpr int kRound = 8;         // float4 rounds in flight per thread in the vocabulary scans
constexpr int kMaxRounds = 256;   // rounds of the CDF draw: V <= 256 * 4 * kSeqThreads

struct RowStat {
    uint64_t Z;
    uint64_t kmin;  // top-p bound in full-vocabulary mode: tokens with a smaller order_key weigh 0
    float lmax;
    int32_t argmax;
    int32_t nk;  // kept tokens; == V in full-vocabulary mode (list unused)
    int32_t pad;
    int32_t idx[kKMax];  // kept token ids, ascending
    uint64_t E[kKMax];
};

struct WarpParams {
    float invT;
    uint32_t top_k;  // 0: full vocabulary
    float top_p;
    int32_t greedy;
    float scale;     // 2^S
    int32_t pad;
};

// top_k modes: a kept list of at most kKMax entries (list_topk), or, for
// larger k, the full-vocabulary kernels with a per-row bound (bound_topk):
// the order key of the k-th token, below which every weight is 0.
__host__ __device__ __forceinline__ bool list_topk(const WarpParams& p, uint32_t V)
{
    return p.top_k > 0 && p.top_k < V && p.top_k <= (uint32_t)kKMax;
}
__host__ __device__ __forceinline__ bool bound_topk(const WarpParams& p, uint32_t V)
{
    return p.top_k > (uint32_t)kKMax && p.top_k < V;
}
// Full-vocabulary rows that need a per-row bound (kmin): top-p, or a large top_k.
__host__ __device__ __forceinline__ bool row_bound(const WarpParams& p, uint32_t V)
{
    return !p.greedy && !list_topk(p, V) && (p.top_p < 1.0f || bound_topk(p, V));
}

// ---- wave scans over DPP lane moves ---------------------------------------------
// Inclusive prefix (max or sum) over the 64 lanes of a fully active wave:
// shifts by 1, 2, 4 and 8 lanes within each row of 16, then lane 15 of rows 0
// and 2 into rows 1 and 3, then lane 31 into rows 2 and 3 (lanes with no
// source take 0, the identity of both).  A DPP move costs a few cycles where
// an LDS permute (__shfl_*) costs a round trip of ~100; on integers the
// result is the same whatever the order.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t dpp_move(uint32_t v)
{
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, 0xf, false);
}
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint64_t dpp_move(uint64_t v)
{
    return (uint64_t)dpp_move<CTRL, ROW_MASK>((uint32_t)v) | (uint64_t)dpp_move<CTRL, ROW_MASK>((uint32_t)(v >> 32))
                                                                 << 32;
}
template <typename T, typename Op>
__device__ __forceinline__ T wave_scan_incl(T v, Op op)
{
    v = op(v, dpp_move<0x111, 0xf>(v));  // row_shr:1
    v = op(v, dpp_move<0x112, 0xf>(v));  // row_shr:2
    v = op(v, dpp_move<0x114, 0xf>(v));  // row_shr:4
    v = op(v, dpp_move<0x118, 0xf>(v));  // row_shr:8
    v = op(v, dpp_move<0x142, 0xa>(v));  // row_bcast:15 into rows 1, 3
    v = op(v, dpp_move<0x143, 0xc>(v));  // row_bcast:31 into rows 2, 3
    return v;
}
__device__ __forceinline__ uint32_t lane63_u32(uint32_t v) { return (uint32_t)__builtin_amdgcn_readlane((int)v, 63); }
__device__ __forceinline__ uint64_t lane63_u64(uint64_t v)
{
    return (uint64_t)lane63_u32((uint32_t)v) | (uint64_t)lane63_u32((uint32_t)(v >> 32)) << 32;
}
struct OpMax {
    template <typename T>
    __device__ T operator()(T a, T b) const { return a > b ? a : b; }
};
struct OpAdd {
    template <typename T>
    __device__ T operator()(T a, T b) const { return a + b; }
};
// Largest / sum over a fully active wave, in every lane.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) { return lane63_u32(wave_scan_incl(v, OpMax{})); }
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) { return lane63_u64(wave_scan_incl(v, OpMax{})); }
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) { return lane63_u64(wave_scan_incl(v, OpAdd{})); }

// Number of the n keys of tops (LDS, 16-byte aligned) that are >= tv: 32
// keys per step, their LDS reads all in flight.
__device__ __forceinline__ uint32_t count_ge(const uint32_t* tops, int n, uint32_t tv)
{
    uint32_t ge = 0;
    int j = 0;
    for (; j + 32 <= n; j += 32) {
        uint4 x[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) x[u] = ((const uint4*)tops)[j / 4 + u];
#pragma unroll
        for (int u = 0; u < 8; ++u) ge += (x[u].x >= tv) + (x[u].y >= tv) + (x[u].z >= tv) + (x[u].w >= tv);
    }
    for (; j < n; ++j) ge += tops[j] >= tv;
    return ge;
}

// ---- workgroup reductions (all threads call, all get the result) -----------
template <int NT>
__device__ uint64_t block_max_u64(uint64_t v, uint64_t* scratch)
{
    v = wave_max_u64(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    uint64_t r = scratch[0];
#pragma unroll
    for (int w = 1; w < NT / 64; ++w) r = scratch[w] > r ? scratch[w] : r;
    return r;
}

template <int NT>
__device__ uint64_t block_sum_u64(uint64_t v, uint64_t* scratch)
{
    v = wave_sum_u64(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    uint64_t r = 0;
#pragma unroll
    for (int w = 0; w < NT / 64; ++w) r += scratch[w];
    return r;
}

// Exclusive prefix sum over the workgroup (thread order); returns the total.
template <int NT>
__device__ uint64_t block_exclusive_scan_u64(uint64_t v, uint64_t& excl, uint64_t* scratch)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint64_t incl = wave_scan_incl(v, OpAdd{});
    __syncthreads();
    if (lane == 63) scratch[wave] = incl;
    __syncthreads();
    uint64_t before = 0, total = 0;
#pragma unroll
    for (int w = 0; w < NT / 64; ++w) {
        if (w < wave) before += scratch[w];
        total += scratch[w];
    }
    excl = before + incl - v;
    return total;
}

// Bitonic sort of n (power of two) u64 keys in LDS, descending.  Strides of
// 64 and more exchange through LDS (one barrier each); for each size the
// strides below 64 pair lanes of one wave (element i on thread i mod NT), so
// they run in registers with lane shuffles between one LDS read and one write.
__device__ void bitonic_desc(uint64_t* a, int n)
{
    const int NT = blockDim.x, tid = threadIdx.x;
    for (int size = 2; size <= n; size <<= 1) {
        int stride = size >> 1;
        for (; stride >= 64; stride >>= 1) {
            __syncthreads();
            for (int i = tid; i < n; i += NT) {
                const int j = i ^ stride;
                if (j > i) {
                    const bool desc = (i & size) == 0;
                    const uint64_t x = a[i], y = a[j];
                    if (desc ? (x < y) : (x > y)) {
                        a[i] = y;
                        a[j] = x;
                    }
                }
            }
        }
        __syncthreads();
        for (int i0 = 0; i0 < n; i0 += NT) {  // uniform
            const int i = i0 + tid;
            const bool have = i < n;
            uint64_t v = have ? a[i] : 0;
            const bool desc = (i & size) == 0;
            for (int st = stride; st > 0; st >>= 1) {
                const uint64_t w = __shfl_xor(v, st);
                const bool keep_max = ((i & st) == 0) == desc;  // the lower index keeps the larger when descending
                v = keep_max ? (v > w ? v : w) : (v < w ? v : w);
            }
            if (have) a[i] = v;
        }
    }
    __syncthreads();
}

// (key desc, index asc) as one descending u64
__device__ __forceinline__ uint64_t order_key(uint32_t key, uint32_t idx)
{
    return ((uint64_t)key << 32) | (uint64_t)(0xffffffffu - idx);
}

// The four values of float4 group q of a row (elements 4q .. 4q+3; past V
// they read element V-1).  A 16-byte-aligned row of a V % 4 == 0 vocabulary
// is read with one 16-byte buffer load per group (q < V / 4), other rows with
// four dword loads.  The two paths use different load instructions so that
// the compiler keeps the branch: written as a float4 dereference, the aligned
// path was merged with the other into four dword loads for every vocabulary
// (each load instruction then reads 4 bytes per lane, a quarter of a line's
// worth per 16 lanes, and a 1024-thread workgroup took ~10 us to read a
// 128 KB row from the cache).
__device__ __forceinline__ float4 load4(const float* __restrict__ row, uint32_t V, uint32_t q)
{
    if ((V & 3u) == 0 && ((uintptr_t)row & 15u) == 0) {
        const __amdgpu_buffer_rsrc_t r =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(row), (short)0, (int)(V * 4u), 0x00020000);
        return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, q * 16u, 0, 0));
    }
    const uint32_t e = 4 * q;
    return make_float4(row[min(e, V - 1)], row[min(e + 1, V - 1)], row[min(e + 2, V - 1)], row[min(e + 3, V - 1)]);
}

// body(i, value) for every i < V, thread t taking float4 groups t, t + NT, ..
// (coalesced), kRound groups loaded before their values are used.
template <int NT, typename Body>
__device__ __forceinline__ void scan_row(const float* __restrict__ row, uint32_t V, Body body)
{
    const uint32_t V4 = (V + 3) / 4;
    for (uint32_t q0 = threadIdx.x; q0 < V4; q0 += kRound * NT) {
        float4 v[kRound];
#pragma unroll
        for (int r = 0; r < kRound; ++r) v[r] = load4(row, V, min(q0 + (uint32_t)(r * NT), V4 - 1));
#pragma unroll
        for (int r = 0; r < kRound; ++r) {
            const uint32_t q = q0 + (uint32_t)(r * NT);
            if (q < V4) {
                const float e[4] = {v[r].x, v[r].y, v[r].z, v[r].w};
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    if (4 * q + c < V) body(4 * q + c, e[c]);
            }
        }
    }
}

__device__ __forceinline__ uint64_t fixed_e(float l, float lmax, const WarpParams& p)
{
    const float e = det_expf((l - lmax) * p.invT);
    return (uint64_t)(e * p.scale);
}

struct W4 {
    uint64_t a, b, c, d;
};

__device__ __forceinline__ W4 fixed_e4(float4 l, float lmax, const WarpParams& p)
{
    return W4{fixed_e(l.x, lmax, p), fixed_e(l.y, lmax, p), fixed_e(l.z, lmax, p), fixed_e(l.w, lmax, p)};
}

// Weight of token i in a full-vocabulary warp whose top-p prefix is the
// tokens with order_key >= kmin (kmin = 0 keeps every token).
__device__ __forceinline__ uint64_t kept_e(float l, uint32_t i, float lmax, uint64_t kmin, const WarpParams& p)
{
    return order_key(float_key(l), i) >= kmin ? fixed_e(l, lmax, p) : 0;
}

__device__ __forceinline__ W4 kept_e4(float4 l, uint32_t q, float lmax, uint64_t kmin, const WarpParams& p)
{
    const uint32_t i = 4 * q;
    return W4{kept_e(l.x, i, lmax, kmin, p), kept_e(l.y, i + 1, lmax, kmin, p), kept_e(l.z, i + 2, lmax, kmin, p),
              kept_e(l.w, i + 3, lmax, kmin, p)};
}

// Kept tokens of a row from buf[0..k) (order keys by (logit desc, index asc)):
// E, Z, the top-p prefix, then the list re-sorted by index into st.  All
// threads call it; buf holds at least kKMax entries.
__device__ void finish_topk(uint64_t* buf, uint32_t k, float lmax, const WarpParams& p, RowStat* st,
                            uint64_t* keptE, uint32_t& cand_count)
{
    const int tid = threadIdx.x;
    const int NT = blockDim.x;
    for (uint32_t t = tid; t < k; t += NT) {
        const uint32_t key = (uint32_t)(buf[t] >> 32);
        keptE[t] = fixed_e(key_float(key), lmax, p);
    }
    __syncthreads();
    // Z = the k weights' sum, then the top-p prefix: the first t whose running
    // sum c_t (as a double) reaches top_p Z keeps t + 1 tokens and Z = c_t
    // (none: all k, Z unchanged).  Wave 0 scans 64 weights at a time; the u64
    // sums are exact, so they equal a serial running sum.
    if (tid < 64) {
        const int lane = tid;
        auto scan = [&](uint32_t base, uint64_t carry) {  // running sum at base + lane
            return wave_scan_incl((uint64_t)(base + lane < k ? keptE[base + lane] : 0), OpAdd{}) + carry;
        };
        uint64_t z = 0, c0 = 0;
        for (uint32_t base = 0; base < k; base += 64) {
            const uint64_t c = scan(base, z);
            if (base == 0) c0 = c;
            z = lane63_u64(c);
        }
        uint32_t nk = k;
        if (p.top_p < 1.0f) {
            const double thr = (double)p.top_p * (double)z;
            uint64_t carry = 0;
            for (uint32_t base = 0; base < k; base += 64) {
                const uint64_t c = base == 0 ? c0 : scan(base, carry);
                const uint64_t hit = __ballot(base + lane < k && (double)c >= thr);
                if (hit) {
                    const int first = __ffsll((unsigned long long)hit) - 1;
                    nk = base + first + 1;
                    z = (uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)c, first) |
                        (uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(c >> 32), first) << 32;
                    break;
                }
                carry = lane63_u64(c);
            }
        }
        if (lane == 0) {
            st->Z = z;
            st->nk = (int32_t)nk;
            cand_count = nk;
        }
    }
    __syncthreads();
    const uint32_t nk = cand_count;
    // the kept tokens in index order (ascending): each one's place is the
    // count of kept tokens of smaller index (indices are distinct); 8 keys
    // per LDS step
    for (int t = tid; t < (int)nk; t += NT) {
        const uint32_t it = 0xffffffffu - (uint32_t)buf[t];
        int pos = 0, u = 0;
        for (; u + 8 <= (int)nk; u += 8) {
            uint64_t x[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) x[j] = buf[u + j];
#pragma unroll
            for (int j = 0; j < 8; ++j) pos += 0xffffffffu - (uint32_t)x[j] < it;
        }
        for (; u < (int)nk; ++u) pos += 0xffffffffu - (uint32_t)buf[u] < it;
        st->idx[pos] = (int32_t)it;
        st->E[pos] = keptE[t];
    }
}

// buf[0 .. k) = the k largest of the n distinct nonzero order keys c[0 .. n),
// descending: each key's place is the count of larger keys.  The count reads
// 8 keys per step, all in flight (one LDS round trip per step, not per key).
// (Splitting each count over several threads with an LDS counter was slower:
// 14.1 against 11.5 us for 272 rows of ~330 candidates.)
__device__ void rank_top_desc(const uint64_t* c, int n, uint32_t k, uint64_t* buf)
{
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const uint64_t v = c[i];
        uint32_t gt = 0;
        int j = 0;
        for (; j + 8 <= n; j += 8) {
            uint64_t x[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) x[u] = c[j + u];
#pragma unroll
            for (int u = 0; u < 8; ++u) gt += x[u] > v;
        }
        for (; j < n; ++j) gt += c[j] > v;
        if (gt < k) buf[gt] = v;
    }
    __syncthreads();
}

// ---- row statistics ----------------------------------------------------------
// Rows a row_stats launch covers: all (n_sel = 0: workgroup r takes row r),
// or rows row[0 .. n_sel) of every group of n_rows (workgroup g takes row
// (g / n_sel) * n_rows + row[g % n_sel]); logits and stats share the row index.
constexpr int kTreeMax = 16;
struct RowSel {
    uint32_t n_sel = 0, n_rows = 0;
    int32_t row[kTreeMax] = {};
};

// Exact top k of a row whose candidates overflow kCandMax (heavy ties): the
// k-th largest key by bisection on counts, then the ties at that key taken by
// lowest index; buf[0..k) = the kept order keys, sorted.  NT threads.
template <int NT>
__device__ void topk_tie_fallback(const float* __restrict__ row, uint32_t V, uint32_t k, uint64_t* buf, uint64_t* red,
                                  uint32_t& cand_count)
{
    const int tid = threadIdx.x;
    // exact fallback for heavily tied rows: k-th largest key by bisection
    // on counts, then ties at that key taken by lowest index
    uint32_t lo = 0, hi = 0xffffffffu;
    while (lo < hi) {
        const uint32_t mid = lo + (uint32_t)(((uint64_t)hi - lo + 1) >> 1);
        uint64_t c = 0;
        for (uint32_t i = tid; i < V; i += NT) c += float_key(row[i]) >= mid;
        c = block_sum_u64<NT>(c, red);
        if (c >= k) lo = mid;
        else hi = mid - 1;
    }
    const uint32_t kt = lo;
    if (tid == 0) cand_count = 0;
    __syncthreads();
    for (uint32_t i = tid; i < V; i += NT) {
        const uint32_t key = float_key(row[i]);
        if (key > kt) buf[atomicAdd(&cand_count, 1u)] = order_key(key, i);  // < k of them
    }
    __syncthreads();
    const uint32_t ngt = cand_count;
    const uint32_t need = k - ngt;
    // ties in index order: thread t owns the contiguous chunk [t*C, (t+1)*C)
    const uint32_t C = (V + NT - 1) / NT;
    const uint32_t c0 = tid * C, c1 = min(V, c0 + C);
    uint64_t mine = 0;
    for (uint32_t i = c0; i < c1; ++i) mine += float_key(row[i]) == kt;
    uint64_t rank = 0;
    block_exclusive_scan_u64<NT>(mine, rank, red);
    for (uint32_t i = c0; i < c1 && rank < need; ++i)
        if (float_key(row[i]) == kt) {
            buf[ngt + rank] = order_key(kt, i);
            ++rank;
        }
    __syncthreads();
    for (int i = tid; i < kKMax; i += NT)
        if (i >= (int)k) buf[i] = 0;
    bitonic_desc(buf, kKMax);
}

// ---- top-p over the whole vocabulary -----------------------------------------
// The kept set of top_p < 1 without top_k is the shortest prefix of the row in
// (logit desc, index asc) order whose fixed-point sum c has (double)c >=
// (double)top_p * (double)Z.  With S(K) = sum of E over order keys >= K
// (non-increasing in K, and (double) is monotone) that prefix ends at the
// largest key K* with (double)S(K*) >= thr, so the kept tokens are those with
// order_key >= K*.  K* is found by a radix select on mass: four passes over
// the 8-bit digits of the 32-bit logit key, each histogramming (mass, count)
// of the tokens that share the digits chosen so far and taking the largest
// digit whose suffix sum (plus the mass of every larger key) reaches thr
// (with a nonempty bin: for thr <= 0 the first token alone).  The tokens of
// the chosen logit all weigh the same E*; the first j of them (index order)
// complete the prefix, j the least with (double)(above + j E*) >= thr, and
// only when j is short of all of them is the j-th index located.
struct ToppLds {
    uint64_t mass[256];
    uint32_t count[256];
    uint32_t digit, count_sel, tie_idx;
    uint64_t excl_sel, mass_sel;
};

// (mass, count) of the wave's active tokens into their digit bins: one LDS
// atomic per distinct digit (all lanes of the wave call it).
__device__ __forceinline__ void wave_bin_add(bool act, uint32_t d, uint64_t w, ToppLds& s)
{
    const int lane = threadIdx.x & 63;
    uint64_t pend = __ballot(act);
    while (pend) {  // wave-uniform
        const int leader = __builtin_ctzll(pend);
        const uint32_t dl = (uint32_t)__builtin_amdgcn_readlane((int)d, leader);
        const bool mine = act && d == dl;
        const uint64_t m = __ballot(mine);
        const uint64_t x = wave_sum_u64(mine ? w : 0);
        if (lane == leader) {
            atomicAdd((unsigned long long*)&s.mass[dl], (unsigned long long)x);
            atomicAdd(&s.count[dl], (uint32_t)__popcll(m));
        }
        pend &= ~m;
    }
}

// (count) of the wave's active tokens into their digit bins (all lanes call it).
__device__ __forceinline__ void wave_bin_count(bool act, uint32_t d, ToppLds& s)
{
    const int lane = threadIdx.x & 63;
    uint64_t pend = __ballot(act);
    while (pend) {  // wave-uniform
        const int leader = __builtin_ctzll(pend);
        const uint32_t dl = (uint32_t)__builtin_amdgcn_readlane((int)d, leader);
        const uint64_t m = __ballot(act && d == dl);
        if (lane == leader) atomicAdd(&s.count[dl], (uint32_t)__popcll(m));
        pend &= ~m;
    }
}

// The order key of the row's k-th token by (logit desc, index asc), for
// 0 < k < V: a radix select on counts over the four 8-bit digits of the logit
// key gives the k-th largest key kt and the number of tokens above it; the
// first (k - above) tokens of key kt in index order complete the set, so
// kmin = order_key(kt, the last of them), or kt << 32 when all of them are
// in (every order key of kt is above it, every smaller key below).  All
// kRowThreads threads call it and get kmin.
__device__ void topk_bound_select(const float* __restrict__ row, uint32_t V, uint32_t k, ToppLds& s, uint64_t* red,
                                  uint64_t& kmin)
{
    constexpr int NT = kRowThreads;
    constexpr int kBatch = 4;  // float4 groups in flight per thread
    const int tid = threadIdx.x;
    const uint32_t V4 = (V + 3) / 4;
    uint32_t prefix = 0;
    uint64_t above = 0;
    for (int lvl = 0; lvl < 4; ++lvl) {
        const int sh = 24 - 8 * lvl;
        for (int t = tid; t < 256; t += NT) s.count[t] = 0;
        __syncthreads();
        for (uint32_t q0 = 0; q0 < V4; q0 += kBatch * NT) {  // uniform
            float4 v[kBatch];
#pragma unroll
            for (int r = 0; r < kBatch; ++r) v[r] = load4(row, V, min(q0 + (uint32_t)(r * NT + tid), V4 - 1));
#pragma unroll
            for (int r = 0; r < kBatch; ++r) {
                const uint32_t q = q0 + (uint32_t)(r * NT + tid);
                const float e[4] = {v[r].x, v[r].y, v[r].z, v[r].w};
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const uint32_t key = float_key(e[c]);
                    const bool act = q < V4 && 4 * q + c < V && (lvl == 0 || (key >> (sh + 8)) == prefix);
                    wave_bin_count(act, (key >> sh) & 255u, s);
                }
            }
        }
        __syncthreads();
        // thread t < 256 holds bin 255 - t (descending digit order): the bin
        // where the count from the top first reaches k (exactly one thread)
        const uint64_t cv = tid < 256 ? s.count[255 - tid] : 0;
        uint64_t excl = 0;
        (void)block_exclusive_scan_u64<NT>(cv, excl, red);
        if (tid < 256 && above + excl < k && above + excl + cv >= k) {
            s.digit = 255u - (uint32_t)tid;
            s.excl_sel = excl;
            s.count_sel = (uint32_t)cv;
        }
        __syncthreads();
        prefix = (prefix << 8) | s.digit;
        above += s.excl_sel;
    }
    const uint32_t n_t = s.count_sel;
    const uint64_t need = k - above;  // 1 .. n_t
    if (need >= n_t) {
        kmin = (uint64_t)prefix << 32;
        return;
    }
    // the need-th token of key kt in index order: thread t owns [t C, (t+1) C)
    const uint32_t C = (V + NT - 1) / NT;
    const uint32_t c0 = min(V, tid * C), c1 = min(V, c0 + C);
    uint64_t mine = 0;
    for (uint32_t i = c0; i < c1; ++i) mine += float_key(row[i]) == prefix;
    uint64_t rank = 0;
    block_exclusive_scan_u64<NT>(mine, rank, red);
    if (mine && rank < need && need <= rank + mine) {
        uint64_t r = rank;
        for (uint32_t i = c0; i < c1; ++i)
            if (float_key(row[i]) == prefix && ++r == need) {
                s.tie_idx = i;
                break;
            }
    }
    __syncthreads();
    kmin = order_key(prefix, s.tie_idx);
}

// kmin (the order key K*) and the kept sum of a row, over the tokens whose
// order key is at least kfloor (0: all; a large top_k's bound otherwise: the
// top-p prefix is then taken inside the top k, as the oracle's sorted walk
// does); all kRowThreads threads call it and get both.
__device__ void topp_select(const float* __restrict__ row, uint32_t V, float lmax, const WarpParams& p, ToppLds& s,
                            uint64_t* red, uint64_t kfloor, uint64_t& kmin, uint64_t& zkept)
{
    constexpr int NT = kRowThreads;
    constexpr int kBatch = 4;  // float4 groups in flight per thread
    const int tid = threadIdx.x;
    const uint32_t V4 = (V + 3) / 4;
    uint32_t prefix = 0;
    uint64_t above = 0;
    double thr = 0.0;
    if (tid == 0) {
        s.digit = 0;
        s.count_sel = 1;
        s.tie_idx = 0;
        s.excl_sel = s.mass_sel = 0;
    }
    for (int lvl = 0; lvl < 4; ++lvl) {
        const int sh = 24 - 8 * lvl;
        for (int t = tid; t < 256; t += NT) {
            s.mass[t] = 0;
            s.count[t] = 0;
        }
        __syncthreads();
        for (uint32_t q0 = 0; q0 < V4; q0 += kBatch * NT) {  // uniform
            float4 v[kBatch];
#pragma unroll
            for (int r = 0; r < kBatch; ++r) v[r] = load4(row, V, min(q0 + (uint32_t)(r * NT + tid), V4 - 1));
#pragma unroll
            for (int r = 0; r < kBatch; ++r) {
                const uint32_t q = q0 + (uint32_t)(r * NT + tid);
                const float e[4] = {v[r].x, v[r].y, v[r].z, v[r].w};
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const uint32_t key = float_key(e[c]);
                    const bool act = q < V4 && 4 * q + c < V && (lvl == 0 || (key >> (sh + 8)) == prefix) &&
                                     order_key(key, 4 * q + c) >= kfloor;
                    const uint64_t w = act ? fixed_e(e[c], lmax, p) : 0;
                    wave_bin_add(act, (key >> sh) & 255u, w, s);
                }
            }
        }
        __syncthreads();
        // thread t < 256 holds bin 255 - t: thread order is descending digit order
        const uint64_t mv = tid < 256 ? s.mass[255 - tid] : 0;
        const uint32_t cv = tid < 256 ? s.count[255 - tid] : 0;
        uint64_t excl = 0;
        const uint64_t total = block_exclusive_scan_u64<NT>(mv, excl, red);
        if (lvl == 0) thr = (double)p.top_p * (double)total;
        const bool ok = cv > 0 && (double)(above + excl + mv) >= thr;
        const uint64_t first = block_max_u64<NT>(ok ? (uint64_t)(NT - tid) : 0, red);  // > 0: see above
        if (tid == NT - (int)first) {
            s.digit = 255u - (uint32_t)tid;
            s.excl_sel = excl;
            s.mass_sel = mv;
            s.count_sel = cv;
        }
        __syncthreads();
        prefix = (prefix << 8) | s.digit;
        above += s.excl_sel;
    }
    // prefix is the logit key of K*; its n_t tokens weigh e_star each
    const uint32_t n_t = s.count_sel;
    const uint64_t e_star = s.mass_sel / n_t;
    uint32_t j = n_t;
    {
        const double need = (thr - (double)above) / (double)e_star;
        if (need < (double)n_t) j = need <= 1.0 ? 1u : (uint32_t)__builtin_ceil(need);
        j = j < 1 ? 1 : (j > n_t ? n_t : j);
        while (j > 1 && (double)(above + (uint64_t)(j - 1) * e_star) >= thr) --j;
        while (j < n_t && (double)(above + (uint64_t)j * e_star) < thr) ++j;
    }
    zkept = above + (uint64_t)j * e_star;
    if (j == n_t) {  // every active token of that logit (kfloor may cut among its ties)
        const uint64_t all = (uint64_t)prefix << 32;
        kmin = all > kfloor ? all : kfloor;
        return;
    }
    // the j-th token of that logit in index order (of those at or above
    // kfloor: the lowest indices of that logit): thread t owns [t C, (t+1) C)
    const uint32_t C = (V + NT - 1) / NT;
    const uint32_t c0 = min(V, tid * C), c1 = min(V, c0 + C);
    uint64_t mine = 0;
    for (uint32_t i = c0; i < c1; ++i) mine += float_key(row[i]) == prefix && order_key(prefix, i) >= kfloor;
    uint64_t rank = 0;
    block_exclusive_scan_u64<NT>(mine, rank, red);
    if (mine && rank < j && j <= rank + mine) {
        uint64_t r = rank;
        for (uint32_t i = c0; i < c1; ++i)
            if (float_key(row[i]) == prefix && order_key(prefix, i) >= kfloor && ++r == j) {
                s.tie_idx = i;
                break;
            }
    }
    __syncthreads();
    kmin = order_key(prefix, s.tie_idx);
}

// The per-row bound of a full-vocabulary warp (row_bound): the large
// top_k's bound, then the top-p prefix inside it; z = the kept sum when the
// top-p select computed it (have_z), else the caller sums the kept weights.
__device__ void row_bound_select(const float* __restrict__ row, uint32_t V, float lmax, const WarpParams& p,
                                 ToppLds& s, uint64_t* red, uint64_t& kmin, uint64_t& z, bool& have_z)
{
    uint64_t kf = 0;
    if (bound_topk(p, V)) topk_bound_select(row, V, p.top_k, s, red, kf);
    have_z = p.top_p < 1.0f;
    if (have_z) {
        topp_select(row, V, lmax, p, s, red, kf, kmin, z);
    } else {
        kmin = kf;
        z = 0;
    }
}

__global__ __launch_bounds__(kRowThreads) void row_stats_kernel(const float* __restrict__ logits, uint32_t V,
                                                                WarpParams p, RowStat* __restrict__ stats,
                                                                RowSel sel)
{
    __shared__ uint64_t red[kRowThreads / 64];
    __shared__ uint64_t buf[kCandMax];  // thread maxima, then candidates
    __shared__ uint32_t cand_count;
    __shared__ uint64_t keptE[kKMax];
    const int tid = threadIdx.x;
    const size_t r_id = sel.n_sel ? (size_t)(blockIdx.x / sel.n_sel) * sel.n_rows + sel.row[blockIdx.x % sel.n_sel]
                                   : (size_t)blockIdx.x;
    const float* row = logits + r_id * V;
    RowStat* st = stats + r_id;

    // pass 1: max key with the lowest index (argmax), per-thread max key
    uint64_t best = 0;
    scan_row<kRowThreads>(row, V, [&](uint32_t i, float l) {
        const uint64_t o = order_key(float_key(l), i);
        best = o > best ? o : best;
    });
    const uint64_t top = block_max_u64<kRowThreads>(best, red);
    const uint32_t top_key = (uint32_t)(top >> 32);
    const float lmax = key_float(top_key);
    if (tid == 0) {
        st->lmax = lmax;
        st->argmax = (int32_t)(0xffffffffu - (uint32_t)top);
        st->kmin = 0;
    }
    if (p.greedy) return;

    const bool topk = list_topk(p, V);
    if (row_bound(p, V)) {  // full vocabulary under a bound: top-p, a large top_k, or both
        __shared__ ToppLds tps;
        uint64_t kmin, z;
        bool have_z;
        row_bound_select(row, V, lmax, p, tps, red, kmin, z, have_z);
        if (!have_z) {
            scan_row<kRowThreads>(row, V, [&](uint32_t i, float l) { z += kept_e(l, i, lmax, kmin, p); });
            z = block_sum_u64<kRowThreads>(z, red);
        }
        if (tid == 0) {
            st->Z = z;
            st->kmin = kmin;
            st->nk = (int32_t)V;
        }
        return;
    }
    if (!topk) {  // full vocabulary: Z over every token
        uint64_t z = 0;
        scan_row<kRowThreads>(row, V, [&](uint32_t, float l) { z += fixed_e(l, lmax, p); });
        z = block_sum_u64<kRowThreads>(z, red);
        if (tid == 0) {
            st->Z = z;
            st->nk = (int32_t)V;
        }
        return;
    }
    const uint32_t k = p.top_k;

    // fast path: the k-th largest per-thread maximum is <= the k-th largest
    // logit, so the tokens with key >= it include the top k
    buf[tid] = best >> 32;  // per-thread max key (0 if the thread has no token)
    bitonic_desc(buf, kRowThreads);
    const uint32_t t0 = (uint32_t)buf[k - 1];
    if (tid == 0) cand_count = 0;
    __syncthreads();
    scan_row<kRowThreads>(row, V, [&](uint32_t i, float l) {
        const uint32_t key = float_key(l);
        if (key >= t0) {
            const uint32_t slot = atomicAdd(&cand_count, 1u);
            if (slot < kCandMax) buf[slot] = order_key(key, i);
        }
    });
    __syncthreads();
    const uint32_t nc = cand_count;
    __syncthreads();
    if (nc <= kCandMax) {
        int n2 = 1;
        while (n2 < (int)nc) n2 <<= 1;
        for (int i = tid; i < n2; i += kRowThreads)
            if (i >= (int)nc) buf[i] = 0;  // sorts last
        bitonic_desc(buf, n2);
    } else {
        topk_tie_fallback<kRowThreads>(row, V, k, buf, red, cand_count);
    }
    finish_topk(buf, k, lmax, p, st, keptE, cand_count);
}

// ---- decisions -----------------------------------------------------------------
// weight of token x in a row's warp (0 if not kept)
__device__ uint64_t weight_of(const RowStat& st, const float* row, uint32_t V, bool topk, int32_t x,
                              const WarpParams& p)
{
    if (x < 0 || (uint32_t)x >= V) return 0;
    if (!topk) return kept_e(row[x], (uint32_t)x, st.lmax, st.kmin, p);
    int lo = 0, hi = st.nk - 1;
    while (lo <= hi) {
        const int mid = (lo + hi) >> 1;
        const int32_t v = st.idx[mid];
        if (v == x) return st.E[mid];
        if (v < x) lo = mid + 1;
        else hi = mid - 1;
    }
    return 0;
}

// Full-vocabulary inverse-CDF draw of per-token weights (u64, exact):
// T = trunc(u * total), first j with T < cumsum, else the last j with w > 0.
// w4(q) gives the weights of elements 4q .. 4q+3 (0 past V).  Round r covers
// float4 groups [r NT, (r+1) NT) (thread t takes group r NT + t, coalesced).
// Round totals first (kRound rounds per pass, wave xor trees, then LDS), the
// round holding T, one block scan inside it, then the 4 elements of the
// owning thread.
template <typename F4>
__device__ int32_t block_cdf_pick(uint32_t V, float u, F4 w4, uint64_t* scratch, int32_t* pick)
{
    constexpr int NW = kSeqThreads / 64;
    __shared__ uint64_t rt[kMaxRounds];
    __shared__ uint64_t wpart[NW][kRound];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t V4 = (V + 3) / 4;
    const uint32_t R = (V4 + kSeqThreads - 1) / kSeqThreads;
    int32_t last = -1;
    for (uint32_t g0 = 0; g0 < R; g0 += kRound) {
        W4 x[kRound];
#pragma unroll
        for (int r = 0; r < kRound; ++r) x[r] = w4(min((g0 + r) * kSeqThreads + tid, V4 - 1));
        uint64_t sr[kRound];
#pragma unroll
        for (int r = 0; r < kRound; ++r) {
            const uint32_t q = (g0 + r) * kSeqThreads + tid;
            sr[r] = 0;
            if (g0 + r < R && q < V4) {
                const uint64_t e[4] = {x[r].a, x[r].b, x[r].c, x[r].d};
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    if (4 * q + c < V && e[c]) {
                        sr[r] += e[c];
                        last = (int32_t)(4 * q + c);
                    }
            }
        }
#pragma unroll
        for (int r = 0; r < kRound; ++r) sr[r] = wave_sum_u64(sr[r]);
        if (lane == 0)
#pragma unroll
            for (int r = 0; r < kRound; ++r) wpart[wave][r] = sr[r];
        __syncthreads();
        if (tid < kRound && g0 + tid < R) {
            uint64_t t = 0;
#pragma unroll
            for (int v = 0; v < NW; ++v) t += wpart[v][tid];
            rt[g0 + tid] = t;
        }
        __syncthreads();
    }
    uint64_t total = 0;
    for (uint32_t r = 0; r < R; ++r) total += rt[r];
    const uint64_t T = (uint64_t)((double)u * (double)total);
    uint32_t rstar = R;
    uint64_t rbefore = 0;
    {
        uint64_t c = 0;
        for (uint32_t r = 0; r < R; ++r) {
            if (rt[r] && T < c + rt[r]) {
                rstar = r;
                rbefore = c;
                break;
            }
            c += rt[r];
        }
    }
    if (tid == 0) *pick = -1;
    __syncthreads();
    if (rstar < R) {  // uniform: every thread read the same round totals
        const uint32_t q = rstar * kSeqThreads + tid;
        W4 x = w4(min(q, V4 - 1));
        const uint64_t e[4] = {x.a, x.b, x.c, x.d};
        uint64_t mine = 0;
#pragma unroll
        for (int c = 0; c < 4; ++c)
            if (q < V4 && 4 * q + c < V) mine += e[c];
        uint64_t before = 0;
        block_exclusive_scan_u64<kSeqThreads>(mine, before, scratch);
        before += rbefore;
        if (mine && T >= before && T < before + mine) {
            uint64_t c = before;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                if (4 * q + k < V) {
                    c += e[k];
                    if (T < c) {
                        *pick = (int32_t)(4 * q + k);
                        break;
                    }
                }
            }
        }
    }
    __syncthreads();
    int32_t r = *pick;
    if (r < 0) {  // T >= total (rounding): the last token with nonzero weight
        const uint64_t lastp = block_max_u64<kSeqThreads>((uint64_t)(int64_t)(last + 1), scratch);
        r = lastp ? (int32_t)lastp - 1 : (int32_t)V - 1;
    }
    __syncthreads();
    return r;
}

// Inverse-CDF draw over a kept list (index order).
__device__ int32_t list_cdf_pick(const int32_t* idx, const uint64_t* W, int n, uint64_t Z, float u, uint32_t V)
{
    const uint64_t T = (uint64_t)((double)u * (double)Z);
    uint64_t c = 0;
    int32_t last = -1;
    for (int t = 0; t < n; ++t) {
        if (!W[t]) continue;
        c += W[t];
        last = idx[t];
        if (T < c) return idx[t];
    }
    return last < 0 ? (int32_t)V - 1 : last;
}

// Draw from a row's warp with uniform u (all threads return the token).
__device__ int32_t draw_row(const RowStat& st, const float* row, uint32_t V, bool topk, float u, const WarpParams& p,
                            uint64_t* scratch, int32_t* pick)
{
    if (topk) return list_cdf_pick(st.idx, st.E, st.nk, st.Z, u, V);
    const float lmax = st.lmax;
    const uint64_t kmin = st.kmin;
    return block_cdf_pick(V, u, [&](uint32_t q) { return kept_e4(load4(row, V, q), q, lmax, kmin, p); }, scratch,
                          pick);
}

__device__ __forceinline__ uint64_t residual_weight(uint64_t P, uint64_t Q, uint64_t Zp, uint64_t Zq, int sh)
{
    const double a = (double)P * (double)Zq;
    const double c = (double)Q * (double)Zp;
    const double r = a - c;
    return r > 0.0 ? (uint64_t)__builtin_ldexp(r, sh) : 0;
}

// Inverse-CDF draw over a kept list in index order (list_cdf_pick with the
// workgroup): thread t < n holds weight wt of entry t; T = trunc(u Z); the
// first entry with T < cumsum, else the last nonzero one, else V - 1.  All
// threads call it and get the token.
__device__ int32_t block_list_pick(const int32_t* idx, uint64_t wt, int n, uint64_t Z, float u, uint32_t V,
                                   uint64_t* scratch, int32_t* pick)
{
    const int tid = threadIdx.x;
    const uint64_t w = tid < n ? wt : 0;
    const uint64_t T = (uint64_t)((double)u * (double)Z);
    uint64_t excl = 0;
    (void)block_exclusive_scan_u64<kSeqThreads>(w, excl, scratch);
    const uint64_t lastp = block_max_u64<kSeqThreads>(w ? (uint64_t)(tid + 1) : 0, scratch);
    if (tid == 0) *pick = -1;
    __syncthreads();
    if (w && T >= excl && T < excl + w) *pick = idx[tid];
    __syncthreads();
    const int32_t r = *pick;
    return r >= 0 ? r : lastp ? idx[lastp - 1] : (int32_t)V - 1;
}

// A row's kept list copied into LDS with coalesced loads (all threads call it).
__device__ __forceinline__ int stage_list(const RowStat& st, int32_t* sidx, uint64_t* sE)
{
    const int n = st.nk;
    for (int t = threadIdx.x; t < n; t += blockDim.x) {
        sidx[t] = st.idx[t];
        sE[t] = st.E[t];
    }
    return n;
}

// Top-k / top-p acceptance of one sequence per workgroup (greedy and
// full-vocabulary acceptance run in the chunk kernels below).  All 2k + 1
// kept lists of the sequence (target rows 0..k, draft rows 0..k-1; each at
// most K = top_k entries) are staged in LDS with one round of loads, the
// weights P(x_i), Q(x_i) of every draft token looked up in one pass, then the
// accept walk, and the residual or bonus draw from the staged lists.
// Dynamic LDS: (2k + 1) K (8 + 4) bytes.
__global__ __launch_bounds__(kSeqThreads) void decide_kernel(const RowStat* __restrict__ stats,
                                                             const int32_t* __restrict__ draft_tokens,
                                                             const float* __restrict__ uniforms, uint32_t k,
                                                             uint32_t K, uint32_t V, int32_t* __restrict__ out,
                                                             int32_t* __restrict__ nacc)
{
    extern __shared__ uint64_t dyn[];
    __shared__ int32_t nks[2 * kMaxK + 1];
    __shared__ uint64_t Zs[2 * kMaxK + 1];
    __shared__ int32_t sx[kMaxK];
    __shared__ uint64_t Pw[kMaxK], Qw[kMaxK];
    __shared__ uint64_t scratch[kSeqThreads / 64];
    __shared__ uint32_t s_rej;
    __shared__ int32_t s_pick;
    const int tid = threadIdx.x;
    const uint32_t b = blockIdx.x, L = 2 * k + 1;
    const RowStat* ts = stats + (size_t)b * (k + 1);                            // target rows
    const RowStat* ds = stats + (size_t)gridDim.x * (k + 1) + (size_t)b * k;   // draft rows
    auto list = [&](uint32_t l) -> const RowStat& { return l <= k ? ts[l] : ds[l - k - 1]; };
    uint64_t* sE = dyn;                          // [L][K]
    int32_t* sI = (int32_t*)(dyn + (size_t)L * K);  // [L][K]
    const int32_t* x = draft_tokens + (size_t)b * k;
    const float* u = uniforms + (size_t)b * (k + 1);
    int32_t* o = out + (size_t)b * (k + 1);

    // one round of loads: entries past a list's length are read (in bounds of
    // its arrays) and never used
    for (uint32_t e = tid; e < L * K; e += kSeqThreads) {
        const uint32_t l = e / K, t = e - l * K;
        sI[e] = list(l).idx[t];
        sE[e] = list(l).E[t];
    }
    if (tid < (int)L) {
        nks[tid] = list(tid).nk;
        Zs[tid] = list(tid).Z;
    }
    if (tid < (int)k) {
        sx[tid] = x[tid];
        Pw[tid] = 0;
        Qw[tid] = 0;
    }
    for (uint32_t i = tid; i <= k; i += kSeqThreads) o[i] = -1;
    __syncthreads();
    // P(x_i) from target list i, Q(x_i) from draft list i (token ids in a list are distinct)
    for (uint32_t e = tid; e < L * K; e += kSeqThreads) {
        const uint32_t l = e / K, t = e - l * K;
        if (l == k || (int)t >= nks[l]) continue;
        const uint32_t i = l < k ? l : l - k - 1;
        if (sI[e] == sx[i]) (l < k ? Pw : Qw)[i] = sE[e];
    }
    __syncthreads();
    if (tid == 0) {  // the accept walk: the first rejected position, k if none
        uint32_t rej = k;
        for (uint32_t i = 0; i < k; ++i) {
            const double lhs = ((double)u[i] * (double)Qw[i]) * (double)Zs[i];
            const double rhs = (double)Pw[i] * (double)Zs[k + 1 + i];
            if (!(lhs < rhs)) {
                rej = i;
                break;
            }
            o[i] = sx[i];
        }
        s_rej = rej;
        nacc[b] = (int32_t)rej;
    }
    __syncthreads();
    const uint32_t i = s_rej;
    if (i == k) {  // every draft accepted: bonus token from the target row k
        const int n = nks[k];
        const int32_t t = block_list_pick(sI + (size_t)k * K, tid < n ? sE[(size_t)k * K + tid] : 0, n, Zs[k], u[k],
                                          V, scratch, &s_pick);
        if (tid == 0) o[k] = t;
        return;
    }
    // first rejection at i: draw from max(0, p - q) with u[k] (from p when that
    // is all zero).  Tokens only in the draft list weigh 0 in the residual, so
    // the draw runs over the target list's entries (index order) with weights
    // R = residual(P, Q) -- Q looked up by binary search in the draft list.
    const uint64_t Zp = Zs[i], Zq = Zs[k + 1 + i];
    const int sh = 62 - bitlen64(Zp) - bitlen64(Zq);
    const int32_t* aidx = sI + (size_t)i * K;
    const uint64_t* aE = sE + (size_t)i * K;
    const int32_t* bidx = sI + (size_t)(k + 1 + i) * K;
    const uint64_t* bE = sE + (size_t)(k + 1 + i) * K;
    const int na = nks[i], nb = nks[k + 1 + i];
    uint64_t R = 0, P = 0;
    if (tid < na) {
        const int32_t j = aidx[tid];
        P = aE[tid];
        int lo = 0, hi = nb - 1;
        uint64_t Q = 0;
        while (lo <= hi) {
            const int mid = (lo + hi) >> 1;
            const int32_t v = bidx[mid];
            if (v == j) {
                Q = bE[mid];
                break;
            }
            if (v < j) lo = mid + 1;
            else hi = mid - 1;
        }
        R = residual_weight(P, Q, Zp, Zq, sh);
    }
    const uint64_t SR = block_sum_u64<kSeqThreads>(R, scratch);
    const int32_t t = SR ? block_list_pick(aidx, R, na, SR, u[k], V, scratch, &s_pick)
                         : block_list_pick(aidx, P, na, Zp, u[k], V, scratch, &s_pick);
    if (tid == 0) o[i] = t;
}

// ---- tree acceptance ------------------------------------------------------------
// Shape of a draft tree: node 0 the root, parent[i] in [0, i) for i >= 1.
struct TreeShape {
    int32_t n;
    int32_t parent[kTreeMax];
};

// One workgroup per tree (multi-draft speculative sampling, SpecInfer, Miao
// et al. 2024, Alg. 2).  At node v: C = warp(target row v) (total Zc), q =
// warp(draft row v); the children c of v in index order are tested with
// u[c-1]: accept iff (u Q_x) Zc < C_x Zq; after a rejection C becomes the
// residual max(0, C Zq - Q Zc) scaled as in decide_kernel (kept when it sums
// to 0).  An accepted child becomes v; otherwise the token is drawn from C
// with u[n-1].  Full vocabulary: C is never stored -- level l of the residual
// chain is recomputed per token from (P_j, Q_j) with the saved (Zc, shift) of
// the levels before.  top_k: C lives in the merged kept list of the two rows
// (at most 2 top_k entries, LDS).  On a chain this is decide_kernel's rule.
__global__ __launch_bounds__(kSeqThreads) void decide_tree_kernel(const RowStat* __restrict__ stats,
                                                                  const float* __restrict__ tl,
                                                                  const float* __restrict__ dl,
                                                                  const int32_t* __restrict__ tokens,
                                                                  const float* __restrict__ uniforms, uint32_t V,
                                                                  WarpParams p, TreeShape shape,
                                                                  int32_t* __restrict__ out,
                                                                  int32_t* __restrict__ path,
                                                                  int32_t* __restrict__ nacc)
{
    __shared__ uint64_t scratch[kSeqThreads / 64];
    __shared__ int32_t pick;
    __shared__ int32_t uidx[2 * kKMax];
    __shared__ uint64_t uC[2 * kKMax];
    __shared__ uint64_t uQ[2 * kKMax];
    __shared__ int32_t un;
    __shared__ uint64_t sSR;
    __shared__ uint64_t lvZ[kTreeMax];
    __shared__ int32_t lvSh[kTreeMax];
    const int tid = threadIdx.x;
    const uint32_t b = blockIdx.x;
    const int n = shape.n;
    const RowStat* ts = stats + (size_t)b * n;
    const RowStat* ds = stats + (size_t)gridDim.x * n + (size_t)b * n;
    const int32_t* tok = tokens + (size_t)b * n;
    const float* u = p.greedy ? nullptr : uniforms + (size_t)b * n;
    int32_t* o = out + (size_t)b * n;
    int32_t* pa = path + (size_t)b * n;
    const bool topk = list_topk(p, V);

    for (int i = tid; i < n; i += kSeqThreads) {
        o[i] = -1;
        pa[i] = i == 0 ? 0 : -1;
    }
    __syncthreads();
    int v = 0, depth = 0;
    for (;;) {
        int next = -1;
        const float* trow = tl + ((size_t)b * n + v) * V;
        if (p.greedy) {
            const int32_t a = ts[v].argmax;
            for (int c = v + 1; c < n; ++c)
                if (shape.parent[c] == v && tok[c] == a) {
                    next = c;
                    break;
                }
            if (tid == 0) o[depth] = a;
            if (next < 0) break;
        } else {
            const float* drow = dl + ((size_t)b * n + v) * V;
            const float lpm = ts[v].lmax, lqm = ds[v].lmax;
            const uint64_t kpm = ts[v].kmin, kqm = ds[v].kmin;
            uint64_t Zc = ts[v].Z;
            const uint64_t Zq = ds[v].Z;  // read only when v has children (draft stats exist then)
            int L = 0;                     // levels of the residual chain (full vocabulary)
            bool have_list = false;
            // weights of elements 4q..4q+3 at the current level (full vocabulary), and the draft's
            auto level4 = [&](uint32_t q, W4& qw) {
                W4 a = kept_e4(load4(trow, V, q), q, lpm, kpm, p);
                qw = kept_e4(load4(drow, V, q), q, lqm, kqm, p);
                for (int l = 0; l < L; ++l) {
                    a.a = residual_weight(a.a, qw.a, lvZ[l], Zq, lvSh[l]);
                    a.b = residual_weight(a.b, qw.b, lvZ[l], Zq, lvSh[l]);
                    a.c = residual_weight(a.c, qw.c, lvZ[l], Zq, lvSh[l]);
                    a.d = residual_weight(a.d, qw.d, lvZ[l], Zq, lvSh[l]);
                }
                return a;
            };
            for (int c = v + 1; c < n; ++c) {
                if (shape.parent[c] != v) continue;
                if (topk && !have_list) {
                    if (tid == 0) {  // merged kept lists, index order
                        const RowStat& A = ts[v];
                        const RowStat& B = ds[v];
                        int ia = 0, ib = 0, m = 0;
                        while (ia < A.nk || ib < B.nk) {
                            const int32_t ja = ia < A.nk ? A.idx[ia] : 0x7fffffff;
                            const int32_t jb = ib < B.nk ? B.idx[ib] : 0x7fffffff;
                            const int32_t j = ja < jb ? ja : jb;
                            uC[m] = ja == j ? A.E[ia++] : 0;
                            uQ[m] = jb == j ? B.E[ib++] : 0;
                            uidx[m++] = j;
                        }
                        un = m;
                    }
                    __syncthreads();
                    have_list = true;
                }
                const int32_t x = tok[c];
                const uint64_t Qx = weight_of(ds[v], drow, V, topk, x, p);
                uint64_t Cx = 0;
                if (topk) {
                    int lo = 0, hi = un - 1;
                    while (lo <= hi) {
                        const int mid = (lo + hi) >> 1;
                        if (uidx[mid] == x) {
                            Cx = uC[mid];
                            break;
                        }
                        if (uidx[mid] < x) lo = mid + 1;
                        else hi = mid - 1;
                    }
                } else {
                    Cx = weight_of(ts[v], trow, V, false, x, p);
                    for (int l = 0; l < L; ++l) Cx = residual_weight(Cx, Qx, lvZ[l], Zq, lvSh[l]);
                }
                const double lhs = ((double)u[c - 1] * (double)Qx) * (double)Zc;
                const double rhs = (double)Cx * (double)Zq;
                if (lhs < rhs) {
                    if (tid == 0) o[depth] = x;
                    next = c;
                    break;
                }
                const int sh = 62 - bitlen64(Zc) - bitlen64(Zq);
                uint64_t SR;
                if (topk) {
                    if (tid == 0) {
                        uint64_t t = 0;
                        for (int i = 0; i < un; ++i) t += residual_weight(uC[i], uQ[i], Zc, Zq, sh);
                        if (t)
                            for (int i = 0; i < un; ++i) uC[i] = residual_weight(uC[i], uQ[i], Zc, Zq, sh);
                        sSR = t;
                    }
                    __syncthreads();
                    SR = sSR;
                    __syncthreads();
                } else {
                    uint64_t mine = 0;
                    const uint32_t V4 = (V + 3) / 4;
                    for (uint32_t q = tid; q < V4; q += kSeqThreads) {
                        W4 qw;
                        const W4 a = level4(q, qw);
                        const uint64_t e[4] = {residual_weight(a.a, qw.a, Zc, Zq, sh), residual_weight(a.b, qw.b, Zc, Zq, sh),
                                               residual_weight(a.c, qw.c, Zc, Zq, sh), residual_weight(a.d, qw.d, Zc, Zq, sh)};
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            if (4 * q + j < V) mine += e[j];
                    }
                    SR = block_sum_u64<kSeqThreads>(mine, scratch);
                    if (SR) {
                        if (tid == 0) {
                            lvZ[L] = Zc;
                            lvSh[L] = sh;
                        }
                        __syncthreads();
                        ++L;
                    }
                }
                if (SR) Zc = SR;
            }
            if (next < 0) {
                int32_t t;
                const float uf = u[n - 1];
                if (topk) {
                    t = have_list ? list_cdf_pick(uidx, uC, un, Zc, uf, V)
                                  : list_cdf_pick(ts[v].idx, ts[v].E, ts[v].nk, Zc, uf, V);
                } else if (L == 0) {
                    t = draw_row(ts[v], trow, V, false, uf, p, scratch, &pick);
                } else {
                    t = block_cdf_pick(V, uf, [&](uint32_t q) { W4 qw; return level4(q, qw); }, scratch, &pick);
                }
                if (tid == 0) o[depth] = t;
                break;
            }
            __syncthreads();  // the list / levels of v are not reused by the next node before every thread is done
        }
        ++depth;
        if (tid == 0) pa[depth] = next;
        v = next;
    }
    if (tid == 0) nacc[b] = depth;
}

// Top-k / top-p draw of one row per workgroup from its kept list (greedy and
// full-vocabulary draws run in the chunk kernels below).
// Draw d (blockIdx.x) comes from row map[d] (row d without a map).
__global__ __launch_bounds__(kSeqThreads) void sample_kernel(const RowStat* __restrict__ stats,
                                                             const float* __restrict__ uniforms, uint32_t V,
                                                             const int32_t* __restrict__ map,
                                                             int32_t* __restrict__ out)
{
    __shared__ int32_t sidx[kKMax];
    __shared__ uint64_t sE[kKMax];
    const uint32_t d = blockIdx.x, r = map ? (uint32_t)map[d] : d;
    const int n = stage_list(stats[r], sidx, sE);
    __syncthreads();
    if (threadIdx.x == 0) out[d] = list_cdf_pick(sidx, sE, n, stats[r].Z, uniforms[d], V);
}

// Greedy tree drafting: workgroup i takes row i and writes its n_kids[i]
// largest tokens by (logit desc, index asc), in that order, to
// out[first_kid[i] ..]: pass r picks the largest order key below pick r-1.
__global__ __launch_bounds__(kRowThreads) void topb_kernel(const float* __restrict__ logits, uint32_t V,
                                                           const int32_t* __restrict__ first_kid,
                                                           const int32_t* __restrict__ n_kids,
                                                           int32_t* __restrict__ out)
{
    __shared__ uint64_t red[kRowThreads / 64];
    const uint32_t i = blockIdx.x;
    const float* row = logits + (size_t)i * V;
    uint64_t prev = ~0ull;
    const int nk = n_kids[i];
    for (int r = 0; r < nk; ++r) {  // uniform
        uint64_t best = 0;
        scan_row<kRowThreads>(row, V, [&](uint32_t idx, float l) {
            const uint64_t o = order_key(float_key(l), idx);
            if (o < prev && o > best) best = o;
        });
        best = block_max_u64<kRowThreads>(best, red);
        if (threadIdx.x == 0) out[first_kid[i] + r] = (int32_t)(0xffffffffu - (uint32_t)best);
        prev = best;
    }
}

// Full-vocabulary (or greedy) draw, each row split over up to kMaxChunks
// workgroups (one workgroup reading a whole row is bound by what a single CU
// keeps in flight): chunk maxima; chunk sums of fixed_e(l - lmax) and the last
// token of nonzero weight; then one workgroup per row takes T = trunc(u * Z),
// finds the chunk holding T from the chunk sums in chunk order and scans that
// chunk alone.  Integer weights make this the draw of block_cdf_pick exactly:
// first j with T < cumsum, else the last j with w > 0.
constexpr int kChunkThreads = 256;
constexpr int kMaxChunks = 64;
constexpr uint32_t kMaxGridRows = 65535;  // rows of a chunk launch run along grid y

struct ChunkPart {
    uint64_t top;  // largest order_key of the chunk
    uint64_t sum;  // sum of its weights
    int32_t last;  // last index of nonzero weight, -1 if none
    int32_t pad;
};

// Chunks of a row of V elements: G chunks of CG float4 groups (the last one shorter).
struct ChunkPlan {
    uint32_t G, CG;
};
__host__ __device__ inline ChunkPlan chunk_plan(uint32_t V)
{
    const uint32_t V4 = (V + 3) / 4;
    uint32_t G = (V4 + kChunkThreads - 1) / kChunkThreads;
    G = G < 1 ? 1 : (G > (uint32_t)kMaxChunks ? (uint32_t)kMaxChunks : G);
    return ChunkPlan{G, (V4 + G - 1) / G};
}

// Rows of a chunk launch: rows r < na of a, then rows of b.
struct RowSrc {
    const float* a;
    uint32_t na;
    const float* b;
    __device__ const float* row(uint32_t r, uint32_t V) const
    {
        return r < na ? a + (size_t)r * V : b + (size_t)(r - na) * V;
    }
};

// Largest order_key of chunk (blockIdx.x) of row (blockIdx.y).
__global__ __launch_bounds__(kChunkThreads) void chunk_max_kernel(RowSrc rs, uint32_t V, ChunkPlan cp,
                                                                  ChunkPart* __restrict__ part)
{
    __shared__ uint64_t scratch[kChunkThreads / 64];
    const uint32_t r = blockIdx.y, g = blockIdx.x, V4 = (V + 3) / 4;
    const float* row = rs.row(r, V);
    const uint32_t q1 = min(V4, (g + 1) * cp.CG);
    uint64_t best = 0;
    for (uint32_t q = g * cp.CG + threadIdx.x; q < q1; q += kChunkThreads) {
        const float4 v = load4(row, V, q);
        const float e[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int c = 0; c < 4; ++c)
            if (4 * q + c < V) {
                const uint64_t o = order_key(float_key(e[c]), 4 * q + c);
                best = o > best ? o : best;
            }
    }
    best = block_max_u64<kChunkThreads>(best, scratch);
    if (threadIdx.x == 0) part[(size_t)r * cp.G + g].top = best;
}

// The row's largest order_key from its chunk maxima (all threads get it).
__device__ __forceinline__ uint64_t row_top(const ChunkPart* part, ChunkPlan cp, uint64_t* scratch)
{
    uint64_t t = 0;
    if (threadIdx.x < cp.G) t = part[threadIdx.x].top;
    return block_max_u64<kChunkThreads>(t, scratch);
}

// Sum and last nonzero index of the chunk's weights fixed_e(l - lmax).
__global__ __launch_bounds__(kChunkThreads) void chunk_sum_kernel(RowSrc rs, uint32_t V, ChunkPlan cp, WarpParams p,
                                                                  const uint64_t* __restrict__ kmin,
                                                                  ChunkPart* __restrict__ part)
{
    __shared__ uint64_t scratch[kChunkThreads / 64];
    const uint32_t r = blockIdx.y, g = blockIdx.x, V4 = (V + 3) / 4;
    const float* row = rs.row(r, V);
    ChunkPart* rp = part + (size_t)r * cp.G;
    const uint32_t q0 = g * cp.CG + threadIdx.x, q1 = min(V4, (g + 1) * cp.CG);
    // this thread's first group is loaded before the chunk maxima are read
    const float4 v0 = load4(row, V, min(q0, V4 - 1));
    const float lmax = key_float((uint32_t)(row_top(rp, cp, scratch) >> 32));
    const uint64_t km = kmin ? kmin[r] : 0;
    uint64_t sum = 0;
    int32_t last = -1;
    for (uint32_t q = q0; q < q1; q += kChunkThreads) {
        const W4 w = kept_e4(q == q0 ? v0 : load4(row, V, q), q, lmax, km, p);
        const uint64_t e[4] = {w.a, w.b, w.c, w.d};
#pragma unroll
        for (int c = 0; c < 4; ++c)
            if (4 * q + c < V && e[c]) {
                sum += e[c];
                last = (int32_t)(4 * q + c);
            }
    }
    sum = block_sum_u64<kChunkThreads>(sum, scratch);
    const uint64_t lastp = block_max_u64<kChunkThreads>((uint64_t)(int64_t)(last + 1), scratch);
    if (threadIdx.x == 0) {
        rp[g].sum = sum;
        rp[g].last = (int32_t)lastp - 1;
    }
}

// Inverse-CDF draw with uniform u over weights w4(q) (float4 group q) whose
// chunk sums and last nonzero indices are in cparts (the row's G chunks):
// T = trunc(u * total), the chunk holding T from the sums in chunk order, then
// a scan of that chunk alone; T >= total (rounding) gives the last index of
// nonzero weight (V - 1 if none).  All threads of the workgroup call it; the
// token is valid in thread 0.
template <typename F4>
__device__ int32_t chunk_draw(uint32_t V, ChunkPlan cp, float u, F4 w4, const ChunkPart* cparts, uint64_t* scratch)
{
    __shared__ int32_t pick;
    __shared__ uint64_t gbase;
    const int tid = threadIdx.x;
    const uint32_t V4 = (V + 3) / 4;
    uint64_t cs = 0;
    int32_t cl = -1;
    if (tid < (int)cp.G) {
        cs = cparts[tid].sum;
        cl = cparts[tid].last;
    }
    const uint64_t total = block_sum_u64<kChunkThreads>(cs, scratch);
    const uint64_t T = (uint64_t)((double)u * (double)total);
    uint64_t before = 0;
    (void)block_exclusive_scan_u64<kChunkThreads>(cs, before, scratch);
    // the chunk with before <= T < before + sum (sum > 0): at most one
    const bool hit = tid < (int)cp.G && cs && T >= before && T < before + cs;
    const uint64_t hitp = block_max_u64<kChunkThreads>(hit ? (uint64_t)(kMaxChunks - tid) : 0, scratch);
    const uint64_t lastp = block_max_u64<kChunkThreads>((uint64_t)(int64_t)(cl + 1), scratch);
    if (tid == 0) pick = -1;
    if (hitp) {  // uniform
        const uint32_t g = kMaxChunks - (uint32_t)hitp;
        if (tid == (int)g) gbase = before;
        __syncthreads();
        uint64_t base = gbase;
        const uint32_t q1 = min(V4, (g + 1) * cp.CG);
        for (uint32_t qb = g * cp.CG; qb < q1; qb += kChunkThreads) {  // uniform
            const uint32_t q = qb + tid;
            const W4 w = w4(min(q, V4 - 1));
            const uint64_t e[4] = {w.a, w.b, w.c, w.d};
            uint64_t mine = 0;
#pragma unroll
            for (int c = 0; c < 4; ++c)
                if (q < q1 && 4 * q + c < V) mine += e[c];
            uint64_t excl = 0;
            const uint64_t pass = block_exclusive_scan_u64<kChunkThreads>(mine, excl, scratch);
            excl += base;
            if (mine && T >= excl && T < excl + mine) {
                uint64_t c = excl;
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    if (4 * q + k < V) {
                        c += e[k];
                        if (T < c) {
                            pick = (int32_t)(4 * q + k);
                            break;
                        }
                    }
            }
            base += pass;
        }
    }
    __syncthreads();
    int32_t t = pick;
    if (t < 0) t = lastp ? (int32_t)lastp - 1 : (int32_t)V - 1;
    return t;
}

// One workgroup per draw d: the argmax (greedy) or the inverse-CDF draw from
// row map[d] (row d without a map) with uniforms[d].
__global__ __launch_bounds__(kChunkThreads) void chunk_pick_kernel(const float* __restrict__ logits,
                                                                   const float* __restrict__ uniforms, uint32_t V,
                                                                   ChunkPlan cp, WarpParams p,
                                                                   const ChunkPart* __restrict__ part,
                                                                   const uint64_t* __restrict__ kmin,
                                                                   const int32_t* __restrict__ map,
                                                                   int32_t* __restrict__ out)
{
    __shared__ uint64_t scratch[kChunkThreads / 64];
    const uint32_t d = blockIdx.x, r = map ? (uint32_t)map[d] : d;
    const ChunkPart* rp = part + (size_t)r * cp.G;
    const uint64_t top = row_top(rp, cp, scratch);
    if (p.greedy) {
        if (threadIdx.x == 0) out[d] = (int32_t)(0xffffffffu - (uint32_t)top);
        return;
    }
    const float* row = logits + (size_t)r * V;
    const float lmax = key_float((uint32_t)(top >> 32));
    const uint64_t km = kmin ? kmin[r] : 0;
    const int32_t t = chunk_draw(V, cp, uniforms[d],
                                 [&](uint32_t q) { return kept_e4(load4(row, V, q), q, lmax, km, p); }, rp, scratch);
    if (threadIdx.x == 0) out[d] = t;
}

// The bound (kmin: top-p, a large top_k, or both) of every row of a chunk
// launch, one workgroup per row; lmax from the row's chunk maxima.
__global__ __launch_bounds__(kRowThreads) void bound_rows_kernel(RowSrc rs, uint32_t V, ChunkPlan cp, WarpParams p,
                                                                 const ChunkPart* __restrict__ part,
                                                                 uint64_t* __restrict__ kmin)
{
    __shared__ uint64_t red[kRowThreads / 64];
    __shared__ ToppLds tps;
    const uint32_t r = blockIdx.x;
    const ChunkPart* rp = part + (size_t)r * cp.G;
    const uint64_t top = block_max_u64<kRowThreads>(threadIdx.x < cp.G ? rp[threadIdx.x].top : 0, red);
    uint64_t km, z;
    bool have_z;
    row_bound_select(rs.row(r, V), V, key_float((uint32_t)(top >> 32)), p, tps, red, km, z, have_z);
    if (threadIdx.x == 0) kmin[r] = km;
}

// ---- acceptance, full vocabulary or greedy -------------------------------------
// Chunk maxima (and sums) of all target rows then all draft rows; a one-wave
// walk per sequence runs the accept tests of decide_kernel on the row totals
// and leaves a plan for the final draw; the residual's chunk sums are taken
// only for a sequence that rejected; then one workgroup per sequence draws.
enum { kPlanDone = 0, kPlanResidual = 1, kPlanBonus = 2 };
struct AcceptPlan {
    int32_t mode, row, sh, pad;
    uint64_t Zp, Zq;
    uint64_t kp, kq;  // top-p bounds of the two rows (0: every token kept)
    float lpm, lqm;
};

// Row total and top from the row's chunk parts (one wave, G <= 64).
__device__ __forceinline__ void row_totals(const ChunkPart* rp, ChunkPlan cp, bool sums, uint64_t& top, uint64_t& Z)
{
    const int lane = threadIdx.x;
    top = wave_max_u64(lane < (int)cp.G ? rp[lane].top : 0);
    Z = sums ? wave_sum_u64(lane < (int)cp.G ? rp[lane].sum : 0) : 0;
}

__global__ __launch_bounds__(64) void accept_walk_kernel(const float* __restrict__ tl, const float* __restrict__ dl,
                                                         const int32_t* __restrict__ draft_tokens,
                                                         const float* __restrict__ uniforms, uint32_t k, uint32_t V,
                                                         ChunkPlan cp, WarpParams p,
                                                         const ChunkPart* __restrict__ part,
                                                         const uint64_t* __restrict__ kmin,
                                                         AcceptPlan* __restrict__ plan, int32_t* __restrict__ out,
                                                         int32_t* __restrict__ nacc)
{
    const uint32_t b = blockIdx.x, B = gridDim.x;
    const int lane = threadIdx.x;
    const int32_t* x = draft_tokens + (size_t)b * k;
    const float* u = p.greedy ? nullptr : uniforms + (size_t)b * (k + 1);
    int32_t* o = out + (size_t)b * (k + 1);
    const ChunkPart* tp = part + (size_t)b * (k + 1) * cp.G;
    const ChunkPart* dp = part + ((size_t)B * (k + 1) + (size_t)b * k) * cp.G;
    AcceptPlan pl = {};
    for (uint32_t i = lane; i <= k; i += 64) o[i] = -1;
    uint32_t i = 0;
    for (; i < k; ++i) {
        const int32_t xi = x[i];
        uint64_t topT, Zp;
        row_totals(tp + (size_t)i * cp.G, cp, !p.greedy, topT, Zp);
        if (p.greedy) {
            const int32_t a = (int32_t)(0xffffffffu - (uint32_t)topT);
            if (lane == 0) o[i] = a;
            if (a != xi) break;
            continue;
        }
        uint64_t topQ, Zq;
        row_totals(dp + (size_t)i * cp.G, cp, true, topQ, Zq);
        const float lpm = key_float((uint32_t)(topT >> 32)), lqm = key_float((uint32_t)(topQ >> 32));
        const bool in = xi >= 0 && (uint32_t)xi < V;
        const size_t rt = (size_t)b * (k + 1) + i, rd = (size_t)B * (k + 1) + (size_t)b * k + i;
        const uint64_t Px = in ? kept_e(tl[rt * V + xi], (uint32_t)xi, lpm, kmin ? kmin[rt] : 0, p) : 0;
        const uint64_t Qx = in ? kept_e(dl[((size_t)b * k + i) * V + xi], (uint32_t)xi, lqm, kmin ? kmin[rd] : 0, p) : 0;
        const double lhs = ((double)u[i] * (double)Qx) * (double)Zp;
        const double rhs = (double)Px * (double)Zq;
        if (lhs < rhs) {
            if (lane == 0) o[i] = xi;
            continue;
        }
        pl.mode = kPlanResidual;  // first rejection: draw from max(0, p - q)
        pl.row = (int32_t)i;
        pl.sh = 62 - bitlen64(Zp) - bitlen64(Zq);
        pl.Zp = Zp;
        pl.Zq = Zq;
        pl.kp = kmin ? kmin[rt] : 0;
        pl.kq = kmin ? kmin[rd] : 0;
        pl.lpm = lpm;
        pl.lqm = lqm;
        break;
    }
    if (i == k) {  // every draft accepted: bonus token from the target row k
        if (p.greedy) {
            uint64_t topT, Z;
            row_totals(tp + (size_t)k * cp.G, cp, false, topT, Z);
            if (lane == 0) o[k] = (int32_t)(0xffffffffu - (uint32_t)topT);
        } else {
            pl.mode = kPlanBonus;
            pl.row = (int32_t)k;
        }
    }
    if (lane == 0) {
        plan[b] = pl;
        nacc[b] = (int32_t)i;
    }
}

// Chunk sums of the residual max(0, P Zq - Q Zp) (scaled as in decide_kernel)
// of a sequence that rejected.
__device__ __forceinline__ W4 residual4(const float* trow, const float* drow, uint32_t V, uint32_t q,
                                        const AcceptPlan& pl, const WarpParams& p)
{
    const W4 a = kept_e4(load4(trow, V, q), q, pl.lpm, pl.kp, p), b = kept_e4(load4(drow, V, q), q, pl.lqm, pl.kq, p);
    return W4{residual_weight(a.a, b.a, pl.Zp, pl.Zq, pl.sh), residual_weight(a.b, b.b, pl.Zp, pl.Zq, pl.sh),
              residual_weight(a.c, b.c, pl.Zp, pl.Zq, pl.sh), residual_weight(a.d, b.d, pl.Zp, pl.Zq, pl.sh)};
}

__global__ __launch_bounds__(kChunkThreads) void residual_sum_kernel(const float* __restrict__ tl,
                                                                     const float* __restrict__ dl, uint32_t k,
                                                                     uint32_t V, ChunkPlan cp, WarpParams p,
                                                                     const AcceptPlan* __restrict__ plan,
                                                                     ChunkPart* __restrict__ rpart)
{
    __shared__ uint64_t scratch[kChunkThreads / 64];
    const uint32_t b = blockIdx.y, g = blockIdx.x, V4 = (V + 3) / 4;
    const AcceptPlan pl = plan[b];
    if (pl.mode != kPlanResidual) return;  // uniform
    const float* trow = tl + ((size_t)b * (k + 1) + pl.row) * V;
    const float* drow = dl + ((size_t)b * k + pl.row) * V;
    const uint32_t q1 = min(V4, (g + 1) * cp.CG);
    uint64_t sum = 0;
    int32_t last = -1;
    for (uint32_t q = g * cp.CG + threadIdx.x; q < q1; q += kChunkThreads) {
        const W4 w = residual4(trow, drow, V, q, pl, p);
        const uint64_t e[4] = {w.a, w.b, w.c, w.d};
#pragma unroll
        for (int c = 0; c < 4; ++c)
            if (4 * q + c < V && e[c]) {
                sum += e[c];
                last = (int32_t)(4 * q + c);
            }
    }
    sum = block_sum_u64<kChunkThreads>(sum, scratch);
    const uint64_t lastp = block_max_u64<kChunkThreads>((uint64_t)(int64_t)(last + 1), scratch);
    if (threadIdx.x == 0) {
        rpart[(size_t)b * cp.G + g].sum = sum;
        rpart[(size_t)b * cp.G + g].last = (int32_t)lastp - 1;
    }
}

// The final draw of each sequence: the residual (or, when it is all zero, the
// target row of the rejection) with u[k], or the bonus from target row k.
__global__ __launch_bounds__(kChunkThreads) void accept_pick_kernel(const float* __restrict__ tl,
                                                                    const float* __restrict__ dl,
                                                                    const float* __restrict__ uniforms, uint32_t k,
                                                                    uint32_t V, ChunkPlan cp, WarpParams p,
                                                                    const ChunkPart* __restrict__ part,
                                                                    const ChunkPart* __restrict__ rpart,
                                                                    const AcceptPlan* __restrict__ plan,
                                                                    const uint64_t* __restrict__ kmin,
                                                                    int32_t* __restrict__ out)
{
    __shared__ uint64_t scratch[kChunkThreads / 64];
    const uint32_t b = blockIdx.x;
    const AcceptPlan pl = plan[b];
    if (pl.mode == kPlanDone) return;  // uniform
    const float u = uniforms[(size_t)b * (k + 1) + k];
    const float* trow = tl + ((size_t)b * (k + 1) + pl.row) * V;
    const ChunkPart* rp = rpart + (size_t)b * cp.G;
    uint64_t SR = 0;
    if (pl.mode == kPlanResidual)
        SR = block_sum_u64<kChunkThreads>(threadIdx.x < cp.G ? rp[threadIdx.x].sum : 0, scratch);
    int32_t t;
    if (SR) {
        const float* drow = dl + ((size_t)b * k + pl.row) * V;
        t = chunk_draw(V, cp, u, [&](uint32_t q) { return residual4(trow, drow, V, q, pl, p); }, rp, scratch);
    } else {  // the bonus, or an all-zero residual: draw from the target row
        const ChunkPart* tp = part + ((size_t)b * (k + 1) + pl.row) * cp.G;
        const float lmax = key_float((uint32_t)(row_top(tp, cp, scratch) >> 32));
        const uint64_t km = kmin ? kmin[(size_t)b * (k + 1) + pl.row] : 0;
        t = chunk_draw(V, cp, u, [&](uint32_t q) { return kept_e4(load4(trow, V, q), q, lmax, km, p); }, tp, scratch);
    }
    if (threadIdx.x == 0) out[(size_t)b * (k + 1) + pl.row] = t;
}



// ---- top-k row statistics over chunk workgroups ---------------------------------
// As row_stats_kernel (same kept tokens), but the passes over the row run on
// G chunk workgroups: per-thread maximum keys of every chunk; the k-th
// largest of those G x 256 maxima (a lower bound of the k-th largest logit,
// radix-selected in one workgroup per row); the tokens at or above it
// collected by the chunks; one workgroup per row sorts the candidates (or,
// past kCandMax of them, runs the exact tie path of row_stats_kernel) and
// finishes the kept list.
struct TopkWs {
    RowStat* stats;   // [rows]
    ChunkPart* part;  // [rows][G] chunk maxima
    uint32_t* tm;     // [rows][G][kChunkThreads] per-thread maximum keys
    uint32_t* t0;     // [rows] candidate threshold
    uint32_t* cnt;    // [rows][kCntPad] candidates collected (one cache line per row: the atomics of
                      // different rows do not queue behind each other)
    uint64_t* cand;   // [rows][kCandMax]
};

inline size_t topk_align(size_t b) { return (b + 255) / 256 * 256; }
constexpr uint32_t kCntPad = 32;

inline size_t topk_ws_bytes(uint32_t rows)
{
    return topk_align((size_t)rows * sizeof(RowStat)) + topk_align((size_t)rows * kMaxChunks * sizeof(ChunkPart)) +
           topk_align((size_t)rows * kMaxChunks * kChunkThreads * 4) + topk_align((size_t)rows * 4) +
           topk_align((size_t)rows * kCntPad * 4) +
           (size_t)rows * kCandMax * 8;
}

inline TopkWs topk_ws(void* ws, uint32_t rows)
{
    uint8_t* b = (uint8_t*)ws;
    TopkWs w;
    w.stats = (RowStat*)b;
    b += topk_align((size_t)rows * sizeof(RowStat));
    w.part = (ChunkPart*)b;
    b += topk_align((size_t)rows * kMaxChunks * sizeof(ChunkPart));
    w.tm = (uint32_t*)b;
    b += topk_align((size_t)rows * kMaxChunks * kChunkThreads * 4);
    w.t0 = (uint32_t*)b;
    b += topk_align((size_t)rows * 4);
    w.cnt = (uint32_t*)b;
    b += topk_align((size_t)rows * kCntPad * 4);
    w.cand = (uint64_t*)b;
    return w;
}

// Leading per-thread maxima the scan keeps per wave when the candidate
// threshold comes from them (topk_m > 0): 4 G m distinct tokens per row, so
// the k-th largest of them is <= the row's k-th largest logit and the tokens
// at or above it include the top k (about k + k/5 of them at m = ceil(k / 4G)
// + 1 on N(0, 3^2) rows).  topk_m = 0: the radix-select threshold over all
// G x 256 per-thread maxima (topk_threshold_kernel), for rows of few chunks.
constexpr int kTopM = 8;
constexpr int kScanWaves = kChunkThreads / 64;

__host__ __device__ inline int topk_m(uint32_t k, uint32_t G)
{
    const uint32_t waves = kScanWaves * G;
    const uint32_t m = (k + waves - 1) / waves + 1;
    if (m <= (uint32_t)kTopM) return (int)m;
    return waves * kTopM >= k ? kTopM : 0;
}

// The row's kept per-wave maximum keys [G][kScanWaves][kTopM] (in the
// per-thread maxima region).
__device__ __forceinline__ uint32_t* topk_tops(const TopkWs& w, uint32_t r)
{
    return w.tm + (size_t)r * kMaxChunks * kScanWaves * kTopM;
}

__global__ __launch_bounds__(kChunkThreads) void topk_scan_kernel(RowSrc rs, uint32_t V, ChunkPlan cp, int m, TopkWs w)
{
    __shared__ uint64_t scratch[kChunkThreads / 64];
    const uint32_t r = blockIdx.y, g = blockIdx.x, V4 = (V + 3) / 4;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const float* row = rs.row(r, V);
    const uint32_t q1 = min(V4, (g + 1) * cp.CG);
    uint64_t best = 0;  // order key: the thread's largest key, lowest index among equals
    for (uint32_t q = g * cp.CG + threadIdx.x; q < q1; q += kChunkThreads) {
        const float4 v = load4(row, V, q);
        const float e[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int c = 0; c < 4; ++c)
            if (4 * q + c < V) {
                const uint64_t o = order_key(float_key(e[c]), 4 * q + c);
                best = o > best ? o : best;
            }
    }
    if (m == 0) {
        w.tm[((size_t)r * cp.G + g) * kChunkThreads + threadIdx.x] = (uint32_t)(best >> 32);  // 0: no token
    } else {
        // the wave's m largest per-thread maximum keys, strictly decreasing (so
        // from distinct tokens; a key equal to one taken is skipped; 0 = none)
        uint32_t* out = topk_tops(w, r) + ((size_t)g * kScanWaves + wave) * kTopM;
        const uint32_t bk = (uint32_t)(best >> 32);
        uint32_t prev = 0xffffffffu;
        for (int j = 0; j < m; ++j) {  // uniform
            const uint32_t v = wave_max_u32(bk < prev ? bk : 0u);
            if (lane == j) out[j] = v;
            prev = v;
        }
        if (g == 0 && threadIdx.x == 0) w.cnt[(size_t)r * kCntPad] = 0;
    }
    best = block_max_u64<kChunkThreads>(best, scratch);
    if (threadIdx.x == 0) w.part[(size_t)r * cp.G + g].top = best;
}

// Candidate threshold of each row (topk_m > 0), one workgroup per row: the
// largest kept key v with at least k kept keys >= v (they are keys of
// distinct tokens, so at least k tokens are >= v; 0 -- every token -- if
// there is none, and the finish then takes its exact fallback), and the
// row's max / argmax from the chunk maxima.
constexpr int kT0Threads = 256;
__global__ __launch_bounds__(kT0Threads) void topk_t0_kernel(ChunkPlan cp, int m, uint32_t k, TopkWs w)
{
    __shared__ uint32_t sv[kMaxChunks * kScanWaves * kTopM];
    __shared__ uint64_t scratch[kT0Threads / 64];
    const uint32_t r = blockIdx.x;
    const int n = (int)cp.G * kScanWaves * m;
    const uint32_t* tops = topk_tops(w, r);
    for (int i = threadIdx.x; i < n; i += kT0Threads) sv[i] = tops[(i / m) * kTopM + i % m];
    const uint64_t top =
        block_max_u64<kT0Threads>(threadIdx.x < cp.G ? w.part[(size_t)r * cp.G + threadIdx.x].top : 0, scratch);
    uint32_t thr = 0;
    for (int i = threadIdx.x; i < n; i += kT0Threads) {
        const uint32_t v = sv[i];
        if (!v) continue;
        uint32_t ge = 0;
        for (int j = 0; j < n; ++j) ge += sv[j] >= v;
        if (ge >= k && v > thr) thr = v;
    }
    thr = (uint32_t)block_max_u64<kT0Threads>(thr, scratch);
    if (threadIdx.x == 0) {
        RowStat* st = w.stats + r;
        st->lmax = key_float((uint32_t)(top >> 32));
        st->argmax = (int32_t)(0xffffffffu - (uint32_t)top);
        w.t0[r] = thr;
    }
}

// The k-th largest of the n values v[e] of thread t at index t + kRowThreads e
// (< n) in a kRowThreads workgroup: an 8-bit radix select, four histogram
// rounds (every thread calls it; the result in every thread).
template <int E>
__device__ uint32_t radix_kth_largest(const uint32_t (&v)[E], uint32_t n, uint32_t k)
{
    constexpr int NWV = kRowThreads / 64 * 4;
    __shared__ uint32_t whist[NWV][256];  // per (wave, lane & 3) histograms: most values share their top bytes
    __shared__ uint32_t hist[256];
    __shared__ uint32_t sel_bucket, sel_k;
    const int tid = threadIdx.x;
    uint32_t prefix = 0, mask = 0, kk = k;
    const int wv = (tid >> 6) * 4 + (tid & 3);
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int b = tid; b < NWV * 256; b += kRowThreads) (&whist[0][0])[b] = 0;
        __syncthreads();
#pragma unroll
        for (int e = 0; e < E; ++e)
            if (tid + kRowThreads * e < n && (v[e] & mask) == prefix) atomicAdd(&whist[wv][(v[e] >> shift) & 255u], 1u);
        __syncthreads();
        if (tid < 256) {
            uint32_t t = 0;
#pragma unroll
            for (int w2 = 0; w2 < NWV; ++w2) t += whist[w2][tid];
            hist[tid] = t;
        }
        __syncthreads();
        if (tid < 64) {  // the bucket holding the kk-th largest: lane l holds buckets 4l .. 4l+3
            const uint32_t h0 = hist[4 * tid], h1 = hist[4 * tid + 1], h2 = hist[4 * tid + 2], h3 = hist[4 * tid + 3];
            const uint32_t sl = h0 + h1 + h2 + h3;
            uint32_t suf = sl;  // sum over buckets >= 4l
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t t = __shfl_down(suf, o);
                if (tid + o < 64) suf += t;
            }
            const uint32_t above = suf - sl;
            if (above < kk && suf >= kk) {
                uint32_t c = above, b;
                if (c + h3 >= kk) {
                    b = 4 * tid + 3;
                } else if ((c += h3) + h2 >= kk) {
                    b = 4 * tid + 2;
                } else if ((c += h2) + h1 >= kk) {
                    b = 4 * tid + 1;
                } else {
                    c += h1;
                    b = 4 * tid;
                }
                sel_bucket = b;
                sel_k = kk - c;
            }
        }
        __syncthreads();
        prefix |= sel_bucket << shift;
        mask |= 255u << shift;
        kk = sel_k;
        __syncthreads();
    }
    return prefix;
}

// k-th largest of the row's G x 256 per-thread maxima; the row's max / argmax
// from the chunk maxima.
__global__ __launch_bounds__(kRowThreads) void topk_threshold_kernel(ChunkPlan cp, uint32_t k, TopkWs w)
{
    constexpr int E = kMaxChunks * kChunkThreads / kRowThreads;  // values per thread
    __shared__ uint64_t scratch[kRowThreads / 64];
    const uint32_t r = blockIdx.x, n = cp.G * kChunkThreads;
    const int tid = threadIdx.x;
    const uint32_t* tm = w.tm + (size_t)r * cp.G * kChunkThreads;
    uint32_t v[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {  // unconditional loads (clamped index), then masked: all in flight together
        const uint32_t i = tid + kRowThreads * e;
        v[e] = tm[min(i, n - 1)];
    }
#pragma unroll
    for (int e = 0; e < E; ++e)
        if (tid + kRowThreads * e >= n) v[e] = 0u;
    const uint32_t prefix = radix_kth_largest<E>(v, n, k);
    const uint64_t top = block_max_u64<kRowThreads>(tid < (int)cp.G ? w.part[(size_t)r * cp.G + tid].top : 0, scratch);
    if (tid == 0) {
        RowStat* st = w.stats + r;
        st->lmax = key_float((uint32_t)(top >> 32));
        st->argmax = (int32_t)(0xffffffffu - (uint32_t)top);
        w.t0[r] = prefix;
        w.cnt[(size_t)r * kCntPad] = 0;
    }
}

// Candidate threshold from a sample of the row (the sampled pipeline: sample,
// collect, finish), one workgroup per row: every F-th run of 64 float4
// groups (1 KB; a wave's load is one run, E per thread, all in flight) --
// 1 / F of the row, where the scan reads all of it.  Each wave keeps its m
// largest per-thread maximum keys (strictly decreasing, so of distinct
// tokens), and the threshold is the largest kept key with at least k kept
// keys at or above it: at least k tokens of the row reach it, so the tokens
// at or above it include the row's top k -- about F k of them on rows
// without heavy ties (past kCandMax the finish takes its exact path).  The
// row's max comes from the candidates in the finish.
__device__ __forceinline__ uint32_t sample_group(uint32_t j, uint32_t F) { return (j >> 6) * 64u * F + (j & 63u); }

template <int E>
__global__ __launch_bounds__(kRowThreads) void topk_sample_kernel(RowSrc rs, uint32_t V, uint32_t F, int m,
                                                                  uint32_t k, TopkWs w)
{
    constexpr int NT = kRowThreads, NWV = NT / 64;
    __shared__ __align__(16) uint32_t tops[NWV * kTopM];
    __shared__ uint64_t red[NWV];
    const uint32_t r = blockIdx.x, V4 = (V + 3) / 4;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float* row = rs.row(r, V);
    float4 x[E];
#pragma unroll
    for (int e = 0; e < E; ++e) x[e] = load4(row, V, min(sample_group(tid + NT * e, F), V4 - 1));
    uint32_t bk = 0;  // the thread's largest sampled key (0: none)
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const uint32_t q = sample_group(tid + NT * e, F);
        const float f[4] = {x[e].x, x[e].y, x[e].z, x[e].w};
#pragma unroll
        for (int c = 0; c < 4; ++c)
            if (q < V4 && 4 * q + c < V) bk = max(bk, float_key(f[c]));
    }
    uint32_t prev = 0xffffffffu;
    for (int j = 0; j < m; ++j) {  // uniform
        const uint32_t t = wave_max_u32(bk < prev ? bk : 0u);
        if (lane == j) tops[wave * m + j] = t;
        prev = t;
    }
    __syncthreads();
    const int n = NWV * m;
    uint32_t thr = 0;
    if (tid < n) {
        const uint32_t tv = tops[tid];
        if (tv && count_ge(tops, n, tv) >= k) thr = tv;
    }
    thr = (uint32_t)block_max_u64<NT>(thr, red);  // 0 (no bound): every token, then the exact path
    if (tid == 0) {
        w.t0[r] = thr;
        w.cnt[(size_t)r * kCntPad] = 0;
    }
}

// Sample fraction 1 / F of the sampled pipeline for top-k k (about F k
// candidates: F = 8 up to k = 64, 4 up to 128) and the sample kernel's
// float4 groups per thread (a power of two <= 8: 32 keys per thread, within
// the registers of a 1024-thread workgroup); 0 where it does not apply.
inline uint32_t topk_sample_F(uint32_t k) { return k <= 64 ? 8u : (k <= 128 ? 4u : 0u); }
inline int topk_sample_E(uint32_t V, uint32_t F)
{
    const uint32_t runs = ((V + 3) / 4 + 63) / 64, ng = (runs + F - 1) / F * 64;  // sampled float4 groups
    const uint32_t per = (ng + kRowThreads - 1) / kRowThreads;
    int e = 1;
    while ((uint32_t)e < per) e <<= 1;
    return e <= 8 ? e : 0;
}

// Tokens with logit key >= the row's threshold into its candidate list: per
// pass, kCollectU float4 groups per thread (all loads in flight); each
// wave's candidates go to a list of the workgroup in LDS (one LDS slot
// reservation per wave and pass), and the workgroup reserves its range of
// the row's list with one device atomic at its end -- a wave never waits on
// a device atomic between its loads (with ~F k candidates per row nearly
// every wave holds one).  Past kCandMax candidates only the count matters
// (the finish then takes its exact path).
constexpr int kCollectU = 4;
__global__ __launch_bounds__(kChunkThreads) void topk_collect_kernel(RowSrc rs, uint32_t V, ChunkPlan cp, TopkWs w)
{
    __shared__ uint64_t lc[kCandMax];
    __shared__ uint32_t ln, lbase;
    const uint32_t r = blockIdx.y, g = blockIdx.x, V4 = (V + 3) / 4;
    const float* row = rs.row(r, V);
    const uint32_t thr = w.t0[r], q1 = min(V4, (g + 1) * cp.CG);
    const int lane = threadIdx.x & 63;
    if (threadIdx.x == 0) ln = 0;
    __syncthreads();
    for (uint32_t qb = g * cp.CG; qb < q1; qb += kChunkThreads * kCollectU) {  // uniform
        float4 v[kCollectU];
#pragma unroll
        for (int u = 0; u < kCollectU; ++u) v[u] = load4(row, V, min(qb + threadIdx.x + u * kChunkThreads, V4 - 1));
        uint32_t key[kCollectU][4], n = 0;
#pragma unroll
        for (int u = 0; u < kCollectU; ++u) {
            const uint32_t q = qb + threadIdx.x + u * kChunkThreads;
            const float e[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                key[u][c] = float_key(e[c]);
                n += q < q1 && 4 * q + c < V && key[u][c] >= thr;
            }
        }
        // one LDS slot reservation per wave: exclusive prefix of the lanes' counts
        const uint32_t incl = wave_scan_incl(n, OpAdd{});
        const uint32_t total = lane63_u32(incl);
        if (!total) continue;  // uniform in the wave
        uint32_t base = 0;
        if (lane == 0) base = atomicAdd(&ln, total);
        base = (uint32_t)__builtin_amdgcn_readfirstlane((int)base);
        uint32_t slot = base + incl - n;
#pragma unroll
        for (int u = 0; u < kCollectU; ++u) {
            const uint32_t q = qb + threadIdx.x + u * kChunkThreads;
#pragma unroll
            for (int c = 0; c < 4; ++c)
                if (q < q1 && 4 * q + c < V && key[u][c] >= thr) {
                    if (slot < (uint32_t)kCandMax) lc[slot] = order_key(key[u][c], 4 * q + c);
                    ++slot;
                }
        }
    }
    __syncthreads();
    const uint32_t n = ln;
    if (!n) return;  // uniform
    if (threadIdx.x == 0) lbase = atomicAdd(&w.cnt[(size_t)r * kCntPad], n);
    __syncthreads();
    const uint32_t base = lbase, nl = min(n, (uint32_t)kCandMax);
    for (uint32_t i = threadIdx.x; i < nl && base + i < (uint32_t)kCandMax; i += kChunkThreads)
        w.cand[(size_t)r * kCandMax + base + i] = lc[i];
}

__global__ __launch_bounds__(kRowThreads) void topk_finish_kernel(RowSrc rs, uint32_t V, WarpParams p, TopkWs w)
{
    __shared__ uint64_t red[kRowThreads / 64];
    __shared__ uint64_t buf[kCandMax];
    __shared__ uint32_t cand_count;
    __shared__ uint64_t keptE[kKMax];
    const uint32_t r = blockIdx.x, k = p.top_k;
    RowStat* st = w.stats + r;
    const uint64_t* c = w.cand + (size_t)r * kCandMax;
    // the first kRankMax slots load beside the count, not behind it (slots
    // past the count hold stale keys that the ranking never reads)
    static_assert(kRankMax <= kRowThreads, "one candidate slot per thread");
    const uint64_t pre = threadIdx.x < kRankMax ? c[threadIdx.x] : 0;
    const uint32_t nc = w.cnt[(size_t)r * kCntPad];
    if (nc <= (uint32_t)kRankMax) {  // few candidates (the usual case): places by counting
        __shared__ uint64_t cs[kRankMax];
        if (threadIdx.x < kRankMax) cs[threadIdx.x] = pre;
        __syncthreads();
        rank_top_desc(cs, (int)nc, k, buf);
    } else if (nc <= (uint32_t)kCandMax) {
        int n2 = 1;
        while (n2 < (int)nc) n2 <<= 1;
        for (int i = threadIdx.x; i < n2; i += kRowThreads) buf[i] = i < (int)nc ? c[i] : 0;
        bitonic_desc(buf, n2);
    } else {
        topk_tie_fallback<kRowThreads>(rs.row(r, V), V, k, buf, red, cand_count);
    }
    __syncthreads();
    // buf holds the top k in descending (logit, then lowest index) order: its
    // first entry is the row's maximum and argmax (the same as the chunk
    // maxima give, which the sampled pipeline does not compute)
    const float lmax = key_float((uint32_t)(buf[0] >> 32));
    if (threadIdx.x == 0) {
        st->lmax = lmax;
        st->argmax = (int32_t)(0xffffffffu - (uint32_t)buf[0]);
    }
    finish_topk(buf, k, lmax, p, st, keptE, cand_count);
}

// A row's whole top-k statistics in one workgroup, for rows that fit in its
// registers (V <= kRowFusedV) and a k that the 16 waves' kept maxima cover
// (topk_m > 0): the row is read once (every load in flight), each wave keeps
// its m largest per-thread maximum keys, the candidate threshold is the
// largest kept key with at least k kept keys at or above it, the tokens at or
// above it go from registers into an LDS list, and topk_finish_kernel's finish
// runs on that list.  The threshold only bounds the candidates (the kept set
// is the exact top k whatever it is), so the statistics equal those of the
// scan / threshold / collect / finish launches.
// NT = 1024, or 512 (twice the groups per thread) so that two workgroups
// share a CU (at most 128 registers) when there are more rows than CUs.
constexpr int kRowF4 = 8;  // float4 groups per thread at kRowThreads
constexpr uint32_t kRowFusedV = 4u * kRowF4 * kRowThreads;

template <int NT>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(4))) void topk_row_kernel(RowSrc rs, uint32_t V,
                                                                                             WarpParams p, int m,
                                                                                             TopkWs w)
{
    constexpr int NWV = NT / 64, F4 = kRowF4 * kRowThreads / NT;
    __shared__ uint64_t red[NWV];
    __shared__ uint64_t buf[kCandMax];
    __shared__ uint64_t cand[kCandMax + 64];  // + a spare entry per lane (below)
    __shared__ __align__(16) uint32_t tops[NWV * kTopM];
    __shared__ uint32_t cand_count;
    __shared__ uint64_t keptE[kKMax];
    const uint32_t r = blockIdx.x, k = p.top_k, V4 = (V + 3) / 4;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float* row = rs.row(r, V);
    float4 v[F4];
#pragma unroll
    for (int i = 0; i < F4; ++i) v[i] = load4(row, V, min((uint32_t)(tid + i * NT), V4 - 1));
    uint64_t best = 0;  // order key: the thread's largest key, lowest index among equals
#pragma unroll
    for (int i = 0; i < F4; ++i) {
        const uint32_t q = tid + i * NT;
        const float e[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
        for (int c = 0; c < 4; ++c)
            if (q < V4 && 4 * q + c < V) {
                const uint64_t o = order_key(float_key(e[c]), 4 * q + c);
                best = o > best ? o : best;
            }
    }
    // the wave's m largest per-thread maximum keys, strictly decreasing (so
    // from distinct tokens; 0 = none)
    const uint32_t bk = (uint32_t)(best >> 32);
    uint32_t prev = 0xffffffffu;
    for (int j = 0; j < m; ++j) {  // uniform
        const uint32_t t = wave_max_u32(bk < prev ? bk : 0u);
        if (lane == j) tops[wave * m + j] = t;  // packed: the n = NWV m kept keys in a row
        prev = t;
    }
    if (tid == 0) cand_count = 0;
    const uint64_t top = block_max_u64<NT>(best, red);  // its barriers publish tops and cand_count
    const int n = NWV * m;
    uint32_t thr = 0;
    if (tid < n) {
        const uint32_t tv = tops[tid];
        if (tv && count_ge(tops, n, tv) >= k) thr = tv;
    }
    thr = (uint32_t)block_max_u64<NT>(thr, red);  // 0 (no bound): every token, then the fallback
    // this thread's candidates (bit 4 i + c: element 4 (tid + i NT) + c),
    // written at slots reserved with one LDS atomic per wave (a wave prefix
    // sum of the counts), not one dependent atomic per candidate.  Both
    // loops are branch-free: every lane of a wave holding a candidate stores
    // every element, the others into the lane's spare entry past kCandMax
    // (unrolled with a branch per element, the loops took ~4 us).
    using Mask = std::conditional_t<(4 * F4 > 32), uint64_t, uint32_t>;
    Mask cm = 0;
#pragma unroll
    for (int i = 0; i < F4; ++i) {
        const uint32_t q = tid + i * NT;
        const float e[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
        for (int c = 0; c < 4; ++c)
            cm |= (Mask)((q < V4) & (4 * q + c < V) & (float_key(e[c]) >= thr)) << (4 * i + c);
    }
    const uint32_t cnt = (uint32_t)__builtin_popcountll((unsigned long long)cm);
    const uint32_t incl = wave_scan_incl(cnt, OpAdd{});
    const uint32_t wtot = lane63_u32(incl);
    if (wtot) {  // uniform
        uint32_t base = 0;
        if (lane == 63) base = atomicAdd(&cand_count, wtot);
        uint32_t slot = lane63_u32(base) + incl - cnt;
#pragma unroll
        for (int i = 0; i < F4; ++i) {
            const uint32_t q = tid + i * NT;
            const float e[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const uint32_t ok = (uint32_t)(cm >> (4 * i + c)) & 1u;
                cand[ok && slot < (uint32_t)kCandMax ? slot : kCandMax + lane] = order_key(float_key(e[c]), 4 * q + c);
                slot += ok;
            }
        }
    }
    __syncthreads();
    const uint32_t nc = cand_count;
    if (nc <= (uint32_t)kRankMax) {
        rank_top_desc(cand, (int)nc, k, buf);
    } else if (nc <= (uint32_t)kCandMax) {
        int n2 = 1;
        while (n2 < (int)nc) n2 <<= 1;
        for (int i = tid; i < n2; i += NT) buf[i] = i < (int)nc ? cand[i] : 0;
        bitonic_desc(buf, n2);
    } else {
        topk_tie_fallback<NT>(row, V, k, buf, red, cand_count);
    }
    RowStat* st = w.stats + r;
    const float lmax = key_float((uint32_t)(top >> 32));
    if (tid == 0) {
        st->lmax = lmax;
        st->argmax = (int32_t)(0xffffffffu - (uint32_t)top);
    }
    finish_topk(buf, k, lmax, p, st, keptE, cand_count);
}

// The one-workgroup-per-row kernel while the rows fit one round of 1024-
// thread workgroups (one row per CU); past that the sampled chunk pipeline
// (top_k <= 128), else the 512-thread one-workgroup kernel up to two rows per
// CU, else the scanned chunk pipeline.  route (ULSPEC_OPT_TOPK_ROUTE) forces
// one of the four where it applies.
void launch_topk_stats(hipStream_t s, RowSrc rs, uint32_t rows, uint32_t V, const WarpParams& p, const TopkWs& w,
                       int n_cu, int route)
{
    const uint32_t cus = (uint32_t)std::max(1, n_cu);
    const int m16 = topk_m(p.top_k, 16 / kScanWaves), m8 = topk_m(p.top_k, 8 / kScanWaves);  // kept keys per wave
    const bool fits16 = V <= kRowFusedV && m16 > 0, fits8 = V <= kRowFusedV && m8 > 0;
    if (fits16 && (route == 1 || (route == 0 && rows <= cus))) {
        hipLaunchKernelGGL(topk_row_kernel<1024>, dim3(rows), dim3(1024), 0, s, rs, V, p, m16, w);
        return;
    }
    const uint32_t F = topk_sample_F(p.top_k);
    const int E = F ? topk_sample_E(V, F) : 0;
    // up to two rows per CU the sampled pipeline beats the 512-thread
    // one-workgroup kernel too (k=8, V=32000, 272 rows: 40.1 against 41.4 us)
    if (fits8 && (route == 2 || (route == 0 && rows <= 2 * cus && !E))) {
        hipLaunchKernelGGL(topk_row_kernel<512>, dim3(rows), dim3(512), 0, s, rs, V, p, m8, w);
        return;
    }
    const ChunkPlan cp = chunk_plan(V);
    const dim3 grid(cp.G, rows), blk(kChunkThreads);
    if (E && route != 3) {  // the sampled pipeline: 1 / F of the row, then one pass (route 3: the scan)
        const dim3 g1(rows), b1(kRowThreads);
        // kept keys per wave of 16: two more than an even share of k (fewer
        // waves' leading maxima cut off, so a threshold closer to the
        // sample's k-th largest and fewer candidates), at most kTopM
        const int ms = (int)std::min<uint32_t>(kTopM, (p.top_k + 15) / 16 + 2);
        switch (E) {
        case 1: hipLaunchKernelGGL(topk_sample_kernel<1>, g1, b1, 0, s, rs, V, F, ms, p.top_k, w); break;
        case 2: hipLaunchKernelGGL(topk_sample_kernel<2>, g1, b1, 0, s, rs, V, F, ms, p.top_k, w); break;
        case 4: hipLaunchKernelGGL(topk_sample_kernel<4>, g1, b1, 0, s, rs, V, F, ms, p.top_k, w); break;
        default: hipLaunchKernelGGL(topk_sample_kernel<8>, g1, b1, 0, s, rs, V, F, ms, p.top_k, w); break;
        }
        // the collect in chunks of one pass (kCollectU float4 groups per thread)
        const uint32_t V4 = (V + 3) / 4, CGc = std::min<uint32_t>(kChunkThreads * kCollectU,
                                                                  (V4 + kChunkThreads - 1) / kChunkThreads * kChunkThreads);
        const ChunkPlan cpc{(V4 + CGc - 1) / CGc, CGc};
        hipLaunchKernelGGL(topk_collect_kernel, dim3(cpc.G, rows), blk, 0, s, rs, V, cpc, w);
        hipLaunchKernelGGL(topk_finish_kernel, dim3(rows), dim3(kRowThreads), 0, s, rs, V, p, w);
        return;
    }
    const int m = topk_m(p.top_k, cp.G);
    hipLaunchKernelGGL(topk_scan_kernel, grid, blk, 0, s, rs, V, cp, m, w);
    if (m == 0) hipLaunchKernelGGL(topk_threshold_kernel, dim3(rows), dim3(kRowThreads), 0, s, cp, p.top_k, w);
    else hipLaunchKernelGGL(topk_t0_kernel, dim3(rows), dim3(kT0Threads), 0, s, cp, m, p.top_k, w);
    hipLaunchKernelGGL(topk_collect_kernel, grid, blk, 0, s, rs, V, cp, w);
    hipLaunchKernelGGL(topk_finish_kernel, dim3(rows), dim3(kRowThreads), 0, s, rs, V, p, w);
}

__global__ void uniforms_kernel(uint64_t seed, uint64_t idx0, uint32_t n, float* __restrict__ out)
{
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = counter_uniform(seed, idx0 + i);
}

ulspec_status make_params(ulspec_ctx* ctx, const ulspec_sampling* s, uint32_t V, WarpParams& p)
{
    if (!s) return fail(ctx, ULSPEC_EINVAL, "sampling parameters are null");
    p.greedy = s->greedy != 0;
    p.top_k = s->top_k;
    p.top_p = s->top_p;
    p.invT = 1.0f;
    p.scale = __builtin_ldexpf(1.0f, warp_shift(V));
    p.pad = 0;
    if (V > (uint32_t)(kMaxRounds * 4 * kSeqThreads))
        return fail(ctx, ULSPEC_EUNSUPPORTED, "vocabulary %u > %d", V, kMaxRounds * 4 * kSeqThreads);
    if (p.greedy) return ULSPEC_OK;
    if (!(s->temperature > 0.0f) || !(s->temperature < __builtin_inff()))
        return fail(ctx, ULSPEC_EINVAL, "temperature must be positive and finite (got %g)", (double)s->temperature);
    if (!(s->top_p == s->top_p)) return fail(ctx, ULSPEC_EINVAL, "top_p is NaN");
    p.invT = 1.0f / s->temperature;
    return ULSPEC_OK;
}

}  // namespace

namespace ulspec {

size_t accept_workspace_bytes(uint32_t B, uint32_t k)
{
    const size_t stats = topk_ws_bytes(B * (k + 1) + B * k);
    const size_t chunks = (size_t)(B * (k + 1) + B * k + B) * kMaxChunks * sizeof(ChunkPart) +
                          B * sizeof(AcceptPlan) + (size_t)(B * (k + 1) + B * k) * sizeof(uint64_t);
    return std::max(stats, chunks);
}

size_t sample_workspace_bytes(uint32_t R)
{
    return std::max((size_t)R * (kMaxChunks * sizeof(ChunkPart) + sizeof(uint64_t)), topk_ws_bytes(R));
}

ulspec_status accept_launch(ulspec_ctx* ctx, const ulspec_sampling* s, uint32_t B, uint32_t k, uint32_t V,
                            const float* target_logits, const float* draft_logits, const int32_t* draft_tokens,
                            const float* uniforms, int32_t* out_tokens, int32_t* out_n_accepted, void* ws)
{
    WarpParams p;
    ulspec_status st = make_params(ctx, s, V, p);
    if (st != ULSPEC_OK) return st;
    if (B == 0 || k == 0 || k > 16 || V == 0)
        return fail(ctx, ULSPEC_EINVAL, "accept: need B >= 1, 1 <= k <= 16, V >= 1 (B=%u k=%u V=%u)", B, k, V);
    if (!target_logits || !draft_tokens || !out_tokens || !out_n_accepted)
        return fail(ctx, ULSPEC_EINVAL, "accept: null device pointer");
    if (!p.greedy && (!draft_logits || !uniforms))
        return fail(ctx, ULSPEC_EINVAL, "accept: sampling needs draft logits and uniforms");
    const uint32_t rows_t = B * (k + 1), rows_d = p.greedy ? 0 : B * k;
    if ((uint64_t)B * (2 * k + 1) > kMaxGridRows)
        return fail(ctx, ULSPEC_EUNSUPPORTED, "accept: B (2k+1) = %llu logit rows (at most %u per call)",
                    (unsigned long long)B * (2 * k + 1), kMaxGridRows);
    if (!ws) {
        st = workspace(ctx, accept_workspace_bytes(B, k), &ws);
        if (st != ULSPEC_OK) return st;
    }
    if (p.greedy || !list_topk(p, V)) {
        const ChunkPlan cp = chunk_plan(V);
        ChunkPart* part = (ChunkPart*)ws;  // [rows_t + rows_d][G]
        ChunkPart* rpart = part + (size_t)(rows_t + rows_d) * cp.G;  // [B][G]
        AcceptPlan* plan = (AcceptPlan*)(rpart + (size_t)B * cp.G);
        const bool bounded = row_bound(p, V);
        uint64_t* kmin = bounded ? (uint64_t*)(plan + B) : nullptr;  // [rows_t + rows_d]
        const RowSrc rs{target_logits, rows_t, draft_logits};
        const dim3 grid(cp.G, rows_t + rows_d), blk(kChunkThreads);
        hipLaunchKernelGGL(chunk_max_kernel, grid, blk, 0, ctx->stream, rs, V, cp, part);
        if (bounded)
            hipLaunchKernelGGL(bound_rows_kernel, dim3(rows_t + rows_d), dim3(kRowThreads), 0, ctx->stream, rs, V, cp,
                               p, (const ChunkPart*)part, kmin);
        if (!p.greedy)
            hipLaunchKernelGGL(chunk_sum_kernel, grid, blk, 0, ctx->stream, rs, V, cp, p, (const uint64_t*)kmin, part);
        hipLaunchKernelGGL(accept_walk_kernel, dim3(B), dim3(64), 0, ctx->stream, target_logits, draft_logits,
                           draft_tokens, uniforms, k, V, cp, p, (const ChunkPart*)part, (const uint64_t*)kmin, plan,
                           out_tokens, out_n_accepted);
        if (!p.greedy) {
            hipLaunchKernelGGL(residual_sum_kernel, dim3(cp.G, B), blk, 0, ctx->stream, target_logits, draft_logits, k,
                               V, cp, p, (const AcceptPlan*)plan, rpart);
            hipLaunchKernelGGL(accept_pick_kernel, dim3(B), blk, 0, ctx->stream, target_logits, draft_logits, uniforms,
                               k, V, cp, p, (const ChunkPart*)part, (const ChunkPart*)rpart, (const AcceptPlan*)plan,
                               (const uint64_t*)kmin, out_tokens);
        }
        return check_launch(ctx, "accept launch");
    }
    const TopkWs tw = topk_ws(ws, rows_t + rows_d);
    RowStat* stats = tw.stats;
    launch_topk_stats(ctx->stream, RowSrc{target_logits, rows_t, draft_logits}, rows_t + rows_d, V, p, tw,
                      ctx->n_cu, ctx->topk_route);
    hipLaunchKernelGGL(decide_kernel, dim3(B), dim3(kSeqThreads), decide_lds_bytes(k, p.top_k), ctx->stream,
                       (const RowStat*)stats, draft_tokens, uniforms, k, p.top_k, V, out_tokens, out_n_accepted);
    return check_launch(ctx, "accept launch");
}

size_t accept_tree_workspace_bytes(uint32_t B, uint32_t n) { return (size_t)2 * B * n * sizeof(RowStat); }

ulspec_status accept_tree_launch(ulspec_ctx* ctx, const ulspec_sampling* s, uint32_t B, uint32_t n, uint32_t V,
                                 const int32_t* parent, const float* target_logits, const float* draft_logits,
                                 const int32_t* tokens, const float* uniforms, int32_t* out_tokens,
                                 int32_t* out_path, int32_t* out_n_accepted, void* ws)
{
    WarpParams p;
    ulspec_status st = make_params(ctx, s, V, p);
    if (st != ULSPEC_OK) return st;
    if (B == 0 || n == 0 || n > (uint32_t)kTreeMax || V == 0)
        return fail(ctx, ULSPEC_EINVAL, "accept_tree: need B >= 1, 1 <= n <= %d, V >= 1 (B=%u n=%u V=%u)", kTreeMax,
                    B, n, V);
    if (!parent) return fail(ctx, ULSPEC_EINVAL, "accept_tree: parent (host array) is null");
    if (!target_logits || !tokens || !out_tokens || !out_path || !out_n_accepted)
        return fail(ctx, ULSPEC_EINVAL, "accept_tree: null device pointer");
    if (!p.greedy && (!draft_logits || !uniforms))
        return fail(ctx, ULSPEC_EINVAL, "accept_tree: sampling needs draft logits and uniforms");
    TreeShape shape{};
    shape.n = (int32_t)n;
    RowSel inner{};  // nodes with children: their draft rows are read
    bool has_kids[kTreeMax] = {};
    for (uint32_t i = 0; i < n; ++i) {
        const int32_t pi = parent[i];
        if (i == 0 ? pi != -1 : (pi < 0 || pi >= (int32_t)i))
            return fail(ctx, ULSPEC_EINVAL, "accept_tree: parent[%u]=%d (need parent[0] = -1, parent[i] in [0, i))", i,
                        pi);
        shape.parent[i] = pi;
        if (i) has_kids[pi] = true;
    }
    inner.n_rows = n;
    for (uint32_t i = 0; i < n; ++i)
        if (has_kids[i]) inner.row[inner.n_sel++] = (int32_t)i;
    if (!ws) {
        st = workspace(ctx, accept_tree_workspace_bytes(B, n), &ws);
        if (st != ULSPEC_OK) return st;
    }
    RowStat* stats = (RowStat*)ws;
    hipLaunchKernelGGL(row_stats_kernel, dim3(B * n), dim3(kRowThreads), 0, ctx->stream, target_logits, V, p, stats,
                       RowSel{});
    if (!p.greedy && inner.n_sel)
        hipLaunchKernelGGL(row_stats_kernel, dim3(B * inner.n_sel), dim3(kRowThreads), 0, ctx->stream, draft_logits,
                           V, p, stats + (size_t)B * n, inner);
    hipLaunchKernelGGL(decide_tree_kernel, dim3(B), dim3(kSeqThreads), 0, ctx->stream, stats, target_logits,
                       draft_logits, tokens, uniforms, V, p, shape, out_tokens, out_path, out_n_accepted);
    return check_launch(ctx, "accept_tree launch");
}

ulspec_status sample_launch(ulspec_ctx* ctx, const ulspec_sampling* s, uint32_t R, uint32_t V, const float* logits,
                            const float* uniforms, int32_t* out_tokens, void* ws)
{
    return sample_mapped_launch(ctx, s, R, V, logits, R, nullptr, uniforms, out_tokens, ws);
}

ulspec_status sample_mapped_launch(ulspec_ctx* ctx, const ulspec_sampling* s, uint32_t R, uint32_t V,
                                   const float* logits, uint32_t D, const int32_t* map, const float* uniforms,
                                   int32_t* out_tokens, void* ws)
{
    WarpParams p;
    ulspec_status st = make_params(ctx, s, V, p);
    if (st != ULSPEC_OK) return st;
    if (R == 0 || V == 0) return fail(ctx, ULSPEC_EINVAL, "sample: need R >= 1 and V >= 1");
    if (R > kMaxGridRows || D > kMaxGridRows)
        return fail(ctx, ULSPEC_EUNSUPPORTED, "sample: R=%u rows, %u draws (at most %u per call)", R, D, kMaxGridRows);
    if (D == 0 || (!map && D != R)) return fail(ctx, ULSPEC_EINVAL, "sample: %u draws from %u rows", D, R);
    if (!logits || !out_tokens || (!p.greedy && !uniforms)) return fail(ctx, ULSPEC_EINVAL, "sample: null pointer");
    if (!ws) {
        st = workspace(ctx, sample_workspace_bytes(R), &ws);
        if (st != ULSPEC_OK) return st;
    }
    if (p.greedy || !list_topk(p, V)) {
        const ChunkPlan cp = chunk_plan(V);
        ChunkPart* part = (ChunkPart*)ws;
        const bool bounded = row_bound(p, V);
        uint64_t* kmin = bounded ? (uint64_t*)(part + (size_t)R * cp.G) : nullptr;  // [R]
        const RowSrc rs{logits, R, nullptr};
        hipLaunchKernelGGL(chunk_max_kernel, dim3(cp.G, R), dim3(kChunkThreads), 0, ctx->stream, rs, V, cp, part);
        if (bounded)
            hipLaunchKernelGGL(bound_rows_kernel, dim3(R), dim3(kRowThreads), 0, ctx->stream, rs, V, cp, p,
                               (const ChunkPart*)part, kmin);
        if (!p.greedy)
            hipLaunchKernelGGL(chunk_sum_kernel, dim3(cp.G, R), dim3(kChunkThreads), 0, ctx->stream, rs, V, cp, p,
                               (const uint64_t*)kmin, part);
        hipLaunchKernelGGL(chunk_pick_kernel, dim3(D), dim3(kChunkThreads), 0, ctx->stream, logits, uniforms, V, cp,
                           p, (const ChunkPart*)part, (const uint64_t*)kmin, map, out_tokens);
        return check_launch(ctx, "sample launch");
    }
    const TopkWs tw = topk_ws(ws, R);
    launch_topk_stats(ctx->stream, RowSrc{logits, R, nullptr}, R, V, p, tw, ctx->n_cu, ctx->topk_route);
    hipLaunchKernelGGL(sample_kernel, dim3(D), dim3(kSeqThreads), 0, ctx->stream, (const RowStat*)tw.stats, uniforms,
                       V, map, out_tokens);
    return check_launch(ctx, "sample launch");
}

}  // namespace ulspec

namespace ulspec {
void topb_launch(ulspec_ctx* ctx, const float* logits, uint32_t V, uint32_t rows, const int32_t* first_kid,
                 const int32_t* n_kids, int32_t* out_tokens)
{
    hipLaunchKernelGGL(topb_kernel, dim3(rows), dim3(kRowThreads), 0, ctx->stream, logits, V, first_kid, n_kids,
                       out_tokens);
}
}  // namespace ulspec

extern "C" ulspec_status ulspec_accept(ulspec_ctx* ctx, const ulspec_sampling* s, uint32_t B, uint32_t k,
                                       uint32_t V, const float* target_logits, const float* draft_logits,
                                       const int32_t* draft_tokens, const float* uniforms, int32_t* out_tokens,
                                       int32_t* out_n_accepted)
{
    ULSPEC_CHECK_CTX(ctx);
    (void)hipSetDevice(ctx->device);
    return accept_launch(ctx, s, B, k, V, target_logits, draft_logits, draft_tokens, uniforms, out_tokens,
                         out_n_accepted, nullptr);
}

// Scratch of the no-allocation entry point, one copy per GPU.  In host code
// `noalloc_scratch` names a host-side stand-in, not device memory: kernels
// get the address hipGetSymbolAddress returns for the context's device
// (accept_init, at context creation).
static __device__ __align__(256) uint8_t noalloc_scratch[ULSPEC_ACCEPT_NOALLOC_SCRATCH];

namespace ulspec {
ulspec_status accept_init(ulspec_ctx* ctx)
{
    // decide_kernel's staged lists reach (2 kMaxK + 1) kKMax (8 + 4) bytes
    hipError_t ea = hipFuncSetAttribute((const void*)decide_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                        (int)decide_lds_bytes(kMaxK, kKMax));
    if (ea != hipSuccess) return hip_fail(ctx, ea, "hipFuncSetAttribute(decide_kernel)");
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(noalloc_scratch));
    if (e != hipSuccess || !p) return hip_fail(ctx, e, "hipGetSymbolAddress(accept scratch)");
    ctx->noalloc_scratch = p;
    return ULSPEC_OK;
}
}  // namespace ulspec

extern "C" ulspec_status ulspec_accept_noalloc(ulspec_ctx* ctx, const ulspec_sampling* s, uint32_t B, uint32_t k,
                                               uint32_t V, const float* target_logits, const float* draft_logits,
                                               const int32_t* draft_tokens, const float* uniforms,
                                               int32_t* out_tokens, int32_t* out_n_accepted)
{
    ULSPEC_CHECK_CTX(ctx);
    if (!ctx->noalloc_scratch) return fail(ctx, ULSPEC_EDEVICE, "accept_noalloc: scratch address not set");
    if (B == 0 || k == 0 || k > 16)
        return fail(ctx, ULSPEC_EINVAL, "accept_noalloc: need B >= 1, 1 <= k <= 16 (B=%u k=%u)", B, k);
    const size_t need = accept_workspace_bytes(B, k);
    if (need > ULSPEC_ACCEPT_NOALLOC_SCRATCH)
        return fail(ctx, ULSPEC_EUNSUPPORTED, "accept_noalloc: %zu bytes of scratch needed, %u available", need,
                    ULSPEC_ACCEPT_NOALLOC_SCRATCH);
    (void)hipSetDevice(ctx->device);
    return accept_launch(ctx, s, B, k, V, target_logits, draft_logits, draft_tokens, uniforms, out_tokens,
                         out_n_accepted, ctx->noalloc_scratch);
}

extern "C" ulspec_status ulspec_accept_tree(ulspec_ctx* ctx, const ulspec_sampling* s, uint32_t B, uint32_t n,
                                            uint32_t V, const int32_t* parent, const float* target_logits,
                                            const float* draft_logits, const int32_t* tokens, const float* uniforms,
                                            int32_t* out_tokens, int32_t* out_path, int32_t* out_n_accepted)
{
    ULSPEC_CHECK_CTX(ctx);
    (void)hipSetDevice(ctx->device);
    return accept_tree_launch(ctx, s, B, n, V, parent, target_logits, draft_logits, tokens, uniforms, out_tokens,
                              out_path, out_n_accepted, nullptr);
}

extern "C" ulspec_status ulspec_sample(ulspec_ctx* ctx, const ulspec_sampling* s, uint32_t R, uint32_t V,
                                       const float* logits, const float* uniforms, int32_t* out_tokens)
{
    ULSPEC_CHECK_CTX(ctx);
    (void)hipSetDevice(ctx->device);
    return sample_launch(ctx, s, R, V, logits, uniforms, out_tokens, nullptr);
}

extern "C" ulspec_status ulspec_uniforms(ulspec_ctx* ctx, uint64_t seed, uint64_t idx0, uint32_t n, float* out)
{
    ULSPEC_CHECK_CTX(ctx);
    if (!out || n == 0) return fail(ctx, ULSPEC_EINVAL, "uniforms: null pointer or n == 0");
    (void)hipSetDevice(ctx->device);
    hipLaunchKernelGGL(uniforms_kernel, dim3((n + 255) / 256), dim3(256), 0, ctx->stream, seed, idx0, n, out);
    return check_launch(ctx, "uniforms launch");
}
