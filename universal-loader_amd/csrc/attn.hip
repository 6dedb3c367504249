// attn.hip -- K2, attention of the nq <= 16 verified tokens over an fp16 KV
// cache (causal chain or draft tree).
//
// Replaces the per-token "flash_attention" dispatch of forward_layer_gpu
// (src/inference/inference_engine.cpp:627-630) and follows the visibility rule
// of src/shaders/attention/flash_attention_v2_fused.glsl:153-166 (key
// position <= query position, scale applied after the dot, online softmax).
//
// Split-KV ("flash-decoding"): grid (heads, splits); a workgroup of 4 waves
// owns a contiguous key range of one head, each wave takes every 4th 16-key
// tile of it and issues the loads of all its tiles before the first MFMA (one
// memory round trip per wave).  Per tile:
//   S^T[key][query] = K_tile . Q^T        16x16x32 fp16 MFMA, K loaded from
//                                         global straight into the A layout
//   online softmax per query in the log2 domain (fp32)
//   O^T[d][query] += V^T[d][key] . P^T    16x16x16 fp16 MFMA; the S^T
//                                         accumulator layout is exactly the
//                                         P^T operand layout; P = P_hi + P_lo
//                                         (two fp16 parts) keeps fp32 accuracy;
//                                         V goes through LDS and comes back
//                                         transposed (ds_read_b64_tr_b16)
// The scores of all tiles of a round come first, then one online-softmax
// update per round.
// The 4 waves are merged in LDS; each workgroup writes its partial (O, m, l)
// and a second kernel merges the splits in split order (deterministic).  (A
// merge by the last workgroup to finish, behind an atomic counter, costs more
// here: the device-scope release before the count writes back the L2.)  Visibility of the nq new keys (rows
// n_prefix .. L-1) is a per-query bitmask built on the host from the parent
// array; prefix keys are visible to every query.
#include "hip_common.h"
#include "ulspec_internal.h"

#include <cmath>

using namespace ulspec;

typedef short short4_t __attribute__((ext_vector_type(4)));

namespace {

constexpr int kAttnWaves = 4;
constexpr int kMaxQ = 16;
constexpr int kAttnMaxSplits = 64;

// nseq sequences (grid z), each with its own queries, cache and prefix.
struct AttnArgs {
    const _Float16* q;  // [nseq][nq][H][D]
    const _Float16* k;  // [nseq][kv_seq / (Hkv D)][Hkv][D]: sequence b's cache from k + b kv_seq
    const _Float16* v;
    void* out;          // [nseq nq][H][D]: fp32, fp16 (out_mode 1) or split fp16 [2][nseq nq][H][D] (2)
    float* part;        // [nseq][H][splits][nq][D + 2]: O (unnormalised), m, l
    const int32_t* dyn_prefix;  // if set, n_prefix of sequence b = dyn_prefix[b] + prefix_add (read on the device)
    size_t kv_seq;      // elements between two sequences' caches
    int nseq;
    int prefix_add;
    int n_prefix, nq, L, H, Hkv, splits, keys_per_split;
    float scale_log2;   // scale * log2(e)
    int out_mode;
    uint32_t mask[kMaxQ];
};

template <int D>
__device__ __forceinline__ void store_out(const AttnArgs& a, size_t i, float v)
{
    if (a.out_mode == 1) {
        ((_Float16*)a.out)[i] = (_Float16)v;
    } else if (a.out_mode == 2) {  // high parts, then low parts (the split X of the next GEMM)
        _Float16 hi, lo;
        split_hl(v, hi, lo);
        ((_Float16*)a.out)[i] = hi;
        ((_Float16*)a.out)[(size_t)a.nseq * a.nq * a.H * D + i] = lo;
    } else {
        ((float*)a.out)[i] = v;
    }
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Prefix length and total keys of sequence b (the split plan covers a.L
// keys; a device-side prefix may make the actual length shorter).
__device__ __forceinline__ void attn_len(const AttnArgs& a, int b, int& n_prefix, int& L)
{
    n_prefix = a.dyn_prefix ? a.dyn_prefix[b] + a.prefix_add : a.n_prefix;
    L = n_prefix + a.nq;
}

template <int D, int T>
__global__ __launch_bounds__(kAttnWaves * 64) void attn_kernel(AttnArgs a)
{
    constexpr int VP = D + 8;  // V tile row pitch in halfs (16 B pad spreads banks)
    __shared__ _Float16 vt[kAttnWaves][16 * VP];
    __shared__ float red_o[kAttnWaves][kMaxQ][D + 1];  // odd pitch: the MFMA-layout writes spread over banks
    __shared__ float red_m[kAttnWaves][kMaxQ], red_l[kAttnWaves][kMaxQ];

    const int h = blockIdx.x, s = blockIdx.y, b = blockIdx.z;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = lane & 15, g = lane >> 4;  // c: query (S^T, O^T columns) / key / d column
    const int hk = h / (a.H / a.Hkv);
    const size_t row_stride = (size_t)a.Hkv * D;
    const _Float16* qs = a.q + (size_t)b * a.nq * a.H * D;
    const _Float16* ks = a.k + (size_t)b * a.kv_seq;
    const _Float16* vs = a.v + (size_t)b * a.kv_seq;

    int n_prefix, L;
    attn_len(a, b, n_prefix, L);
    const int j0 = s * a.keys_per_split;
    if (j0 >= L) return;  // only when the prefix is read on the device
    const int j1 = min(L, j0 + a.keys_per_split);

    // Q^T operand: lane (query c, group g) holds Q[c][h][32 st + 8 g .. +7]
    half8_t qb[D / 32];
    const bool qvalid = c < a.nq;
#pragma unroll
    for (int st = 0; st < D / 32; ++st)
        qb[st] = qvalid ? *(const half8_t*)(qs + ((size_t)c * a.H + h) * D + 32 * st + 8 * g) : half8_t{};
    uint32_t mask = 0;
#pragma unroll
    for (int i = 0; i < kMaxQ; ++i)
        if (c == i) mask = a.mask[i];

    float m = -INFINITY, l = 0.0f;
    float4_t oacc[D / 16];
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) oacc[dt] = float4_t{0.f, 0.f, 0.f, 0.f};
    _Float16* myv = vt[wave];

    // rounds of 64 T keys; in each, every K / V load of the wave is issued
    // first: tile i covers keys jr + 16 (wave + 4 i) ..
    for (int jr = j0; jr < j1; jr += 16 * kAttnWaves * T) {
        half8_t ka[T][D / 32], va[T][D / 32];
#pragma unroll
        for (int i = 0; i < T; ++i) {
            const int key = jr + 16 * (wave + kAttnWaves * i) + c;
            const size_t kbase = (size_t)(key < j1 ? key : j0) * row_stride + (size_t)hk * D + 8 * g;
#pragma unroll
            for (int st = 0; st < D / 32; ++st) {
                ka[i][st] = *(const half8_t*)(ks + kbase + 32 * st);
                va[i][st] = *(const half8_t*)(vs + kbase + 32 * st);
            }
        }
        asm volatile("" ::: "memory");  // keep every load of the round ahead of the first use
        // scores of every tile of the round, then one softmax update for the
        // round (rescale, max and sum shuffles once per round, not per tile)
        float s2[T][4];
        float tmax = -INFINITY;
#pragma unroll
        for (int i = 0; i < T; ++i) {
            const int jt = jr + 16 * (wave + kAttnWaves * i);
            float4_t sacc = {0.f, 0.f, 0.f, 0.f};
            if (jt < j1) {  // uniform in the wave
#pragma unroll
                for (int st = 0; st < D / 32; ++st) sacc = mfma16x16x32(ka[i][st], qb[st], sacc);
            }
            // lane holds S^T[key 4g + r][query c]
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int j = jt + 4 * g + r;
                const bool vis = j < j1 && (j < n_prefix || ((mask >> (j - n_prefix)) & 1u));
                s2[i][r] = vis ? sacc[r] * a.scale_log2 : -INFINITY;
                tmax = fmaxf(tmax, s2[i][r]);
            }
        }
        tmax = fmaxf(tmax, xor_lane<16>(tmax));
        tmax = fmaxf(tmax, xor_lane<32>(tmax));
        const float mnew = fmaxf(m, tmax);
        const float muse = mnew == -INFINITY ? 0.0f : mnew;
        const float alpha = exp2_fast(m - muse);
        float p[T][4], psum = 0.0f;
#pragma unroll
        for (int i = 0; i < T; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                p[i][r] = exp2_fast(s2[i][r] - muse);
                psum += p[i][r];
            }
        psum += xor_lane<16>(psum);
        psum += xor_lane<32>(psum);
        l = l * alpha + psum;
        m = mnew;
        if (jr != j0) {  // the first round starts from O = 0: nothing to rescale
#pragma unroll
            for (int dt = 0; dt < D / 16; ++dt) oacc[dt] = oacc[dt] * alpha;
        }
#pragma unroll
        for (int i = 0; i < T; ++i) {
            const int jt = jr + 16 * (wave + kAttnWaves * i);
            if (jt < j1) {  // uniform in the wave
                // V rows to the wave's LDS slot (LDS ops of one wave stay in order)
#pragma unroll
                for (int st = 0; st < D / 32; ++st) *(half8_t*)(myv + c * VP + 32 * st + 8 * g) = va[i][st];
                half4_t phi, plo;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    phi[r] = (_Float16)p[i][r];
                    plo[r] = (_Float16)(p[i][r] - (float)phi[r]);
                }
#pragma unroll
                for (int dt = 0; dt < D / 16; ++dt) {
                    // V^T operand: lane (d = 16 dt + c, group g) holds V[key 4g + r][d],
                    // r = 0..3: one transposing read, lane x = 4r + q of each 16-lane
                    // group addressing V[key 4g + r][16 dt + 4q .. +3]
                    const half4_t vv = __builtin_bit_cast(
                        half4_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                     (__attribute__((address_space(3))) short4_t*)(myv + (4 * g + (c >> 2)) * VP +
                                                                                     16 * dt + 4 * (c & 3))));
                    oacc[dt] = mfma16x16x16(vv, phi, oacc[dt]);
                    oacc[dt] = mfma16x16x16(vv, plo, oacc[dt]);
                }
            }
        }
    }

    // merge the 4 waves: lane holds O^T[d = 16 dt + 4 g + r][query c]
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt)
#pragma unroll
        for (int r = 0; r < 4; ++r) red_o[wave][c][16 * dt + 4 * g + r] = oacc[dt][r];
    if (g == 0) {
        red_m[wave][c] = m;
        red_l[wave][c] = l;
    }
    __syncthreads();
    float* pp = a.part + (((size_t)b * a.H + h) * a.splits + s) * a.nq * (D + 2);
    // the nq * D outputs only, d fastest (coalesced stores, conflict-free reads)
    for (int idx = threadIdx.x; idx < a.nq * D; idx += kAttnWaves * 64) {
        const int qi = idx / D, d = idx - qi * D;
        float M = red_m[0][qi];
#pragma unroll
        for (int w = 1; w < kAttnWaves; ++w) M = fmaxf(M, red_m[w][qi]);
        const float Mu = M == -INFINITY ? 0.0f : M;
        float o = 0.0f, Lw = 0.0f;
#pragma unroll
        for (int w = 0; w < kAttnWaves; ++w) {
            const float f = exp2_fast(red_m[w][qi] - Mu);
            o += red_o[w][qi][d] * f;
            Lw += red_l[w][qi] * f;
        }
        if (a.splits == 1) {
            store_out<D>(a, (((size_t)b * a.nq + qi) * a.H + h) * D + d, o / Lw);
        } else {
            pp[qi * (D + 2) + d] = o;
            if (d == 0) {
                pp[qi * (D + 2) + D] = M;
                pp[qi * (D + 2) + D + 1] = Lw;
            }
        }
    }
}

// out[qi][h][d] = sum_s O_s e^(m_s - M) / sum_s l_s e^(m_s - M) over the
// splits that hold keys, in split order (deterministic).  Grid (H, nq), D
// threads; (m, l) of every split staged in LDS.  SU >= splits (16, 32 or
// 64): every O load and every LDS read is issued before the first use, none
// waits for the device-side prefix length.  They read splits
// 0..min(u, splits - 1) of the workspace (which holds all `splits` partials,
// so every read is in bounds; a split past the last one holding keys reads
// stale values) and the count of live splits masks them afterwards with
// selects, so the sums keep split order.
template <int D, int SU>
__global__ __launch_bounds__(D) void attn_merge_kernel(AttnArgs a)
{
    __shared__ float sm[kAttnMaxSplits], sl[kAttnMaxSplits];
    static_assert(SU <= kAttnMaxSplits, "SU splits staged in LDS");
    const int h = blockIdx.x, qi = blockIdx.y, b = blockIdx.z, d = threadIdx.x;
    const int S = a.splits;
    const size_t stride = (size_t)a.nq * (D + 2);
    const float* q0 = a.part + ((size_t)b * a.H + h) * S * stride + qi * (D + 2);
    float ov[SU];
#pragma unroll
    for (int u = 0; u < SU; ++u) ov[u] = q0[min(u, S - 1) * stride + d];
    const int ds = min(d, S - 1);
    const float mv = q0[ds * stride + D], lv = q0[ds * stride + D + 1];
    int n_prefix, L;
    attn_len(a, b, n_prefix, L);
    const int ns = min(S, (L + a.keys_per_split - 1) / a.keys_per_split);
    if (d < S) {
        sm[d] = mv;
        sl[d] = lv;
    }
    __syncthreads();
    float mu[SU], lu[SU];
#pragma unroll
    for (int u = 0; u < SU; ++u) {
        mu[u] = sm[u];
        lu[u] = sl[u];
    }
    float M = -INFINITY;
#pragma unroll
    for (int u = 0; u < SU; ++u) M = u < ns ? fmaxf(M, mu[u]) : M;
    const float Mu = M == -INFINITY ? 0.0f : M;
    float o = 0.0f, Ls = 0.0f;
#pragma unroll
    for (int u = 0; u < SU; ++u) {
        const float f = exp2_fast(mu[u] - Mu);
        const bool live = u < ns;
        o = live ? o + ov[u] * f : o;
        Ls = live ? Ls + lu[u] * f : Ls;
    }
    store_out<D>(a, (((size_t)b * a.nq + qi) * a.H + h) * D + d, o / Ls);
}

template <int D>
void launch_attn(const AttnArgs& a, int T, hipStream_t st)
{
    const dim3 grid(a.H, a.splits, a.nseq), block(kAttnWaves * 64);
    switch (T) {
    case 1: hipLaunchKernelGGL((attn_kernel<D, 1>), grid, block, 0, st, a); break;
    case 2: hipLaunchKernelGGL((attn_kernel<D, 2>), grid, block, 0, st, a); break;
    default: hipLaunchKernelGGL((attn_kernel<D, 4>), grid, block, 0, st, a); break;
    }
    if (a.splits > 1) {
        const dim3 mg(a.H, a.nq, a.nseq);
        if (a.splits <= 16) hipLaunchKernelGGL((attn_merge_kernel<D, 16>), mg, dim3(D), 0, st, a);
        else if (a.splits <= 32) hipLaunchKernelGGL((attn_merge_kernel<D, 32>), mg, dim3(D), 0, st, a);
        else hipLaunchKernelGGL((attn_merge_kernel<D, kAttnMaxSplits>), mg, dim3(D), 0, st, a);
    }
}

}  // namespace

namespace ulspec {

// Splits so that heads x splits is about two workgroups per CU, at most
// kAttnMaxSplits; keys per split a multiple of 64, covered in rounds of 64 T
// keys (T = 4, 2 or 1 tiles of 16 keys per wave, the largest that divides
// it; all of a round's loads are issued before its first MFMA).
void attn_plan(int L, int H, int n_cu, int& splits, int& kps)
{
    int want = (2 * n_cu + H - 1) / H;
    want = want < 1 ? 1 : (want > kAttnMaxSplits ? kAttnMaxSplits : want);
    const int need = (L + want - 1) / want;
    kps = (need + 63) / 64 * 64;
    splits = (L + kps - 1) / kps;
}

int attn_tiles(int kps)
{
    return kps % 256 == 0 ? 4 : (kps % 128 == 0 ? 2 : 1);
}

size_t attn_workspace_bytes(int splits, int H, int nq, int D, int nseq)
{
    return splits > 1 ? (size_t)nseq * splits * H * nq * (D + 2) * sizeof(float) : 0;
}

}  // namespace ulspec

namespace ulspec {

ulspec_status attn_launch(ulspec_ctx* ctx, const AttnCall& c)
{
    if (!c.q || !c.k_cache || !c.v_cache || !c.out) return fail(ctx, ULSPEC_EINVAL, "verify_attention: null pointer");
    if (c.nq == 0 || c.nq > (uint32_t)kMaxQ)
        return fail(ctx, ULSPEC_EINVAL, "verify_attention: nq=%u not in [1, 16]", c.nq);
    if (c.D != 64 && c.D != 128) return fail(ctx, ULSPEC_EUNSUPPORTED, "verify_attention: head dim %u (64 or 128)", c.D);
    if (c.H == 0 || c.Hkv == 0 || c.H % c.Hkv) return fail(ctx, ULSPEC_EINVAL, "verify_attention: H=%u Hkv=%u", c.H, c.Hkv);
    if (!(c.scale > 0.0f) || !std::isfinite(c.scale)) return fail(ctx, ULSPEC_EINVAL, "verify_attention: scale");
    if ((uint64_t)c.n_prefix + c.nq > (uint64_t)INT32_MAX) return fail(ctx, ULSPEC_EINVAL, "verify_attention: length");
    AttnArgs a;
    a.q = (const _Float16*)c.q;
    a.k = (const _Float16*)c.k_cache;
    a.v = (const _Float16*)c.v_cache;
    a.out = c.out;
    a.out_mode = c.out_split ? 2 : c.out_f16 ? 1 : 0;
    a.dyn_prefix = c.dyn_prefix;
    a.prefix_add = c.prefix_add;
    a.nseq = (int)c.nseq;
    a.kv_seq = c.kv_seq;
    a.n_prefix = (int)c.n_prefix;  // with dyn_prefix: the largest prefix the call may see
    a.nq = (int)c.nq;
    a.L = (int)(c.n_prefix + c.nq);
    a.H = (int)c.H;
    a.Hkv = (int)c.Hkv;
    a.scale_log2 = c.scale * 1.4426950408889634f;
    for (int i = 0; i < kMaxQ; ++i) a.mask[i] = 0;
    for (uint32_t i = 0; i < c.nq; ++i) {
        uint32_t mk = 0;
        if (!c.parent) {
            mk = (1u << (i + 1)) - 1u;
        } else {
            if (c.parent[i] >= (int32_t)i || c.parent[i] < -1)
                return fail(ctx, ULSPEC_EINVAL, "verify_attention: parent[%u]=%d must be in [-1, %u)", i, c.parent[i], i);
            mk = 1u << i;
            for (int32_t pnode = c.parent[i]; pnode >= 0; pnode = c.parent[pnode]) mk |= 1u << pnode;
        }
        a.mask[i] = mk;
    }
    if (c.nseq < 1 || c.nseq > (uint32_t)kMaxSeqs || (c.nseq > 1 && !c.dyn_prefix))
        return fail(ctx, ULSPEC_EINVAL, "verify_attention: %u sequences (1..%d, device prefixes)", c.nseq, kMaxSeqs);
    attn_plan(a.L, a.H * a.nseq, ctx->n_cu, a.splits, a.keys_per_split);
    if (c.dyn_prefix && a.splits == 1) a.splits = 2;  // keep the merge: a split may return early
    if (a.splits > kAttnMaxSplits)  // the merge stages at most kAttnMaxSplits (m, l) pairs
        return fail(ctx, ULSPEC_EUNSUPPORTED, "verify_attention: %d splits (at most %d)", a.splits, kAttnMaxSplits);
    void* ws = c.part;
    const size_t wsb = attn_workspace_bytes(a.splits, a.H, a.nq, (int)c.D, a.nseq);
    if (wsb && ws && wsb > c.part_bytes)
        return fail(ctx, ULSPEC_EINVAL, "verify_attention: %d splits need %zu B of partials, the workspace holds %zu B",
                    a.splits, wsb, c.part_bytes);
    if (wsb && !ws) {
        ulspec_status st = workspace(ctx, wsb, &ws);
        if (st != ULSPEC_OK) return st;
    }
    a.part = (float*)ws;
    const int T = attn_tiles(a.keys_per_split);
    if (c.D == 128) launch_attn<128>(a, T, ctx->stream);
    else launch_attn<64>(a, T, ctx->stream);
    return check_launch(ctx, "verify_attention launch");
}

}  // namespace ulspec

extern "C" ulspec_status ulspec_verify_attention(ulspec_ctx* ctx, const uint16_t* q, const uint16_t* k_cache,
                                                 const uint16_t* v_cache, uint32_t n_prefix, uint32_t nq,
                                                 const int32_t* parent, uint32_t H, uint32_t Hkv, uint32_t D,
                                                 float scale, float* out)
{
    ULSPEC_CHECK_CTX(ctx);
    (void)hipSetDevice(ctx->device);
    AttnCall c;
    c.q = q;
    c.k_cache = k_cache;
    c.v_cache = v_cache;
    c.n_prefix = n_prefix;
    c.nq = nq;
    c.parent = parent;
    c.H = H;
    c.Hkv = Hkv;
    c.D = D;
    c.scale = scale;
    c.out = out;
    return attn_launch(ctx, c);
}
