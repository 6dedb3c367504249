// ulspec_internal.h -- context state shared by the C-ABI translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>
#include <vector>

#include "../../include/ulspec.h"

namespace ulspec {

// One uploaded linear weight, re-tiled for the dequant-GEMM kernels.
struct Weight {
    uint32_t type = 0;      // tile format: ULSPEC_GGML_Q4_0 / Q4_K / F16
    uint32_t src_type = 0;  // the uploaded GGUF type (Q8_0 and Q6_K are held as F16)
    uint32_t n = 0, k = 0;  // rows (N) and elements per row (K)
    uint32_t n_tiles = 0;   // ceil(N / 16)
    uint32_t n_chunks = 0;  // per tile: Q4_0 block quads, Q4_K super-blocks, F16 128-element runs
    uint32_t ksplit = 1;    // K slices of the split-K launch (fixed per weight)
    size_t bytes = 0;
    uint8_t* dev = nullptr;
};

}  // namespace ulspec

struct ulspec_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    int n_cu = 0;
    std::string err;
    std::vector<ulspec::Weight> weights;
    // Reusable device workspace (grown on demand, freed with the context).
    void* ws = nullptr;
    size_t ws_bytes = 0;
    // Host staging for weight uploads.
    void* staging = nullptr;
    size_t staging_bytes = 0;
    // Device address of the no-allocation scratch on this context's device.
    void* noalloc_scratch = nullptr;
    // ULSPEC_OPT_TOPK_ROUTE (0: automatic)
    int topk_route = 0;
    // Captured graphs and timing events.
    std::vector<hipGraphExec_t> graphs;
    bool capturing = false;
    hipEvent_t events[16] = {};
};

namespace ulspec {

inline ulspec_status fail(ulspec_ctx* ctx, ulspec_status st, const char* fmt, ...)
{
    if (ctx) {
        char buf[512];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof(buf), fmt, ap);
        va_end(ap);
        ctx->err = buf;
    }
    return st;
}

inline ulspec_status hip_fail(ulspec_ctx* ctx, hipError_t e, const char* what)
{
    return fail(ctx, e == hipErrorOutOfMemory ? ULSPEC_ENOMEM : ULSPEC_EDEVICE, "%s: %s", what,
                hipGetErrorString(e));
}

// One-time kernel attributes of the dequant-GEMM and the no-allocation
// scratch address (called by ulspec_create, with the context's device current).
ulspec_status gemm_init(ulspec_ctx* ctx);
ulspec_status accept_init(ulspec_ctx* ctx);

// Sequences of one batched forward (each with its own K / V cache slot).
constexpr int kMaxSeqs = 8;

// Row scale and epilogues of the dequant-GEMM in the model forward.
enum { kEpiStore = 0, kEpiRope = 1, kEpiSilu = 2, kEpiResid = 3 };
// Rows per launch: fp16 X through the ABI GEMM, split X through the fused GEMM.
constexpr int kGemmRowsH16 = 64;
constexpr int kGemmRowsSplit = 48;
struct GemmFuse {
    int epi = kEpiStore;
    // row scale (the RMSNorm before this GEMM): Y[m][:] *= 1 / sqrt(sum_p
    // rs_pss[m][p] / K + rs_eps), p < rs_P <= 256; X is then split(h * w),
    // written by the producer of h (the resid epilogue's xn, the embedding)
    const float* rs_pss = nullptr;
    int rs_P = 0;
    float rs_eps = 0.0f;
    // kEpiRope: rows are nseq groups of seq_rows (one per sequence, sequence
    // slots seq0 ..); row j of sequence b takes RoPE position pos_dev[b] +
    // pos_add + j (with tree != 0: + depth(j), depth(j) = bits 4j .. 4j+3 of
    // row_depth) and its K / V go to cache row (seq0 + b) seq_slots +
    // pos_dev[b] + pos_add + j; Q rows [0, qdim) -> q16, K rows -> kc, V rows -> vc
    const int32_t* pos_dev = nullptr;
    int pos_add = 0;
    int nseq = 1, seq_rows = 0, seq0 = 0;
    uint32_t seq_slots = 0;  // cache rows per sequence (max_ctx)
    uint32_t rope_rows = 0;  // positions of the rope table
    int tree = 0;
    uint64_t row_depth = 0;
    const float2* rope = nullptr;
    _Float16* q16 = nullptr;
    _Float16* kc = nullptr;
    _Float16* vc = nullptr;
    int qdim = 0, kvdim = 0, hd = 0;
    // kEpiSilu: rows interleaved gate / up -> act, split fp16 pairs [2M][N / 2] (hi rows, then lo rows)
    _Float16* act = nullptr;
    // kEpiResid: h [M][N] += Y; pss_out [M][n_tiles] = per-tile sums of h^2;
    // with xn the next GEMM's split X: rows m (hi) and xn_lo + m (lo) of h * xn_w
    float* h = nullptr;
    float* pss_out = nullptr;
    const float* xn_w = nullptr;
    _Float16* xn = nullptr;
    int xn_lo = 0;
    // split-K path (rows or K beyond what the whole-X kernels hold): slice
    // partials (NULL = the context workspace)
    float* part = nullptr;
    size_t part_bytes = 0;
};

// Kernel launchers shared by the C ABI and the host engine (no validation of
// device pointers; arguments checked as in the corresponding ABI entry point).
ulspec_status gemm_launch(ulspec_ctx* ctx, const Weight& w, const uint16_t* x, uint32_t M, float* y);
// Rows of GGUF blocks (device) to fp16 rows out[out_row0 + r * out_row_step][K].
ulspec_status rows_to_f16(ulspec_ctx* ctx, uint32_t type, const void* raw, uint32_t rows, uint32_t K,
                          _Float16* out, uint32_t out_row0, uint32_t out_row_step);
// The dequant-GEMM with a fused row scale / epilogue over split X (the model
// forward; the low part of row m at row lo_rows + m): the whole-X kernels for
// M <= 8 rows that fit in LDS, else the split-K kernel and the reducing
// epilogue.
ulspec_status gemm_fused(ulspec_ctx* ctx, const Weight& w, const GemmFuse& f, const uint16_t* x, uint32_t M,
                         uint32_t lo_rows, float* y);
size_t gemm_workspace_bytes(const Weight& w);
uint32_t choose_ksplit(uint32_t n_tiles, uint32_t n_chunks, int n_cu);
size_t gemm_split_part_bytes(const Weight& w, uint32_t M);
ulspec_status weight_create(ulspec_ctx* ctx, uint32_t type, const void* blocks, size_t nbytes, uint32_t N, uint32_t K,
                            bool on_device, uint32_t* out_id);
struct AttnCall {
    const uint16_t* q = nullptr;
    const uint16_t* k_cache = nullptr;
    const uint16_t* v_cache = nullptr;
    uint32_t n_prefix = 0;   // with dyn_prefix: an upper bound of the prefix (sizes the split plan)
    uint32_t nq = 0;
    const int32_t* parent = nullptr;  // host array, NULL = causal
    uint32_t H = 0, Hkv = 0, D = 0;
    float scale = 0.0f;
    void* out = nullptr;
    bool out_f16 = false;
    bool out_split = false;  // split fp16 pair [2][nq][H][D] (hi, lo) for the next GEMM's X
    const int32_t* dyn_prefix = nullptr;  // device int per sequence: prefix = dyn_prefix[b] + prefix_add
    int prefix_add = 0;
    void* part = nullptr;    // split partials; NULL = the context workspace
    size_t part_bytes = 0;   // bytes at part (the launch fails if its plan needs more)
    // nseq sequences: q and out hold nseq groups of nq rows, sequence b's
    // cache starts kv_seq elements after sequence b-1's (needs dyn_prefix)
    uint32_t nseq = 1;
    size_t kv_seq = 0;
};
ulspec_status attn_launch(ulspec_ctx* ctx, const AttnCall& c);
void attn_plan(int L, int H, int n_cu, int& splits, int& kps);
size_t attn_workspace_bytes(int splits, int H, int nq, int D, int nseq = 1);
size_t accept_workspace_bytes(uint32_t B, uint32_t k);
size_t sample_workspace_bytes(uint32_t R);
ulspec_status accept_launch(ulspec_ctx* ctx, const ulspec_sampling* s, uint32_t B, uint32_t k, uint32_t V,
                            const float* target_logits, const float* draft_logits, const int32_t* draft_tokens,
                            const float* uniforms, int32_t* out_tokens, int32_t* out_n_accepted, void* ws);
size_t accept_tree_workspace_bytes(uint32_t B, uint32_t n);
ulspec_status accept_tree_launch(ulspec_ctx* ctx, const ulspec_sampling* s, uint32_t B, uint32_t n, uint32_t V,
                                 const int32_t* parent, const float* target_logits, const float* draft_logits,
                                 const int32_t* tokens, const float* uniforms, int32_t* out_tokens,
                                 int32_t* out_path, int32_t* out_n_accepted, void* ws);
ulspec_status sample_launch(ulspec_ctx* ctx, const ulspec_sampling* s, uint32_t R, uint32_t V, const float* logits,
                            const float* uniforms, int32_t* out_tokens, void* ws);
// D draws, draw d from row map[d] of logits [R][V] with uniforms[d] (the
// workspace of sample_workspace_bytes(R)).
ulspec_status sample_mapped_launch(ulspec_ctx* ctx, const ulspec_sampling* s, uint32_t R, uint32_t V,
                                   const float* logits, uint32_t D, const int32_t* map, const float* uniforms,
                                   int32_t* out_tokens, void* ws);
// Greedy tree drafting: the n_kids[i] best tokens of row i (logit desc, index
// asc) to out_tokens[first_kid[i] ..].
void topb_launch(ulspec_ctx* ctx, const float* logits, uint32_t V, uint32_t rows, const int32_t* first_kid,
                 const int32_t* n_kids, int32_t* out_tokens);

// Grow the context workspace to at least `bytes` (stream-ordered reuse).
ulspec_status workspace(ulspec_ctx* ctx, size_t bytes, void** out);

// Launch-after checks: reports a failed launch as ULSPEC_EDEVICE.
inline ulspec_status check_launch(ulspec_ctx* ctx, const char* what)
{
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(ctx, e, what);
    return ULSPEC_OK;
}

}  // namespace ulspec

#define ULSPEC_CHECK_CTX(ctx)                  \
    do {                                       \
        if (!(ctx)) return ULSPEC_EINVAL;      \
        (ctx)->err.clear();                    \
    } while (0)
