// model.cpp -- Llama-shaped model on the device: GGUF tensors by name, fp16
// KV cache, and the block forward of InferenceEngine::forward_layer_gpu
// (src/inference/inference_engine.cpp:602-682) over M <= 16 rows, with every
// linear layer on the verify dequant-GEMM and attention on the verify
// attention kernel.  Activations stay fp32: each GEMM takes its input as
// split fp16 pairs (hi, lo), so the products are fp32-exact; only the
// attention queries and the K / V cache are fp16.
//
// Weight map as Model::load_from_gguf (src/inference/model.cpp:190-246):
// "blk.N." or "layers.N." layer prefixes, GGUF and Meta tensor names.  Q, K, V
// rows are concatenated into one weight (one GEMM over (H+2Hkv)D rows), and
// gate and up rows are interleaved into another (row 2i = gate i, 2i+1 = up
// i); GGUF rows are independent block runs, so both are byte copies.
//
// Five GEMMs per layer with fused steps, plus the attention:
//   QKV   X = RMSNorm(h) in the prologue; RoPE, fp16 Q, K / V cache append in
//         the epilogue
//   attention over the cache -> split X of O
//   O     epilogue h += Y, with the per-tile sums of h^2 the next norm needs
//   GU    X = RMSNorm(h); epilogue SiLU(gate) * up -> split X of down
//   down  epilogue h += Y (+ sums of h^2)
// and the LM head with the final RMSNorm in its prologue.  Rows up to 8 whose
// split X fits in LDS run the whole-X kernels with both steps fused; others
// (the 7B FFN width, trees and prefill chunks past 8 rows) the split-K kernel,
// a norm kernel before it and the epilogue in its slice reduction.
#include "model.h"

#include <cmath>
#include <cstring>

#include "../layer_ops.h"

using namespace ulspec;

namespace {

__global__ void set_i32_kernel(int32_t* p, int32_t v) { *p = v; }

// Tree compaction of the K/V caches: rows pos + path[j] -> pos + j for j = 1
// .. cnt - 1, cnt = min(*n_acc + 1, n_max) (row pos, the root, stays), in
// every layer's K (blockIdx.z = 0) and V (1) cache.  Thread t of the grid
// moves 16-byte column group t of every row: it reads all its source rows
// before it writes any (a destination row may be another entry's source),
// and no other thread touches its columns.  Entries outside [0, n_max) or
// rows past max_ctx are skipped.
constexpr int kCompactMax = 16;
static_assert(kCompactMax >= (int)ulspec_model::kRows, "a compaction moves every row a tree forward can hold");
__global__ __launch_bounds__(256) void kv_compact_kernel(_Float16* const* __restrict__ tab, uint32_t n_layers,
                                                         uint32_t kvdim8, uint32_t max_ctx,
                                                         const int32_t* __restrict__ pos_dev, int32_t pos_add,
                                                         const int32_t* __restrict__ path,
                                                         const int32_t* __restrict__ n_acc, uint32_t n_max)
{
    const uint32_t col = blockIdx.x * 256 + threadIdx.x;
    if (col >= kvdim8) return;
    uint4* base = (uint4*)tab[blockIdx.z * n_layers + blockIdx.y];
    const int64_t pos = (int64_t)(pos_dev ? *pos_dev : 0) + pos_add;
    const int32_t cnt = min(max(*n_acc + 1, 1), (int32_t)n_max);
    uint4 r[kCompactMax];
    bool ok[kCompactMax];
#pragma unroll
    for (int j = 1; j < kCompactMax; ++j) {
        const int32_t src = j < cnt ? path[j] : -1;
        ok[j] = src >= 0 && src < (int32_t)n_max && pos >= 0 && pos + src < (int64_t)max_ctx &&
                pos + j < (int64_t)max_ctx;
        if (ok[j]) r[j] = base[(size_t)(pos + src) * kvdim8 + col];
    }
#pragma unroll
    for (int j = 1; j < kCompactMax; ++j)
        if (ok[j]) base[(size_t)(pos + j) * kvdim8 + col] = r[j];
}

// Which tensor a GGUF name is: layer (or -1 for globals) and a role.
enum Role { R_NONE, R_EMBED, R_OUT_NORM, R_OUT, R_ATTN_NORM, R_Q, R_K, R_V, R_O, R_FFN_NORM, R_GATE, R_UP, R_DOWN };

Role parse_name(const std::string& full, int& layer)
{
    layer = -1;
    std::string name = full;
    if (name.size() > 7 && name.compare(name.size() - 7, 7, ".weight") == 0) name.resize(name.size() - 7);
    if (name == "token_embd" || name == "tok_embeddings") return R_EMBED;
    if (name == "output_norm" || name == "norm") return R_OUT_NORM;
    if (name == "output") return R_OUT;
    size_t start = std::string::npos;
    if (name.compare(0, 4, "blk.") == 0) start = 4;
    else if (name.compare(0, 7, "layers.") == 0) start = 7;
    if (start == std::string::npos) return R_NONE;
    const size_t dot = name.find('.', start);
    if (dot == std::string::npos || dot == start) return R_NONE;
    long v = 0;
    for (size_t i = start; i < dot; ++i) {
        if (name[i] < '0' || name[i] > '9' || v > 1000000) return R_NONE;
        v = v * 10 + (name[i] - '0');
    }
    layer = (int)v;
    const std::string base = name.substr(dot + 1);
    if (base == "attn_norm" || base == "attention_norm") return R_ATTN_NORM;
    if (base == "attn_q" || base == "attention.wq") return R_Q;
    if (base == "attn_k" || base == "attention.wk") return R_K;
    if (base == "attn_v" || base == "attention.wv") return R_V;
    if (base == "attn_output" || base == "attention.wo") return R_O;
    if (base == "ffn_norm") return R_FFN_NORM;
    if (base == "ffn_gate" || base == "mlp_gate" || base == "feed_forward.w1") return R_GATE;
    if (base == "ffn_up" || base == "mlp_up" || base == "feed_forward.w3") return R_UP;
    if (base == "ffn_down" || base == "mlp_down" || base == "feed_forward.w2") return R_DOWN;
    return R_NONE;
}

size_t row_bytes(uint32_t type, uint64_t k)
{
    const int bs = ulspec_ggml_blck_size(type), ts = ulspec_ggml_type_size(type);
    return bs ? (size_t)(k / bs) * ts : 0;
}

ulspec_status dev_alloc(ulspec_model* m, size_t bytes, void** p)
{
    hipError_t e = hipMalloc(p, bytes);
    if (e != hipSuccess) return hip_fail(m->ctx, e, "model hipMalloc");
    m->allocs.push_back(*p);
    return ULSPEC_OK;
}

ulspec_status copy_in(ulspec_model* m, void* dst, const void* src, size_t bytes, bool on_device)
{
    hipError_t e = hipMemcpyAsync(dst, src, bytes, on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice,
                                  m->ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(m->ctx->stream);
    return e == hipSuccess ? ULSPEC_OK : hip_fail(m->ctx, e, "set_tensor copy");
}

}  // namespace

namespace ulspec {
void launch_set_i32(hipStream_t st, int32_t* p, int32_t v)
{
    hipLaunchKernelGGL(set_i32_kernel, dim3(1), dim3(1), 0, st, p, v);
}

void launch_kv_compact(hipStream_t st, _Float16* const* kv_tab, uint32_t n_layers, uint32_t kvdim, uint32_t max_ctx,
                       const int32_t* pos_dev, int32_t pos_add, const int32_t* path, const int32_t* n_acc,
                       uint32_t n_max)
{
    const uint32_t kvdim8 = kvdim / 8;  // kvdim = Hkv * D, a multiple of 64
    hipLaunchKernelGGL(kv_compact_kernel, dim3((kvdim8 + 255) / 256, n_layers, 2), dim3(256), 0, st, kv_tab,
                       n_layers, kvdim8, max_ctx, pos_dev, pos_add, path, n_acc, std::min<uint32_t>(n_max, kCompactMax));
}
}  // namespace ulspec

bool ulspec_model::complete() const
{
    if (!embed || !out_norm || w_out == ~0u) return false;
    for (const Layer& L : layers)
        if (L.wqkv == ~0u || L.wo == ~0u || L.wgu == ~0u || L.wdown == ~0u || !L.attn_norm || !L.ffn_norm)
            return false;
    return true;
}

GemmFuse ulspec_model::fuse_base() const
{
    GemmFuse f;  // split-K partials when a GEMM takes that path
    f.part = part;
    f.part_bytes = part_bytes;
    return f;
}

// X of a GEMM after an RMSNorm is split(h * w), written with h by its
// producer; the GEMM scales its rows by 1 / rms(h) from the partial sums.
void ulspec_model::normed(GemmFuse& f, const float* pss_rows, int P) const
{
    f.rs_pss = pss_rows;
    f.rs_P = P;
    f.rs_eps = cfg.rms_eps;
}

// Linear `which` of layer l over the rows of one forward with its fused
// prologue and epilogue (P: RMSNorm partials per row of h):
//   kLinQkv     X = RMSNorm(h) (from xn); RoPE, fp16 Q -> q16, K / V -> cache
//   kLinO       X = attention output (att); h += Y, next norm's X -> xn
//   kLinGateUp  X = RMSNorm(h); SiLU(gate) * up -> act
//   kLinDown    X = act; h += Y, the next layer's (or the final) norm's X -> xn
ulspec_status ulspec_model::linear(uint32_t l, int which, const Rows& rw, int P)
{
    const ulspec_model_cfg& c = cfg;
    const Layer& L = layers[l];
    const std::vector<Weight>& W = ctx->weights;
    GemmFuse f = fuse_base();
    switch (which) {
    case kLinQkv:
        normed(f, pss, P);
        f.epi = kEpiRope;
        f.pos_dev = rw.pos_dev;
        f.pos_add = rw.pos_add;
        f.nseq = (int)rw.nseq;
        f.seq_rows = (int)rw.r;
        f.seq0 = (int)rw.seq0;
        f.seq_slots = c.max_ctx;
        f.rope_rows = c.max_ctx;
        f.tree = rw.tree;
        f.row_depth = rw.depth_bits;
        f.rope = rope;
        f.q16 = q16;
        f.kc = L.kc;
        f.vc = L.vc;
        f.qdim = (int)(c.n_heads * head_dim);
        f.kvdim = (int)(c.n_kv_heads * head_dim);
        f.hd = (int)head_dim;
        return gemm_fused(ctx, W[L.wqkv], f, (const uint16_t*)xn, rw.M, rw.M, nullptr);
    case kLinO:
        f.epi = kEpiResid;
        f.h = h;
        f.pss_out = pss;
        f.xn_w = L.ffn_norm;
        f.xn = xn;
        f.xn_lo = (int)rw.M;
        return gemm_fused(ctx, W[L.wo], f, (const uint16_t*)att, rw.M, rw.M, nullptr);
    case kLinGateUp:
        normed(f, pss, P);
        f.epi = kEpiSilu;
        f.act = act;
        return gemm_fused(ctx, W[L.wgu], f, (const uint16_t*)xn, rw.M, rw.M, nullptr);
    case kLinDown:
        f.epi = kEpiResid;
        f.h = h;
        f.pss_out = pss;
        f.xn_w = l + 1 < c.n_layers ? layers[l + 1].attn_norm : out_norm;
        f.xn = xn;
        f.xn_lo = (int)rw.M;
        return gemm_fused(ctx, W[L.wdown], f, (const uint16_t*)act, rw.M, rw.M, nullptr);
    default:
        return fail(ctx, ULSPEC_EINVAL, "linear: %d is not a layer linear", which);
    }
}

ulspec_status ulspec_model::forward(const int32_t* tok_dev, uint32_t M, const int32_t* pos_dev, int32_t pos_add,
                                    float* logits_dev, uint32_t n_logits, const int32_t* parent, uint32_t nseq,
                                    uint32_t seq0)
{
    const ulspec_model_cfg& c = cfg;
    const uint32_t H = c.n_heads, Hkv = c.n_kv_heads, D = head_dim;
    if (nseq == 0 || nseq > (uint32_t)kMaxSeqs || seq0 + nseq > n_seq || M % nseq || (parent && nseq > 1))
        return fail(ctx, ULSPEC_EINVAL, "forward: %u sequences from slot %u (of %u), M=%u", nseq, seq0, n_seq, M);
    const uint32_t r = M / nseq;  // rows per sequence
    if (M == 0 || r > rows_max || M > rows_cap || n_logits > r)
        return fail(ctx, ULSPEC_EINVAL, "forward: %u rows of %u sequences (max %u each, %u in all)", M, nseq, rows_max,
                    rows_cap);
    const size_t kv_seq = (size_t)c.max_ctx * Hkv * D;
    uint64_t depth_bits = 0;  // 4-bit depth of each tree row (depth <= M - 1 <= 15)
    if (parent) {
        uint32_t depth[kRows];
        for (uint32_t i = 0; i < M; ++i) {
            if (parent[i] < -1 || parent[i] >= (int32_t)i)
                return fail(ctx, ULSPEC_EINVAL, "forward: parent[%u]=%d must be in [-1, %u)", i, parent[i], i);
            depth[i] = parent[i] < 0 ? 0 : depth[parent[i]] + 1;
            depth_bits |= (uint64_t)depth[i] << (4 * i);
        }
    }
    const std::vector<Weight>& W = ctx->weights;
    const Rows rows{M, r, nseq, seq0, pos_dev, pos_add, parent != nullptr, depth_bits};
    launch_embed(ctx->stream, embed, embed_type, c.dim, tok_dev, M, c.vocab, h, pss, layers[0].attn_norm, xn);
    int P = (int)embed_partials(c.dim);
    ulspec_status s = ULSPEC_OK;
    for (uint32_t l = 0; l < c.n_layers && s == ULSPEC_OK; ++l) {
        const Layer& L = layers[l];
        s = linear(l, kLinQkv, rows, P);
        if (s != ULSPEC_OK) break;
        AttnCall a;
        a.q = (const uint16_t*)q16;
        a.k_cache = (const uint16_t*)(L.kc + seq0 * kv_seq);
        a.v_cache = (const uint16_t*)(L.vc + seq0 * kv_seq);
        a.n_prefix = c.max_ctx - r;
        a.nq = r;
        a.nseq = nseq;
        a.kv_seq = kv_seq;
        a.parent = parent;
        a.H = H;
        a.Hkv = Hkv;
        a.D = D;
        a.scale = 1.0f / std::sqrt((float)D);
        a.out = att;
        a.out_split = true;
        a.dyn_prefix = pos_dev;
        a.prefix_add = pos_add;
        a.part = attn_part;
        a.part_bytes = attn_part_bytes;
        s = attn_launch(ctx, a);
        if (s != ULSPEC_OK) break;
        s = linear(l, kLinO, rows, P);
        if (s != ULSPEC_OK) break;
        P = (int)W[L.wo].n_tiles;
        s = linear(l, kLinGateUp, rows, P);
        if (s != ULSPEC_OK) break;
        s = linear(l, kLinDown, rows, P);
        P = (int)W[L.wdown].n_tiles;
    }
    if (s != ULSPEC_OK) return s;
    if (n_logits && (nseq == 1 || n_logits == r)) {
        // the last n_logits rows (every row of every sequence when n_logits = r):
        // their high parts from row M - nseq n_logits, low parts M rows below
        const uint32_t nl = nseq * n_logits;
        GemmFuse z = fuse_base();
        normed(z, pss + (size_t)(M - nl) * P, P);
        s = gemm_fused(ctx, W[w_out], z, (const uint16_t*)(xn + (size_t)(M - nl) * c.dim), nl, M, logits_dev);
    } else if (n_logits) {
        // the last n_logits rows of each sequence, gathered first
        const uint32_t nl = nseq * n_logits;
        launch_gather_rows(ctx->stream, xn, pss, M, c.dim, (uint32_t)P, r, n_logits, nseq, xg, pg);
        GemmFuse z = fuse_base();
        normed(z, pg, P);
        s = gemm_fused(ctx, W[w_out], z, (const uint16_t*)xg, nl, nl, logits_dev);
    }
    if (s != ULSPEC_OK) return s;
    return check_launch(ctx, "model forward launch");
}

extern "C" ulspec_status ulspec_model_create(ulspec_ctx* ctx, const ulspec_model_cfg* cfg, ulspec_model** out)
{
    return ulspec_model_create_batch(ctx, cfg, 1, out);
}

extern "C" ulspec_status ulspec_model_create_batch(ulspec_ctx* ctx, const ulspec_model_cfg* cfg, uint32_t n_seq,
                                                   ulspec_model** out)
{
    ULSPEC_CHECK_CTX(ctx);
    if (!cfg || !out) return fail(ctx, ULSPEC_EINVAL, "model_create: null pointer");
    if (n_seq == 0 || n_seq > (uint32_t)kMaxSeqs)
        return fail(ctx, ULSPEC_EINVAL, "model_create: %u sequences (1 .. %d)", n_seq, kMaxSeqs);
    const ulspec_model_cfg& c = *cfg;
    if (c.n_heads == 0 || c.n_kv_heads == 0 || c.n_heads % c.n_kv_heads || c.dim % c.n_heads)
        return fail(ctx, ULSPEC_EINVAL, "model_create: dim=%u heads=%u kv_heads=%u", c.dim, c.n_heads, c.n_kv_heads);
    const uint32_t D = c.dim / c.n_heads;
    if (D != 64 && D != 128) return fail(ctx, ULSPEC_EUNSUPPORTED, "model_create: head dim %u (64 or 128)", D);
    if (c.dim > 4096 || c.dim % 16)
        return fail(ctx, ULSPEC_EUNSUPPORTED, "model_create: dim %u (a multiple of 16, at most 4096)", c.dim);
    if (c.n_layers == 0 || c.ffn == 0 || c.vocab == 0 || c.max_ctx < 2 || c.max_ctx > (1u << 24))
        return fail(ctx, ULSPEC_EINVAL, "model_create: layers=%u ffn=%u vocab=%u max_ctx=%u", c.n_layers, c.ffn,
                    c.vocab, c.max_ctx);
    if (!(c.rms_eps > 0.0f) || !(c.rope_base > 1.0f) || !std::isfinite(c.rope_base))
        return fail(ctx, ULSPEC_EINVAL, "model_create: rms_eps / rope_base");
    (void)hipSetDevice(ctx->device);
    const uint32_t H = c.n_heads, Hkv = c.n_kv_heads, F = c.ffn;
    // rows of one forward: 16 for one sequence, 6 per sequence (k + 1 <= 6) up to 48 for a batch
    const uint32_t R = n_seq == 1 ? ulspec_model::kRows
                                  : std::max(ulspec_model::kRows, std::min(ulspec_model::kBatchRows, 6 * n_seq));
    ulspec_model* m = new ulspec_model;
    m->ctx = ctx;
    m->cfg = c;
    m->head_dim = D;
    m->layers.resize(c.n_layers);
    m->rows_max = ulspec_model::kRows;
    m->rows_cap = R;
    m->n_seq = n_seq;
    // slice partials of the split-K path: the most any of the model's weights
    // needs at R rows (slices are chosen at upload from the tile and chunk
    // counts; a weight's chunks are ceil(K / 128), or ceil(K / 256) for the
    // super-block types)
    {
        const uint32_t shapes[5][2] = {{(H + 2 * Hkv) * D, c.dim}, {c.dim, H * D}, {2 * F, c.dim}, {c.dim, F},
                                       {c.vocab, c.dim}};
        for (const auto& nk : shapes)
            for (uint32_t ck : {128u, 256u}) {
                const uint32_t ks = choose_ksplit((nk[0] + 15) / 16, (nk[1] + ck - 1) / ck, ctx->n_cu);
                m->part_bytes = std::max(m->part_bytes, (size_t)ks * R * nk[0] * sizeof(float));
            }
    }
    m->pss_stride = std::max(embed_partials(c.dim), (c.dim + 15) / 16);
    const size_t kv_bytes = (size_t)n_seq * c.max_ctx * Hkv * D * sizeof(_Float16);
    int splits = 0, kps = 0;
    attn_plan((int)c.max_ctx, (int)H, ctx->n_cu, splits, kps);
    if (splits < 2) splits = 2;
    m->attn_part_bytes = attn_workspace_bytes(splits, (int)H, (int)R, (int)D);
    struct Want {
        void** p;
        size_t bytes;
    } wants[] = {
        {(void**)&m->h, (size_t)R * c.dim * 4},
        {(void**)&m->pss, (size_t)R * m->pss_stride * 4},
        {(void**)&m->logits, (size_t)R * c.vocab * 4},
        {(void**)&m->q16, (size_t)R * H * D * 2},
        {(void**)&m->att, (size_t)2 * R * H * D * 2},
        {(void**)&m->act, (size_t)2 * R * F * 2},
        {(void**)&m->xn, (size_t)2 * R * c.dim * 2},
        {(void**)&m->part, m->part_bytes},
        {(void**)&m->tok, (size_t)R * 4},
        {(void**)&m->pos, 4 * kMaxSeqs},
        {(void**)&m->lin_pos, 4},
        {(void**)&m->attn_part, m->attn_part_bytes},
        {(void**)&m->rope, (size_t)c.max_ctx * (D / 2) * sizeof(float2)},
        {(void**)&m->kv_tab, (size_t)2 * c.n_layers * sizeof(_Float16*)},
        {(void**)&m->xg, (size_t)2 * R * c.dim * 2},
        {(void**)&m->pg, (size_t)R * m->pss_stride * 4},
    };
    ulspec_status st = ULSPEC_OK;
    for (const Want& w : wants)
        if (st == ULSPEC_OK) st = dev_alloc(m, w.bytes, w.p);
    for (uint32_t l = 0; l < c.n_layers && st == ULSPEC_OK; ++l) {
        st = dev_alloc(m, kv_bytes, (void**)&m->layers[l].kc);
        if (st == ULSPEC_OK) st = dev_alloc(m, kv_bytes, (void**)&m->layers[l].vc);
    }
    if (st == ULSPEC_OK) {
        std::vector<_Float16*> tab(2 * (size_t)c.n_layers);
        for (uint32_t l = 0; l < c.n_layers; ++l) {
            tab[l] = m->layers[l].kc;
            tab[c.n_layers + l] = m->layers[l].vc;
        }
        hipError_t e = hipMemcpy(m->kv_tab, tab.data(), tab.size() * sizeof(_Float16*), hipMemcpyHostToDevice);
        if (e != hipSuccess) st = hip_fail(ctx, e, "model kv table");
    }
    if (st == ULSPEC_OK) {
        // RoPE angles theta_i = pos * base^(-2i / D) for pair i (src/shaders/rope.glsl:50-56),
        // evaluated in double on the host, stored as fp32 (cos, sin).
        std::vector<float2> tab((size_t)c.max_ctx * (D / 2));
        for (uint32_t p = 0; p < c.max_ctx; ++p)
            for (uint32_t i = 0; i < D / 2; ++i) {
                const double th = (double)p * std::pow((double)c.rope_base, -2.0 * (double)i / (double)D);
                tab[(size_t)p * (D / 2) + i] = make_float2((float)std::cos(th), (float)std::sin(th));
            }
        hipError_t e = hipMemcpy(m->rope, tab.data(), tab.size() * sizeof(float2), hipMemcpyHostToDevice);
        if (e != hipSuccess) st = hip_fail(ctx, e, "model rope table");
    }
    if (st != ULSPEC_OK) {
        ulspec_model_destroy(m);
        return st;
    }
    *out = m;
    return ULSPEC_OK;
}

extern "C" void ulspec_model_destroy(ulspec_model* m)
{
    if (!m) return;
    (void)hipSetDevice(m->ctx->device);
    (void)hipStreamSynchronize(m->ctx->stream);
    for (void* p : m->allocs) (void)hipFree(p);
    for (auto& kv : m->pending)
        for (auto& q : kv.second.part)
            if (q.dev) (void)hipFree(q.dev);
    delete m;
}

extern "C" ulspec_status ulspec_model_set_tensor(ulspec_model* m, const char* name, uint32_t type, const void* data,
                                                 size_t nbytes, uint64_t ne0, uint64_t ne1, int on_device)
{
    if (!m) return ULSPEC_EINVAL;
    ulspec_ctx* ctx = m->ctx;
    if (!name || !data) return fail(ctx, ULSPEC_EINVAL, "set_tensor: null pointer");
    const ulspec_model_cfg& c = m->cfg;
    const uint32_t H = c.n_heads, Hkv = c.n_kv_heads, D = m->head_dim, F = c.ffn;
    int layer = -1;
    const Role role = parse_name(name, layer);
    if (role == R_NONE) return fail(ctx, ULSPEC_EINVAL, "set_tensor: unknown tensor name '%s'", name);
    if (layer >= (int)c.n_layers) return fail(ctx, ULSPEC_EINVAL, "set_tensor: '%s' beyond %u layers", name, c.n_layers);
    const bool is_norm = role == R_OUT_NORM || role == R_ATTN_NORM || role == R_FFN_NORM;
    // expected shape (ne0 = K, ne1 = rows)
    uint64_t want0 = c.dim, want1 = 1;
    switch (role) {
    case R_EMBED: want1 = c.vocab; break;
    case R_OUT: want1 = c.vocab; break;
    case R_Q: want1 = (uint64_t)H * D; break;
    case R_K:
    case R_V: want1 = (uint64_t)Hkv * D; break;
    case R_O: want0 = (uint64_t)H * D; want1 = c.dim; break;
    case R_GATE:
    case R_UP: want1 = F; break;
    case R_DOWN: want0 = F; want1 = c.dim; break;
    default: break;
    }
    if (ne0 != want0 || ne1 != want1)
        return fail(ctx, ULSPEC_EINVAL, "set_tensor: '%s' is %llu x %llu, expected %llu x %llu", name,
                    (unsigned long long)ne0, (unsigned long long)ne1, (unsigned long long)want0,
                    (unsigned long long)want1);
    (void)hipSetDevice(ctx->device);
    if (is_norm) {
        if (type != 0) return fail(ctx, ULSPEC_EUNSUPPORTED, "set_tensor: norm '%s' must be F32 (type 0)", name);
        if (nbytes != c.dim * 4) return fail(ctx, ULSPEC_EINVAL, "set_tensor: '%s' size %zu", name, nbytes);
        float** dst = role == R_OUT_NORM ? &m->out_norm
                      : role == R_ATTN_NORM ? &m->layers[layer].attn_norm : &m->layers[layer].ffn_norm;
        if (!*dst) {
            ulspec_status st = dev_alloc(m, nbytes, (void**)dst);
            if (st != ULSPEC_OK) return st;
        }
        return copy_in(m, *dst, data, nbytes, on_device != 0);
    }
    if (type != ULSPEC_GGML_Q4_0 && type != ULSPEC_GGML_Q4_K && type != ULSPEC_GGML_F16 && type != ULSPEC_GGML_Q8_0 &&
        type != ULSPEC_GGML_Q6_K)
        return fail(ctx, ULSPEC_EUNSUPPORTED, "set_tensor: '%s' type %u (Q4_0, Q4_K, Q6_K, Q8_0 or F16)", name, type);
    const size_t rb = row_bytes(type, ne0);
    if (rb == 0 || ne0 % ulspec_ggml_blck_size(type))
        return fail(ctx, ULSPEC_EINVAL, "set_tensor: '%s' row length %llu not a multiple of the block", name,
                    (unsigned long long)ne0);
    if (nbytes != rb * ne1) return fail(ctx, ULSPEC_EINVAL, "set_tensor: '%s' has %zu bytes, expected %zu", name, nbytes, rb * ne1);
    if (role == R_EMBED) {
        if (m->embed && m->embed_bytes != nbytes)
            return fail(ctx, ULSPEC_EINVAL, "set_tensor: '%s' already set with another type", name);
        if (!m->embed) {
            ulspec_status st = dev_alloc(m, nbytes, (void**)&m->embed);
            if (st != ULSPEC_OK) return st;
            m->embed_bytes = nbytes;
        }
        m->embed_type = type;
        return copy_in(m, m->embed, data, nbytes, on_device != 0);
    }
    if (role == R_OUT || role == R_O || role == R_DOWN) {
        uint32_t* id = role == R_OUT ? &m->w_out : role == R_O ? &m->layers[layer].wo : &m->layers[layer].wdown;
        if (*id != ~0u) return fail(ctx, ULSPEC_EINVAL, "set_tensor: '%s' already set", name);
        return weight_create(ctx, type, data, nbytes, (uint32_t)ne1, (uint32_t)ne0, on_device != 0, id);
    }
    // fused groups: Q | K | V and gate | up
    const bool qkv = role == R_Q || role == R_K || role == R_V;
    const std::string key = std::to_string(layer) + (qkv ? ".qkv" : ".gu");
    uint32_t* id = qkv ? &m->layers[layer].wqkv : &m->layers[layer].wgu;
    if (*id != ~0u) return fail(ctx, ULSPEC_EINVAL, "set_tensor: '%s' already set", name);
    const uint64_t rows_total = qkv ? (uint64_t)(H + 2 * Hkv) * D : 2ull * F;
    const int slot = role == R_Q || role == R_GATE ? 0 : role == R_K || role == R_UP ? 1 : 2;
    const uint32_t bit = 1u << slot;
    ulspec_model::Pending& p = m->pending[key];
    p.need = qkv ? 7u : 3u;
    if (p.have & bit) return fail(ctx, ULSPEC_EINVAL, "set_tensor: '%s' already set", name);
    ulspec_model::Pending::Part& part = p.part[slot];
    hipError_t e = hipMalloc(&part.dev, nbytes);
    if (e != hipSuccess) {
        part.dev = nullptr;
        return hip_fail(ctx, e, "set_tensor staging");
    }
    part.type = type;
    part.rows = ne1;
    ulspec_status st = copy_in(m, part.dev, data, nbytes, on_device != 0);
    if (st != ULSPEC_OK) {
        (void)hipFree(part.dev);
        part.dev = nullptr;
        return st;
    }
    p.have |= bit;
    if (p.have != p.need) return ULSPEC_OK;
    // all parts here: one type -> its blocks fused as they are; mixed types ->
    // every part as fp16 rows
    const int n_parts = qkv ? 3 : 2;
    bool same = true;
    for (int i = 1; i < n_parts; ++i) same = same && p.part[i].type == p.part[0].type;
    const uint32_t K = (uint32_t)ne0;
    uint64_t row0[3] = {0, (uint64_t)H * D, (uint64_t)(H + Hkv) * D};
    uint8_t* fused = nullptr;
    size_t fused_bytes = 0;
    uint32_t fused_type = same ? p.part[0].type : (uint32_t)ULSPEC_GGML_F16;
    if (same) {
        const size_t frb = row_bytes(fused_type, K);
        fused_bytes = frb * rows_total;
        e = hipMalloc(&fused, fused_bytes);
        if (e != hipSuccess) st = hip_fail(ctx, e, "set_tensor fused staging");
        for (int i = 0; i < n_parts && st == ULSPEC_OK; ++i) {
            const auto& q = p.part[i];
            if (qkv)
                e = hipMemcpyAsync(fused + frb * row0[i], q.dev, frb * q.rows, hipMemcpyDeviceToDevice, ctx->stream);
            else  // gate row r -> fused row 2r, up row r -> 2r + 1
                e = hipMemcpy2DAsync(fused + (i ? frb : 0), 2 * frb, q.dev, frb, frb, q.rows, hipMemcpyDeviceToDevice,
                                     ctx->stream);
            if (e != hipSuccess) st = hip_fail(ctx, e, "set_tensor fuse");
        }
    } else {
        fused_bytes = (size_t)rows_total * K * 2;
        e = hipMalloc(&fused, fused_bytes);
        if (e != hipSuccess) st = hip_fail(ctx, e, "set_tensor fused staging");
        for (int i = 0; i < n_parts && st == ULSPEC_OK; ++i) {
            const auto& q = p.part[i];
            st = qkv ? rows_to_f16(ctx, q.type, q.dev, (uint32_t)q.rows, K, (_Float16*)fused, (uint32_t)row0[i], 1)
                     : rows_to_f16(ctx, q.type, q.dev, (uint32_t)q.rows, K, (_Float16*)fused, (uint32_t)i, 2);
        }
    }
    if (st == ULSPEC_OK)
        st = weight_create(ctx, fused_type, fused, fused_bytes, (uint32_t)rows_total, K, true, id);
    (void)hipStreamSynchronize(ctx->stream);
    if (fused) (void)hipFree(fused);
    for (auto& q : p.part)
        if (q.dev) (void)hipFree(q.dev);
    m->pending.erase(key);
    return st;
}

extern "C" ulspec_status ulspec_model_forward(ulspec_model* m, const int32_t* tokens, uint32_t M, uint32_t pos,
                                              float* logits, uint32_t n_logits)
{
    if (!m) return ULSPEC_EINVAL;
    return m->forward_host(tokens, M, pos, logits, n_logits, 0);
}

extern "C" ulspec_status ulspec_model_forward_seq(ulspec_model* m, uint32_t seq, const int32_t* tokens, uint32_t M,
                                                  uint32_t pos, float* logits, uint32_t n_logits)
{
    if (!m) return ULSPEC_EINVAL;
    if (seq >= m->n_seq) return fail(m->ctx, ULSPEC_EINVAL, "model_forward_seq: sequence %u of %u", seq, m->n_seq);
    return m->forward_host(tokens, M, pos, logits, n_logits, seq);
}

ulspec_status ulspec_model::forward_host(const int32_t* tokens, uint32_t M, uint32_t pos, float* logits,
                                         uint32_t n_logits, uint32_t seq)
{
    ulspec_model* m = this;
    if (!tokens || M == 0) return fail(ctx, ULSPEC_EINVAL, "model_forward: no tokens");
    if (n_logits > m->rows_max || n_logits > M || (n_logits && !logits))
        return fail(ctx, ULSPEC_EINVAL, "model_forward: n_logits=%u (<= %u and <= M, with an output)", n_logits,
                    m->rows_max);
    if ((uint64_t)pos + M > m->cfg.max_ctx)
        return fail(ctx, ULSPEC_EINVAL, "model_forward: positions %u + %u beyond max_ctx %u", pos, M, m->cfg.max_ctx);
    if (!m->complete()) return fail(ctx, ULSPEC_EINVAL, "model_forward: model tensors missing");
    for (uint32_t i = 0; i < M; ++i)
        if (tokens[i] < 0 || (uint32_t)tokens[i] >= m->cfg.vocab)
            return fail(ctx, ULSPEC_EINVAL, "model_forward: token %d out of range", tokens[i]);
    (void)hipSetDevice(ctx->device);
    // chunks of rows_max; the last chunk is the last min(rows_max, M) rows (holds the logit rows)
    const uint32_t R = m->rows_max;
    const uint32_t last = M > R ? M - R : 0;
    uint32_t m0 = 0;
    while (true) {
        const uint32_t mc = m0 < last ? std::min(R, last - m0) : M - m0;
        const bool final_chunk = m0 + mc == M;
        hipError_t e = hipMemcpyAsync(m->tok, tokens + m0, mc * sizeof(int32_t), hipMemcpyHostToDevice, ctx->stream);
        if (e != hipSuccess) return hip_fail(ctx, e, "model_forward tokens");
        launch_set_i32(ctx->stream, m->pos, (int32_t)(pos + m0));
        ulspec_status st = m->forward(m->tok, mc, m->pos, 0, m->logits, final_chunk ? n_logits : 0, nullptr, 1, seq);
        if (st != ULSPEC_OK) return st;
        if (final_chunk) break;
        m0 += mc;
    }
    if (n_logits) {
        hipError_t e = hipMemcpyAsync(logits, m->logits, (size_t)n_logits * m->cfg.vocab * sizeof(float),
                                      hipMemcpyDeviceToHost, ctx->stream);
        if (e != hipSuccess) return hip_fail(ctx, e, "model_forward logits");
    }
    hipError_t e = hipStreamSynchronize(ctx->stream);
    return e == hipSuccess ? ULSPEC_OK : hip_fail(ctx, e, "model_forward sync");
}

extern "C" ulspec_status ulspec_model_forward_tree(ulspec_model* m, const int32_t* tokens, const int32_t* parent,
                                                   uint32_t M, uint32_t pos, float* logits)
{
    if (!m) return ULSPEC_EINVAL;
    ulspec_ctx* ctx = m->ctx;
    if (!tokens || !parent || !logits || M == 0)
        return fail(ctx, ULSPEC_EINVAL, "model_forward_tree: null pointer or no nodes");
    if (M > m->rows_max)
        return fail(ctx, ULSPEC_EINVAL, "model_forward_tree: %u nodes (at most %u)", M, m->rows_max);
    if ((uint64_t)pos + M > m->cfg.max_ctx)
        return fail(ctx, ULSPEC_EINVAL, "model_forward_tree: slots %u + %u beyond max_ctx %u", pos, M, m->cfg.max_ctx);
    if (!m->complete()) return fail(ctx, ULSPEC_EINVAL, "model_forward_tree: model tensors missing");
    for (uint32_t i = 0; i < M; ++i) {
        if (tokens[i] < 0 || (uint32_t)tokens[i] >= m->cfg.vocab)
            return fail(ctx, ULSPEC_EINVAL, "model_forward_tree: token %d out of range", tokens[i]);
        if (parent[i] < -1 || parent[i] >= (int32_t)i)
            return fail(ctx, ULSPEC_EINVAL, "model_forward_tree: parent[%u]=%d must be in [-1, %u)", i, parent[i], i);
    }
    (void)hipSetDevice(ctx->device);
    hipError_t e = hipMemcpyAsync(m->tok, tokens, M * sizeof(int32_t), hipMemcpyHostToDevice, ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "model_forward_tree tokens");
    launch_set_i32(ctx->stream, m->pos, (int32_t)pos);
    ulspec_status st = m->forward(m->tok, M, m->pos, 0, m->logits, M, parent);
    if (st != ULSPEC_OK) return st;
    e = hipMemcpyAsync(logits, m->logits, (size_t)M * m->cfg.vocab * sizeof(float), hipMemcpyDeviceToHost,
                       ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "model_forward_tree logits");
    e = hipStreamSynchronize(ctx->stream);
    return e == hipSuccess ? ULSPEC_OK : hip_fail(ctx, e, "model_forward_tree sync");
}

extern "C" ulspec_status ulspec_model_linear(ulspec_model* m, uint32_t layer, uint32_t which, uint32_t M,
                                             uint32_t pos)
{
    if (!m) return ULSPEC_EINVAL;
    ulspec_ctx* ctx = m->ctx;
    const ulspec_model_cfg& c = m->cfg;
    if (which > (uint32_t)ulspec_model::kLinHead || (which != (uint32_t)ulspec_model::kLinHead && layer >= c.n_layers))
        return fail(ctx, ULSPEC_EINVAL, "model_linear: linear %u of layer %u (0..4, layer < %u)", which, layer,
                    c.n_layers);
    if (M == 0 || M > m->rows_max || (uint64_t)pos + M > c.max_ctx)
        return fail(ctx, ULSPEC_EINVAL, "model_linear: %u rows at %u (1 .. %u rows within max_ctx %u)", M, pos,
                    m->rows_max, c.max_ctx);
    if (!m->complete()) return fail(ctx, ULSPEC_EINVAL, "model_linear: model tensors missing");
    (void)hipSetDevice(ctx->device);
    const std::vector<Weight>& W = ctx->weights;
    const ulspec_model::Layer& L = m->layers[which == (uint32_t)ulspec_model::kLinHead ? c.n_layers - 1 : layer];
    // RMSNorm partials per row of h where each linear reads them: after the
    // previous layer's down projection (the embedding's for layer 0), or after O
    const int P_in = layer == 0 ? (int)embed_partials(c.dim) : (int)W[m->layers[layer - 1].wdown].n_tiles;
    if (m->lin_pos_set != (int64_t)pos) {  // written once per position: consecutive calls launch only the GEMM
        launch_set_i32(ctx->stream, m->lin_pos, (int32_t)pos);
        m->lin_pos_set = pos;
    }
    const ulspec_model::Rows rows{M, M, 1, 0, m->lin_pos, 0, false, 0};
    ulspec_status st;
    if (which == (uint32_t)ulspec_model::kLinHead) {
        GemmFuse z = m->fuse_base();
        m->normed(z, m->pss, (int)W[L.wdown].n_tiles);
        st = gemm_fused(ctx, W[m->w_out], z, (const uint16_t*)m->xn, M, M, m->logits);
    } else {
        st = m->linear(layer, (int)which, rows, which == (uint32_t)ulspec_model::kLinGateUp ? (int)W[L.wo].n_tiles : P_in);
    }
    return st != ULSPEC_OK ? st : check_launch(ctx, "model_linear launch");
}

extern "C" ulspec_status ulspec_model_kv_compact(ulspec_model* m, uint32_t pos, const int32_t* path,
                                                 const int32_t* n_accepted, uint32_t n_max)
{
    if (!m) return ULSPEC_EINVAL;
    ulspec_ctx* ctx = m->ctx;
    if (!path || !n_accepted) return fail(ctx, ULSPEC_EINVAL, "model_kv_compact: null device pointer");
    if (n_max == 0 || n_max > ulspec_model::kRows || (uint64_t)pos + n_max > m->cfg.max_ctx)
        return fail(ctx, ULSPEC_EINVAL, "model_kv_compact: n_max=%u at %u (1 .. %u rows within max_ctx %u)", n_max,
                    pos, ulspec_model::kRows, m->cfg.max_ctx);
    (void)hipSetDevice(ctx->device);
    launch_set_i32(ctx->stream, m->pos, (int32_t)pos);
    launch_kv_compact(ctx->stream, m->kv_tab, m->cfg.n_layers, m->cfg.n_kv_heads * m->head_dim, m->cfg.max_ctx,
                      m->pos, 0, path, n_accepted, n_max);
    return check_launch(ctx, "model_kv_compact launch");
}

extern "C" ulspec_status ulspec_model_kv_io(ulspec_model* m, uint32_t layer, int dir, uint32_t pos0, uint32_t n,
                                            uint16_t* k, uint16_t* v)
{
    return ulspec_model_kv_io_seq(m, 0, layer, dir, pos0, n, k, v);
}

extern "C" ulspec_status ulspec_model_kv_io_seq(ulspec_model* m, uint32_t seq, uint32_t layer, int dir, uint32_t pos0,
                                                uint32_t n, uint16_t* k, uint16_t* v)
{
    if (!m) return ULSPEC_EINVAL;
    ulspec_ctx* ctx = m->ctx;
    if (seq >= m->n_seq || layer >= m->cfg.n_layers || (uint64_t)pos0 + n > m->cfg.max_ctx || (dir != 0 && dir != 1) ||
        (n && (!k || !v)))
        return fail(ctx, ULSPEC_EINVAL, "model_kv_io: sequence %u layer %u rows %u+%u dir %d", seq, layer, pos0, n, dir);
    (void)hipSetDevice(ctx->device);
    const size_t row = (size_t)m->cfg.n_kv_heads * m->head_dim;
    const size_t bytes = (size_t)n * row * sizeof(uint16_t);
    const size_t base = ((size_t)seq * m->cfg.max_ctx + pos0) * row;
    _Float16* kc = m->layers[layer].kc + base;
    _Float16* vc = m->layers[layer].vc + base;
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e == hipSuccess && bytes) {
        if (dir == 0) {
            e = hipMemcpy(k, kc, bytes, hipMemcpyDeviceToHost);
            if (e == hipSuccess) e = hipMemcpy(v, vc, bytes, hipMemcpyDeviceToHost);
        } else {
            e = hipMemcpy(kc, k, bytes, hipMemcpyHostToDevice);
            if (e == hipSuccess) e = hipMemcpy(vc, v, bytes, hipMemcpyHostToDevice);
        }
    }
    return e == hipSuccess ? ULSPEC_OK : hip_fail(ctx, e, "model_kv_io copy");
}
