// spec.cpp -- the speculative decoding loop on the device.
//
// Replaces SpeculativeDecoder::generate_with_speculation
// (src/inference/speculative_decoder.cpp:25-71): instead of host callbacks and
// first-match acceptance, one step is
//   draft:  forward [t_{n-2}, t_{n-1}] at positions n-2, n-1 (re-computing
//           row n-2 keeps the draft cache whole when the previous step
//           accepted every draft token), sample d_1; then forward d_j at n-1+j
//           and sample d_{j+1}, j = 1 .. k-1
//   target: forward [t_{n-1}, d_1 .. d_k] at positions n-1 .. n-1+k
//   accept: the speculative-sampling / greedy rule -> n_acc + 1 tokens
//   commit: append them to the sequence, n += n_acc + 1
// Every position, token and counter lives in device memory, so a step is a
// fixed kernel sequence: it is captured once into a HIP graph and replayed,
// with no host synchronisation inside or between steps.  Uniforms of step s:
// draft j uses counter s*(2k+1) + j, the accept rule s*(2k+1) + k + j.
//
// k = 0 is plain decoding of the target (no draft model): a step forwards
// t_{n-1} at n-1 and samples t_n from its logits with counter s.  A prompt of
// one token starts the same way for k > 0: the first step is such a plain
// step (the draft's catch-up pair needs two committed tokens), after which
// the draft catches up on [t_0, t_1].
//
// Tree steps (ulspec_spec_create_tree, one sequence): a fixed draft tree of n
// <= 16 nodes in breadth-first order (node 0 the root t_{n-1}).  The draft
// runs one tree-masked forward per level l < depth over [t_{n-2}, root, the
// nodes of levels <= l] (row 0 re-computes t_{n-2}, as the chain's catch-up
// pair does) and draws the children of level l from their parents' logits:
// i.i.d. with the uniforms of the node (sampling; the multi-draft rule needs
// children drawn from q), or the parent's best tokens in order (greedy).  The
// target scores all n nodes in one tree forward, ulspec_accept_tree picks the
// path, both caches are compacted along it, and the path plus the final
// token are committed.  Uniforms of step s: node i's draw u(seed,
// s(2n-1) + i - 1), the acceptance u(seed, s(2n-1) + n - 1 + j) -- the chain's
// counters when the tree is a chain of k + 1 nodes.
#include <algorithm>

#include "../detmath.h"
#include "model.h"

using namespace ulspec;

namespace {

struct SpecState {
    int32_t n;        // committed tokens (prompt included)
    int32_t pad;
    uint64_t step;
    uint64_t accepted;  // accepted draft tokens
    uint64_t proposed;  // proposed draft tokens
};

// Uniforms of step s for every sequence b: counter (s B + b)(2k+1) + j, j = 0
// .. 2k, to unif [B][2k+1]; draft draws j < k also to udraft [k][B] (one
// contiguous row of B per draft step), the accept rule's to uacc [B][k+1].
// The draft's catch-up pair [t_{n-2}, t_{n-1}] of each sequence to tok_d [B][2].
__global__ void spec_begin_kernel(const int32_t* __restrict__ npos, const int32_t* __restrict__ seq, uint32_t cap,
                                  const SpecState* __restrict__ st, uint64_t seed, uint32_t k, uint32_t B,
                                  float* __restrict__ unif, float* __restrict__ udraft, float* __restrict__ uacc,
                                  int32_t* __restrict__ tok_d)
{
    const uint32_t per = 2 * k + 1;
    const uint64_t step = st[0].step;
    for (uint32_t i = threadIdx.x; i < B * per; i += blockDim.x) {
        const uint32_t b = i / per, j = i - b * per;
        const float u = counter_uniform(seed, (step * B + b) * per + j);
        unif[i] = u;
        if (j < k) udraft[j * B + b] = u;
        else uacc[b * (k + 1) + (j - k)] = u;
    }
    for (uint32_t b = threadIdx.x; b < B; b += blockDim.x) {
        tok_d[2 * b] = seq[(size_t)b * cap + npos[b] - 2];
        tok_d[2 * b + 1] = seq[(size_t)b * cap + npos[b] - 1];
    }
}

// Plain (target-only) step: the uniform of counter (s B + b)(2k+1) and the
// last token of every sequence.
__global__ void spec_plain_begin_kernel(const int32_t* __restrict__ npos, const int32_t* __restrict__ seq,
                                        uint32_t cap, const SpecState* __restrict__ st, uint64_t seed, uint32_t k,
                                        uint32_t B, float* __restrict__ unif, float* __restrict__ uplain,
                                        int32_t* __restrict__ tok_t)
{
    const uint64_t step = st[0].step;
    for (uint32_t b = threadIdx.x; b < B; b += blockDim.x) {
        const float u = counter_uniform(seed, (step * B + b) * (2 * k + 1));
        unif[b * (2 * k + 1)] = u;
        uplain[b] = u;
        tok_t[b] = seq[(size_t)b * cap + npos[b] - 1];
    }
}

// Target rows of every sequence: [t_{n-1}, d_1 .. d_k] from dtok_s [k][B].
__global__ void spec_verify_tokens_kernel(const int32_t* __restrict__ npos, const int32_t* __restrict__ seq,
                                          uint32_t cap, const int32_t* __restrict__ dtok_s, uint32_t k, uint32_t B,
                                          int32_t* __restrict__ tok_t)
{
    for (uint32_t i = threadIdx.x; i < B * (k + 1); i += blockDim.x) {
        const uint32_t b = i / (k + 1), j = i - b * (k + 1);
        tok_t[i] = j == 0 ? seq[(size_t)b * cap + npos[b] - 1] : dtok_s[(j - 1) * B + b];
    }
}

// Draft tokens and logits from step-major [k][B] to sequence-major [B][k]
// (the accept rule's layout); float4 groups of the V-float rows (V % 4 == 0).
__global__ __launch_bounds__(256) void spec_gather_draft_kernel(const int32_t* __restrict__ dtok_s,
                                                                const float4* __restrict__ dl_s, uint32_t k,
                                                                uint32_t B, uint32_t V4, int32_t* __restrict__ dtok,
                                                                float4* __restrict__ dl)
{
    const uint32_t row = blockIdx.y;  // sequence-major row b k + j
    const uint32_t b = row / k, j = row - b * k;
    const float4* src = dl_s + (size_t)(j * B + b) * V4;
    float4* dst = dl + (size_t)row * V4;
    for (uint32_t q = blockIdx.x * 256 + threadIdx.x; q < V4; q += gridDim.x * 256) dst[q] = src[q];
    if (blockIdx.x == 0 && threadIdx.x == 0) dtok[row] = dtok_s[j * B + b];
}

// Tree step: the 2n - 1 uniforms, the draft's first row t_{n-2} and the root t_{n-1}.
__global__ void spec_tree_begin_kernel(const int32_t* __restrict__ npos, const int32_t* __restrict__ seq,
                                       const SpecState* __restrict__ st, uint64_t seed, uint32_t n,
                                       float* __restrict__ unif, int32_t* __restrict__ trow)
{
    const uint64_t step = st[0].step;
    for (uint32_t j = threadIdx.x; j < 2 * n - 1; j += blockDim.x)
        unif[j] = counter_uniform(seed, step * (2 * n - 1) + j);
    if (threadIdx.x == 0) {
        trow[0] = seq[npos[0] - 2];
        trow[1] = seq[npos[0] - 1];
    }
}

// One thread per sequence: append its n_acc + 1 tokens.
__global__ void spec_commit_kernel(SpecState* __restrict__ st, int32_t* __restrict__ npos, int32_t* __restrict__ seq,
                                   uint32_t cap, const int32_t* __restrict__ out_tok, const int32_t* __restrict__ nacc,
                                   uint32_t k, uint32_t kout, uint32_t B)
{
    const uint32_t b = threadIdx.x;
    if (b >= B) return;
    const int32_t a = nacc[b];
    const int32_t n = npos[b];
    for (int32_t i = 0; i <= a; ++i) seq[(size_t)b * cap + n + i] = out_tok[b * (kout + 1) + i];
    npos[b] = n + a + 1;
    st[b].n = n + a + 1;
    st[b].step += 1;
    st[b].accepted += (uint64_t)a;
    st[b].proposed += k;
}

__global__ void spec_reset_kernel(SpecState* st, int32_t* npos, const int32_t* __restrict__ n, uint32_t B)
{
    const uint32_t b = threadIdx.x;
    if (b >= B) return;
    st[b].n = n[b];
    st[b].pad = 0;
    st[b].step = 0;
    st[b].accepted = 0;
    st[b].proposed = 0;
    npos[b] = n[b];
}

}  // namespace

struct ulspec_spec {
    ulspec_ctx* ctx = nullptr;
    ulspec_model* t = nullptr;
    ulspec_model* d = nullptr;
    uint32_t k = 0, V = 0, cap = 0, B = 1;
    ulspec_sampling s{};
    uint64_t seed = 0;
    SpecState* st = nullptr;   // [B]
    int32_t* npos = nullptr;   // [B] committed tokens (the forwards' positions)
    int32_t* nset = nullptr;   // [B] prefill lengths
    int32_t* seq = nullptr;    // [B][cap]
    int32_t* tok_d = nullptr;  // [B][2]
    int32_t* dtok_s = nullptr; // [k][B]
    int32_t* dtok = nullptr;   // [B][k] (== dtok_s when B = 1)
    int32_t* tok_t = nullptr;  // [B][k+1]
    int32_t* out_tok = nullptr;  // [B][k+1]
    int32_t* nacc = nullptr;   // [B]
    int32_t* zero = nullptr;   // [B] zeros: the accepted counts of a plain step
    float* unif = nullptr;     // [B][2k+1]
    float* udraft = nullptr;   // [max(k, 1)][B]
    float* uacc = nullptr;     // [B][k+1]
    float* dl_s = nullptr;     // [k][B][V] (draft logits, step-major)
    float* dlogits = nullptr;  // [B][k][V] (== dl_s when B = 1)
    float* tlogits = nullptr;  // [B][k+1][V]
    void* ws_accept = nullptr;
    void* ws_sample = nullptr;
    SpecState* host_st = nullptr;  // pinned [B]
    std::vector<void*> allocs;
    bool prefilled = false;
    bool plain_first = false;  // one-token prompt: the next step is a plain step
    bool use_graph = true;
    hipGraphExec_t graph = nullptr;
    void* graph_ws = nullptr;       // context workspace the graph was captured with
    uint32_t n_hi = 0;              // upper bound of the longest committed count
    // tree steps
    bool tree = false;
    uint32_t depth = 0;                 // levels below the root
    std::vector<int32_t> parent_h;      // [n] the tree (target forward, acceptance)
    std::vector<int32_t> dparent_h;     // [n + 1] the draft's rows: t_{n-2}, then the tree under it
    std::vector<uint32_t> lv_first, lv_count;  // nodes of each level
    int32_t* trow = nullptr;            // [n + 1]: t_{n-2}, then the n node tokens
    int32_t* tmap = nullptr;            // [n] child -> its parent's row among its level's logits
    int32_t* kid_first = nullptr;       // [n] first child of each node
    int32_t* kid_count = nullptr;       // [n]
    int32_t* path = nullptr;            // [n]
    ulspec_status enqueue_step();
    ulspec_status launch_step();
    ulspec_status launch_plain_step();
    ulspec_status launch_tree_step();
    ulspec_status sync_state();
    ulspec_status prefill(const int32_t* prompts, const uint32_t* lens);
};

ulspec_status ulspec_spec::launch_plain_step()
{
    hipStream_t stream = ctx->stream;
    hipLaunchKernelGGL(spec_plain_begin_kernel, dim3(1), dim3(64), 0, stream, (const int32_t*)npos,
                       (const int32_t*)seq, cap, (const SpecState*)st, seed, k, B, unif, udraft, tok_t);
    ulspec_status r = t->forward(tok_t, B, npos, -1, tlogits, 1, nullptr, B, 0);
    if (r == ULSPEC_OK) r = sample_launch(ctx, &s, B, V, tlogits, udraft, out_tok, ws_sample);
    if (r != ULSPEC_OK) return r;
    hipLaunchKernelGGL(spec_commit_kernel, dim3(1), dim3(64), 0, stream, st, npos, seq, cap, (const int32_t*)out_tok,
                       (const int32_t*)zero, 0u, 0u, B);
    return check_launch(ctx, "plain step launch");
}

ulspec_status ulspec_spec::launch_tree_step()
{
    hipStream_t stream = ctx->stream;
    const uint32_t n = k + 1;
    hipLaunchKernelGGL(spec_tree_begin_kernel, dim3(1), dim3(64), 0, stream, (const int32_t*)npos, (const int32_t*)seq,
                       (const SpecState*)st, seed, n, unif, trow);
    ulspec_status r = ULSPEC_OK;
    for (uint32_t l = 0; l < depth && r == ULSPEC_OK; ++l) {
        const uint32_t f = lv_first[l], c = lv_count[l], rows = 1 + f + c;
        r = d->forward(trow, rows, npos, -2, dlogits + (size_t)f * V, c, dparent_h.data());
        if (r != ULSPEC_OK) break;
        const uint32_t f1 = lv_first[l + 1], c1 = lv_count[l + 1];
        if (s.greedy)
            topb_launch(ctx, dlogits + (size_t)f * V, V, c, kid_first + f, kid_count + f, trow + 1);
        else
            r = sample_mapped_launch(ctx, &s, c, V, dlogits + (size_t)f * V, c1, tmap + f1, unif + f1 - 1,
                                     trow + 1 + f1, ws_sample);
    }
    if (r == ULSPEC_OK) r = t->forward(trow + 1, n, npos, -1, tlogits, n, parent_h.data());
    if (r == ULSPEC_OK)
        r = accept_tree_launch(ctx, &s, 1, n, V, parent_h.data(), tlogits, dlogits, trow + 1, unif + n - 1, out_tok,
                               path, nacc, ws_accept);
    if (r != ULSPEC_OK) return r;
    launch_kv_compact(stream, t->kv_tab, t->cfg.n_layers, t->cfg.n_kv_heads * t->head_dim, t->cfg.max_ctx, npos, -1,
                      path, nacc, n);
    launch_kv_compact(stream, d->kv_tab, d->cfg.n_layers, d->cfg.n_kv_heads * d->head_dim, d->cfg.max_ctx, npos, -1,
                      path, nacc, n);
    hipLaunchKernelGGL(spec_commit_kernel, dim3(1), dim3(64), 0, stream, st, npos, seq, cap, (const int32_t*)out_tok,
                       (const int32_t*)nacc, depth, n - 1, 1u);
    return check_launch(ctx, "tree step launch");
}

ulspec_status ulspec_spec::launch_step()
{
    if (tree) return launch_tree_step();
    if (k == 0) return launch_plain_step();
    hipStream_t stream = ctx->stream;
    hipLaunchKernelGGL(spec_begin_kernel, dim3(1), dim3(256), 0, stream, (const int32_t*)npos, (const int32_t*)seq,
                       cap, (const SpecState*)st, seed, k, B, unif, udraft, uacc, tok_d);
    // draft: catch-up pair, then single tokens (B rows per forward, one per sequence)
    ulspec_status r = d->forward(tok_d, 2 * B, npos, -2, dl_s, 1, nullptr, B, 0);
    if (r == ULSPEC_OK) r = sample_launch(ctx, &s, B, V, dl_s, udraft, dtok_s, ws_sample);
    for (uint32_t j = 1; j < k && r == ULSPEC_OK; ++j) {
        r = d->forward(dtok_s + (j - 1) * B, B, npos, (int32_t)j - 1, dl_s + (size_t)j * B * V, 1, nullptr, B, 0);
        if (r == ULSPEC_OK)
            r = sample_launch(ctx, &s, B, V, dl_s + (size_t)j * B * V, udraft + j * B, dtok_s + j * B, ws_sample);
    }
    if (r != ULSPEC_OK) return r;
    hipLaunchKernelGGL(spec_verify_tokens_kernel, dim3(1), dim3(256), 0, stream, (const int32_t*)npos,
                       (const int32_t*)seq, cap, (const int32_t*)dtok_s, k, B, tok_t);
    r = t->forward(tok_t, (k + 1) * B, npos, -1, tlogits, k + 1, nullptr, B, 0);
    if (r != ULSPEC_OK) return r;
    if (B > 1)
        hipLaunchKernelGGL(spec_gather_draft_kernel, dim3((V / 4 + 255) / 256, B * k), dim3(256), 0, stream,
                           (const int32_t*)dtok_s, (const float4*)dl_s, k, B, V / 4, dtok, (float4*)dlogits);
    r = accept_launch(ctx, &s, B, k, V, tlogits, dlogits, dtok, uacc, out_tok, nacc, ws_accept);
    if (r != ULSPEC_OK) return r;
    hipLaunchKernelGGL(spec_commit_kernel, dim3(1), dim3(64), 0, stream, st, npos, seq, cap, (const int32_t*)out_tok,
                       (const int32_t*)nacc, k, k, B);
    return check_launch(ctx, "spec step launch");
}

ulspec_status ulspec_spec::enqueue_step()
{
    if (!use_graph) return launch_step();
    if (graph && graph_ws != ctx->ws) {  // the context workspace moved: capture again
        (void)hipGraphExecDestroy(graph);
        graph = nullptr;
    }
    if (!graph) {
        hipError_t e = hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal);
        if (e != hipSuccess) return hip_fail(ctx, e, "spec step capture begin");
        ulspec_status r = launch_step();
        hipGraph_t g = nullptr;
        e = hipStreamEndCapture(ctx->stream, &g);
        if (r != ULSPEC_OK) {
            if (g) (void)hipGraphDestroy(g);
            return r;
        }
        if (e != hipSuccess) return hip_fail(ctx, e, "spec step capture end");
        e = hipGraphInstantiate(&graph, g, nullptr, nullptr, 0);
        (void)hipGraphDestroy(g);
        if (e != hipSuccess) {
            graph = nullptr;
            return hip_fail(ctx, e, "spec step graph instantiate");
        }
        graph_ws = ctx->ws;
    }
    hipError_t e = hipGraphLaunch(graph, ctx->stream);
    return e == hipSuccess ? ULSPEC_OK : hip_fail(ctx, e, "spec step graph launch");
}

ulspec_status ulspec_spec::sync_state()
{
    hipError_t e = hipMemcpyAsync(host_st, st, B * sizeof(SpecState), hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "spec state sync");
    n_hi = 0;
    for (uint32_t b = 0; b < B; ++b) n_hi = std::max(n_hi, (uint32_t)host_st[b].n);
    return ULSPEC_OK;
}

// Prompts of every sequence (concatenated, lens[b] tokens each): both models
// process tokens 0 .. n_b - 2 on the sequence's slot; counters reset.
ulspec_status ulspec_spec::prefill(const int32_t* prompts, const uint32_t* lens)
{
    const uint32_t min_len = k > 0 && B > 1 ? 2 : 1;
    size_t off = 0;
    for (uint32_t b = 0; b < B; ++b) {
        if (lens[b] < min_len)
            return fail(ctx, ULSPEC_EINVAL, "spec_prefill: sequence %u has %u tokens (at least %u)", b, lens[b],
                        min_len);
        if ((uint64_t)lens[b] + k + 1 > cap)
            return fail(ctx, ULSPEC_EINVAL, "spec_prefill: %u tokens leave no room", lens[b]);
        for (uint32_t i = 0; i < lens[b]; ++i)
            if (prompts[off + i] < 0 || (uint32_t)prompts[off + i] >= V)
                return fail(ctx, ULSPEC_EINVAL, "spec_prefill: token %d out of range", prompts[off + i]);
        off += lens[b];
    }
    (void)hipSetDevice(ctx->device);
    if (hipMemset(nacc, 0, 4 * B) != hipSuccess) return fail(ctx, ULSPEC_EDEVICE, "spec_prefill: reset");
    std::vector<int32_t> n(B);
    off = 0;
    for (uint32_t b = 0; b < B; ++b) {
        const uint32_t nb = lens[b];
        ulspec_status st_ = ULSPEC_OK;
        if (nb > 1) {
            st_ = t->forward_host(prompts + off, nb - 1, 0, nullptr, 0, b);
            if (st_ == ULSPEC_OK && d) st_ = d->forward_host(prompts + off, nb - 1, 0, nullptr, 0, b);
            if (st_ != ULSPEC_OK) return st_;
        }
        hipError_t e = hipMemcpy(seq + (size_t)b * cap, prompts + off, (size_t)nb * 4, hipMemcpyHostToDevice);
        if (e != hipSuccess) return hip_fail(ctx, e, "spec_prefill copy");
        n[b] = (int32_t)nb;
        off += nb;
    }
    hipError_t e = hipMemcpy(nset, n.data(), B * sizeof(int32_t), hipMemcpyHostToDevice);
    if (e != hipSuccess) return hip_fail(ctx, e, "spec_prefill copy");
    hipLaunchKernelGGL(spec_reset_kernel, dim3(1), dim3(64), 0, ctx->stream, st, npos, (const int32_t*)nset, B);
    ulspec_status r = check_launch(ctx, "spec_prefill launch");
    if (r != ULSPEC_OK) return r;
    prefilled = true;
    plain_first = B == 1 && lens[0] == 1 && k > 0;
    return sync_state();
}

// tree: the caller sizes and allocates the acceptance and draw workspaces
// (those of a tree step), so the chain step's are not allocated here.
static ulspec_status spec_create(ulspec_model* target, ulspec_model* draft, uint32_t k, const ulspec_sampling* s,
                                 uint64_t seed, uint32_t B, ulspec_spec** out, bool tree = false)
{
    if (!target || (!draft && k > 0)) return ULSPEC_EINVAL;
    ulspec_ctx* ctx = target->ctx;
    if (k == 0) draft = nullptr;  // plain decoding of the target: no draft model
    if (draft && draft->ctx != ctx) return fail(ctx, ULSPEC_EINVAL, "spec_create: models on different contexts");
    if (!s || !out) return fail(ctx, ULSPEC_EINVAL, "spec_create: null pointer");
    if (B == 0 || B > (uint32_t)kMaxSeqs || target->n_seq < B || (draft && draft->n_seq < B))
        return fail(ctx, ULSPEC_EINVAL, "spec_create: %u sequences (1 .. %d, and at most the models' slots)", B,
                    kMaxSeqs);
    if (k + 1 > target->rows_max || (k + 1) * B > target->rows_cap ||
        (draft && (draft->rows_max < 2 || 2 * B > draft->rows_cap)))
        return fail(ctx, ULSPEC_EINVAL, "spec_create: k=%u for %u sequences (k <= %u, (k + 1) B <= %u target rows)", k,
                    B, target->rows_max - 1, target->rows_cap);
    if (draft && target->cfg.vocab != draft->cfg.vocab)
        return fail(ctx, ULSPEC_EINVAL, "spec_create: vocabularies differ");
    if (!target->complete() || (draft && !draft->complete()))
        return fail(ctx, ULSPEC_EINVAL, "spec_create: model tensors missing");
    const uint32_t V = target->cfg.vocab;
    if (B > 1 && V % 4) return fail(ctx, ULSPEC_EUNSUPPORTED, "spec_create: batches need a vocabulary multiple of 4");
    // the sampling parameters are validated by a dry check of the accept rule's limits
    if (!s->greedy) {
        if (!(s->temperature > 0.0f) || !(s->temperature < __builtin_inff()))
            return fail(ctx, ULSPEC_EINVAL, "spec_create: temperature must be positive and finite");
        if (!(s->top_p == s->top_p)) return fail(ctx, ULSPEC_EINVAL, "spec_create: top_p is NaN");
    }
    (void)hipSetDevice(ctx->device);
    ulspec_spec* sp = new ulspec_spec;
    sp->ctx = ctx;
    sp->t = target;
    sp->d = draft;
    sp->k = k;
    sp->V = V;
    sp->B = B;
    sp->s = *s;
    sp->seed = seed;
    sp->cap = draft ? std::min(target->cfg.max_ctx, draft->cfg.max_ctx) : target->cfg.max_ctx;
    const size_t kk = std::max<uint32_t>(k, 1);
    struct Want {
        void** p;
        size_t bytes;
    } wants[] = {
        {(void**)&sp->st, B * sizeof(SpecState)},
        {(void**)&sp->npos, 4 * B},
        {(void**)&sp->nset, 4 * B},
        {(void**)&sp->seq, (size_t)B * sp->cap * 4},
        {(void**)&sp->tok_d, 8 * B},
        {(void**)&sp->dtok_s, 4 * kk * B},
        {(void**)&sp->dtok, B > 1 ? 4 * kk * B : 0},
        {(void**)&sp->tok_t, 4 * (size_t)(k + 1) * B},
        {(void**)&sp->out_tok, 4 * (size_t)(k + 1) * B},
        {(void**)&sp->nacc, 4 * B},
        {(void**)&sp->zero, 4 * B},
        {(void**)&sp->unif, 4 * (size_t)(2 * k + 1) * B},
        {(void**)&sp->udraft, 4 * kk * B},
        {(void**)&sp->uacc, 4 * (size_t)(k + 1) * B},
        {(void**)&sp->dl_s, (size_t)k * B * V * 4},
        {(void**)&sp->dlogits, B > 1 ? (size_t)k * B * V * 4 : 0},
        {(void**)&sp->tlogits, (size_t)(k + 1) * B * V * 4},
        {(void**)&sp->ws_accept, k && !tree ? accept_workspace_bytes(B, k) : 0},
        {(void**)&sp->ws_sample, tree ? 0 : sample_workspace_bytes(B)},
    };
    ulspec_status st = ULSPEC_OK;
    for (const Want& w : wants) {
        if (st != ULSPEC_OK) break;
        if (!w.bytes) continue;  // k = 0: no draft rows, no acceptance; B = 1: no re-layout
        hipError_t e = hipMalloc(w.p, w.bytes);
        if (e != hipSuccess) st = hip_fail(ctx, e, "spec_create hipMalloc");
        else sp->allocs.push_back(*w.p);
    }
    if (st == ULSPEC_OK && B == 1) {  // the accept rule reads the step-major buffers directly
        sp->dtok = sp->dtok_s;
        sp->dlogits = sp->dl_s;
    }
    if (st == ULSPEC_OK) {
        hipError_t e = hipMemset(sp->zero, 0, 4 * B);
        if (e == hipSuccess) e = hipMemset(sp->nacc, 0, 4 * B);
        if (e == hipSuccess) e = hipMemset(sp->st, 0, B * sizeof(SpecState));  // no tokens before the prefill
        if (e == hipSuccess) e = hipHostMalloc((void**)&sp->host_st, B * sizeof(SpecState), hipHostMallocDefault);
        if (e != hipSuccess) st = hip_fail(ctx, e, "spec_create hipHostMalloc");
    }
    if (st != ULSPEC_OK) {
        ulspec_spec_destroy(sp);
        return st;
    }
    *out = sp;
    return ULSPEC_OK;
}

extern "C" ulspec_status ulspec_spec_create(ulspec_model* target, ulspec_model* draft, uint32_t k,
                                            const ulspec_sampling* s, uint64_t seed, ulspec_spec** out)
{
    return spec_create(target, draft, k, s, seed, 1, out);
}

extern "C" ulspec_status ulspec_spec_create_batch(ulspec_model* target, ulspec_model* draft, uint32_t k,
                                                  const ulspec_sampling* s, uint64_t seed, uint32_t n_seq,
                                                  ulspec_spec** out)
{
    return spec_create(target, draft, k, s, seed, n_seq, out);
}

extern "C" ulspec_status ulspec_spec_create_tree(ulspec_model* target, ulspec_model* draft, uint32_t n,
                                                 const int32_t* parent, const ulspec_sampling* s, uint64_t seed,
                                                 ulspec_spec** out)
{
    if (!target || !draft || !out) return ULSPEC_EINVAL;
    ulspec_ctx* ctx = target->ctx;
    if (!parent || n < 2 || n > ulspec_model::kRows)
        return fail(ctx, ULSPEC_EINVAL, "spec_create_tree: %u nodes (2 .. %u) and a parent array", n,
                    ulspec_model::kRows);
    // breadth-first order: parents before children, depths non-decreasing,
    // the children of a node consecutive
    std::vector<int32_t> depth(n, 0), first(n, -1), count(n, 0);
    if (parent[0] != -1) return fail(ctx, ULSPEC_EINVAL, "spec_create_tree: parent[0] must be -1");
    for (uint32_t i = 1; i < n; ++i) {
        const int32_t p = parent[i];
        if (p < 0 || p >= (int32_t)i) return fail(ctx, ULSPEC_EINVAL, "spec_create_tree: parent[%u]=%d", i, p);
        depth[i] = depth[p] + 1;
        if (depth[i] < depth[i - 1] || (first[p] >= 0 && first[p] + count[p] != (int32_t)i) ||
            (i > 1 && parent[i - 1] > p))
            return fail(ctx, ULSPEC_EINVAL, "spec_create_tree: nodes must be in breadth-first order (node %u)", i);
        if (first[p] < 0) first[p] = (int32_t)i;
        ++count[p];
    }
    ulspec_status st = spec_create(target, draft, n - 1, s, seed, 1, out, true);
    if (st != ULSPEC_OK) return st;
    ulspec_spec* sp = *out;
    sp->tree = true;
    sp->depth = (uint32_t)depth[n - 1];
    sp->parent_h.assign(parent, parent + n);
    sp->dparent_h.resize(n + 1);
    sp->dparent_h[0] = -1;
    for (uint32_t i = 0; i < n; ++i) sp->dparent_h[1 + i] = (int32_t)(parent[i] + 1);
    sp->lv_first.assign(sp->depth + 1, 0);
    sp->lv_count.assign(sp->depth + 1, 0);
    for (uint32_t i = 0; i < n; ++i) {
        if (sp->lv_count[depth[i]]++ == 0) sp->lv_first[depth[i]] = i;
    }
    std::vector<int32_t> tmap(n, 0), kf(n, 0), kc(n, 0);
    for (uint32_t i = 1; i < n; ++i) tmap[i] = parent[i] - (int32_t)sp->lv_first[depth[i] - 1];
    for (uint32_t i = 0; i < n; ++i) {
        kf[i] = first[i] < 0 ? 0 : first[i];
        kc[i] = count[i];
    }
    struct Want {
        void** p;
        size_t bytes;
        const void* init;
    } wants[] = {
        {(void**)&sp->trow, 4 * (size_t)(n + 1), nullptr}, {(void**)&sp->tmap, 4 * (size_t)n, tmap.data()},
        {(void**)&sp->kid_first, 4 * (size_t)n, kf.data()}, {(void**)&sp->kid_count, 4 * (size_t)n, kc.data()},
        {(void**)&sp->path, 4 * (size_t)n, nullptr},
    };
    for (const Want& w : wants) {
        hipError_t e = hipMalloc(w.p, w.bytes);
        if (e == hipSuccess) sp->allocs.push_back(*w.p);
        if (e == hipSuccess && w.init) e = hipMemcpy(*w.p, w.init, w.bytes, hipMemcpyHostToDevice);
        if (e != hipSuccess) st = hip_fail(ctx, e, "spec_create_tree");
        if (st != ULSPEC_OK) break;
    }
    // workspaces: the tree rule's, and the draws' over up to n - 1 parent rows of one level
    const size_t ws_bytes[2] = {accept_tree_workspace_bytes(1, n), sample_workspace_bytes(n)};
    void** ws_ptr[2] = {&sp->ws_accept, &sp->ws_sample};
    for (int i = 0; i < 2 && st == ULSPEC_OK; ++i) {
        void* ws = nullptr;
        hipError_t e = hipMalloc(&ws, ws_bytes[i]);
        if (e == hipSuccess) {
            sp->allocs.push_back(ws);
            *ws_ptr[i] = ws;
        } else {
            st = hip_fail(ctx, e, "spec_create_tree");
        }
    }
    if (st != ULSPEC_OK) {
        ulspec_spec_destroy(sp);
        *out = nullptr;
    }
    return st;
}

extern "C" ulspec_status ulspec_spec_tree_last_step(ulspec_spec* sp, float* target_logits, float* draft_logits,
                                                    int32_t* tokens, float* uniforms, int32_t* out_tokens,
                                                    int32_t* path, int32_t* n_accepted)
{
    if (!sp) return ULSPEC_EINVAL;
    ulspec_ctx* ctx = sp->ctx;
    if (!sp->tree) return fail(ctx, ULSPEC_EINVAL, "spec_tree_last_step: not a tree loop");
    (void)hipSetDevice(ctx->device);
    hipError_t e = hipStreamSynchronize(ctx->stream);
    const size_t n = sp->k + 1, V = sp->V;
    struct Copy {
        void* dst;
        const void* src;
        size_t bytes;
    } copies[] = {
        {target_logits, sp->tlogits, n * V * 4}, {draft_logits, sp->dlogits, (n - 1) * V * 4},
        {tokens, sp->trow + 1, n * 4},           {uniforms, sp->unif, (2 * n - 1) * 4},
        {out_tokens, sp->out_tok, n * 4},        {path, sp->path, n * 4},
        {n_accepted, sp->nacc, 4},
    };
    for (const Copy& c : copies)
        if (e == hipSuccess && c.dst && c.bytes) e = hipMemcpy(c.dst, c.src, c.bytes, hipMemcpyDeviceToHost);
    return e == hipSuccess ? ULSPEC_OK : hip_fail(ctx, e, "spec_tree_last_step copy");
}

extern "C" void ulspec_spec_destroy(ulspec_spec* sp)
{
    if (!sp) return;
    (void)hipSetDevice(sp->ctx->device);
    (void)hipStreamSynchronize(sp->ctx->stream);
    if (sp->graph) (void)hipGraphExecDestroy(sp->graph);
    for (void* p : sp->allocs) (void)hipFree(p);
    if (sp->host_st) (void)hipHostFree(sp->host_st);
    delete sp;
}

extern "C" ulspec_status ulspec_spec_prefill(ulspec_spec* sp, const int32_t* prompt, uint32_t n)
{
    if (!sp) return ULSPEC_EINVAL;
    if (sp->B != 1) return fail(sp->ctx, ULSPEC_EINVAL, "spec_prefill: %u sequences (ulspec_spec_prefill_batch)", sp->B);
    if (!prompt || n < 1) return fail(sp->ctx, ULSPEC_EINVAL, "spec_prefill: need at least 1 prompt token");
    return sp->prefill(prompt, &n);
}

extern "C" ulspec_status ulspec_spec_prefill_batch(ulspec_spec* sp, const int32_t* prompts, const uint32_t* lens)
{
    if (!sp) return ULSPEC_EINVAL;
    if (!prompts || !lens) return fail(sp->ctx, ULSPEC_EINVAL, "spec_prefill_batch: null pointer");
    return sp->prefill(prompts, lens);
}

extern "C" ulspec_status ulspec_spec_steps(ulspec_spec* sp, uint32_t n_steps)
{
    if (!sp) return ULSPEC_EINVAL;
    ulspec_ctx* ctx = sp->ctx;
    if (!sp->prefilled) return fail(ctx, ULSPEC_EINVAL, "spec_steps: no prefill");
    if (sp->tree && sp->plain_first) return fail(ctx, ULSPEC_EINVAL, "spec_steps: a tree loop needs 2 prompt tokens");
    (void)hipSetDevice(ctx->device);
    if ((uint64_t)sp->n_hi + (uint64_t)n_steps * (sp->k + 1) > sp->cap) {
        ulspec_status st = sp->sync_state();
        if (st != ULSPEC_OK) return st;
        if ((uint64_t)sp->n_hi + (uint64_t)n_steps * (sp->k + 1) > sp->cap)
            return fail(ctx, ULSPEC_EINVAL, "spec_steps: %u steps could pass the context of %u (at %u)", n_steps,
                        sp->cap, sp->n_hi);
    }
    for (uint32_t i = 0; i < n_steps; ++i) {
        ulspec_status st;
        if (sp->plain_first) {  // direct launches: the graph holds the speculative step
            st = sp->launch_plain_step();
            sp->plain_first = false;
        } else {
            st = sp->enqueue_step();
        }
        if (st != ULSPEC_OK) return st;
        sp->n_hi += sp->k + 1;
    }
    return ULSPEC_OK;
}

extern "C" ulspec_status ulspec_spec_generate(ulspec_spec* sp, uint32_t n_new, uint32_t* n_out)
{
    if (!sp) return ULSPEC_EINVAL;
    ulspec_ctx* ctx = sp->ctx;
    if (!sp->prefilled) return fail(ctx, ULSPEC_EINVAL, "spec_generate: no prefill");
    ulspec_status st = sp->sync_state();
    if (st != ULSPEC_OK) return st;
    std::vector<uint32_t> start(sp->B);
    for (uint32_t b = 0; b < sp->B; ++b) start[b] = (uint32_t)sp->host_st[b].n;
    uint32_t produced = 0;  // by the sequence that has produced the fewest
    while (produced < n_new) {
        // as many steps as cannot pass n_new (each commits <= k+1), at least one
        const uint32_t r = std::max<uint32_t>(1, (n_new - produced) / (sp->k + 1));
        st = ulspec_spec_steps(sp, r);
        if (st != ULSPEC_OK) return st;
        st = sp->sync_state();
        if (st != ULSPEC_OK) return st;
        produced = ~0u;
        for (uint32_t b = 0; b < sp->B; ++b) produced = std::min(produced, (uint32_t)sp->host_st[b].n - start[b]);
    }
    if (n_out) *n_out = produced;
    return ULSPEC_OK;
}

extern "C" ulspec_status ulspec_spec_state(ulspec_spec* sp, uint32_t* n_tokens, uint64_t* steps, uint64_t* accepted,
                                           uint64_t* proposed)
{
    if (!sp) return ULSPEC_EINVAL;
    (void)hipSetDevice(sp->ctx->device);
    ulspec_status st = sp->sync_state();
    if (st != ULSPEC_OK) return st;
    uint64_t n = 0, acc = 0, prop = 0;
    for (uint32_t b = 0; b < sp->B; ++b) {
        n += (uint64_t)sp->host_st[b].n;
        acc += sp->host_st[b].accepted;
        prop += sp->host_st[b].proposed;
    }
    if (n_tokens) *n_tokens = (uint32_t)n;
    if (steps) *steps = sp->host_st[0].step;
    if (accepted) *accepted = acc;
    if (proposed) *proposed = prop;
    return ULSPEC_OK;
}

extern "C" ulspec_status ulspec_spec_seq_state(ulspec_spec* sp, uint32_t seq, uint32_t* n_tokens, uint64_t* accepted,
                                               uint64_t* proposed)
{
    if (!sp) return ULSPEC_EINVAL;
    if (seq >= sp->B) return fail(sp->ctx, ULSPEC_EINVAL, "spec_seq_state: sequence %u of %u", seq, sp->B);
    (void)hipSetDevice(sp->ctx->device);
    ulspec_status st = sp->sync_state();
    if (st != ULSPEC_OK) return st;
    if (n_tokens) *n_tokens = (uint32_t)sp->host_st[seq].n;
    if (accepted) *accepted = sp->host_st[seq].accepted;
    if (proposed) *proposed = sp->host_st[seq].proposed;
    return ULSPEC_OK;
}

extern "C" ulspec_status ulspec_spec_seq_tokens(ulspec_spec* sp, uint32_t seq, uint32_t start, uint32_t n,
                                                int32_t* out)
{
    if (!sp) return ULSPEC_EINVAL;
    ulspec_ctx* ctx = sp->ctx;
    if (seq >= sp->B) return fail(ctx, ULSPEC_EINVAL, "spec_tokens: sequence %u of %u", seq, sp->B);
    ulspec_status st = sp->sync_state();
    if (st != ULSPEC_OK) return st;
    if (!out || (uint64_t)start + n > (uint64_t)sp->host_st[seq].n)
        return fail(ctx, ULSPEC_EINVAL, "spec_tokens: %u+%u beyond %d committed", start, n, sp->host_st[seq].n);
    hipError_t e = n ? hipMemcpy(out, sp->seq + (size_t)seq * sp->cap + start, (size_t)n * 4, hipMemcpyDeviceToHost)
                     : hipSuccess;
    return e == hipSuccess ? ULSPEC_OK : hip_fail(ctx, e, "spec_tokens copy");
}

extern "C" ulspec_status ulspec_spec_tokens(ulspec_spec* sp, uint32_t start, uint32_t n, int32_t* out)
{
    return ulspec_spec_seq_tokens(sp, 0, start, n, out);
}

extern "C" ulspec_status ulspec_spec_last_step(ulspec_spec* sp, float* target_logits, float* draft_logits,
                                               int32_t* draft_tokens, float* uniforms, int32_t* out_tokens,
                                               int32_t* n_accepted)
{
    if (!sp) return ULSPEC_EINVAL;
    ulspec_ctx* ctx = sp->ctx;
    (void)hipSetDevice(ctx->device);
    hipError_t e = hipStreamSynchronize(ctx->stream);
    const size_t k = sp->k, V = sp->V, B = sp->B;
    struct Copy {
        void* dst;
        const void* src;
        size_t bytes;
    } copies[] = {
        {target_logits, sp->tlogits, B * (k + 1) * V * 4}, {draft_logits, sp->dlogits, B * k * V * 4},
        {draft_tokens, sp->dtok, B * k * 4},                {uniforms, sp->unif, B * (2 * k + 1) * 4},
        {out_tokens, sp->out_tok, B * (k + 1) * 4},         {n_accepted, sp->nacc, B * 4},
    };
    for (const Copy& c : copies)
        if (e == hipSuccess && c.dst && c.bytes) e = hipMemcpy(c.dst, c.src, c.bytes, hipMemcpyDeviceToHost);
    return e == hipSuccess ? ULSPEC_OK : hip_fail(ctx, e, "spec_last_step copy");
}

extern "C" ulspec_status ulspec_spec_set_graph(ulspec_spec* sp, int use_graph)
{
    if (!sp) return ULSPEC_EINVAL;
    sp->use_graph = use_graph != 0;
    return ULSPEC_OK;
}
