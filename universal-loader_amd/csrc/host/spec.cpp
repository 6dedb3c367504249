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

__global__ void spec_begin_kernel(const SpecState* __restrict__ st, const int32_t* __restrict__ seq, uint64_t seed,
                                  uint32_t k, float* __restrict__ unif, int32_t* __restrict__ tok_d)
{
    const uint32_t i = threadIdx.x;
    const uint64_t base = st->step * (2 * k + 1);
    if (i < 2 * k + 1) unif[i] = counter_uniform(seed, base + i);
    if (i == 0) {
        tok_d[0] = seq[st->n - 2];
        tok_d[1] = seq[st->n - 1];
    }
}

// Plain (target-only) step: the uniform of counter step (2k+1) and the last token.
__global__ void spec_plain_begin_kernel(const SpecState* __restrict__ st, const int32_t* __restrict__ seq,
                                        uint64_t seed, uint32_t k, float* __restrict__ unif,
                                        int32_t* __restrict__ tok_t)
{
    if (threadIdx.x != 0) return;
    unif[0] = counter_uniform(seed, st->step * (2 * k + 1));
    tok_t[0] = seq[st->n - 1];
}

__global__ void spec_verify_tokens_kernel(const SpecState* __restrict__ st, const int32_t* __restrict__ seq,
                                          const int32_t* __restrict__ dtok, uint32_t k, int32_t* __restrict__ tok_t)
{
    const uint32_t i = threadIdx.x;
    if (i == 0) tok_t[0] = seq[st->n - 1];
    else if (i <= k) tok_t[i] = dtok[i - 1];
}

__global__ void spec_commit_kernel(SpecState* __restrict__ st, int32_t* __restrict__ seq,
                                   const int32_t* __restrict__ out_tok, const int32_t* __restrict__ nacc, uint32_t k)
{
    if (threadIdx.x != 0) return;
    const int32_t a = *nacc;
    const int32_t n = st->n;
    for (int32_t i = 0; i <= a; ++i) seq[n + i] = out_tok[i];
    st->n = n + a + 1;
    st->step += 1;
    st->accepted += (uint64_t)a;
    st->proposed += k;
}

__global__ void spec_reset_kernel(SpecState* st, int32_t n)
{
    st->n = n;
    st->pad = 0;
    st->step = 0;
    st->accepted = 0;
    st->proposed = 0;
}

}  // namespace

struct ulspec_spec {
    ulspec_ctx* ctx = nullptr;
    ulspec_model* t = nullptr;
    ulspec_model* d = nullptr;
    uint32_t k = 0, V = 0, cap = 0;
    ulspec_sampling s{};
    uint64_t seed = 0;
    SpecState* st = nullptr;
    int32_t* seq = nullptr;
    int32_t* tok_d = nullptr;
    int32_t* dtok = nullptr;
    int32_t* tok_t = nullptr;
    int32_t* out_tok = nullptr;
    int32_t* nacc = nullptr;
    int32_t* zero = nullptr;  // 0: the accepted count of a plain step
    float* unif = nullptr;
    float* dlogits = nullptr;  // [k][V]
    float* tlogits = nullptr;  // [k+1][V]
    void* ws_accept = nullptr;
    void* ws_sample = nullptr;
    SpecState* host_st = nullptr;  // pinned
    std::vector<void*> allocs;
    bool prefilled = false;
    bool plain_first = false;  // one-token prompt: the next step is a plain step
    bool use_graph = true;
    hipGraphExec_t graph = nullptr;
    void* graph_ws = nullptr;       // context workspace the graph was captured with
    uint32_t n_hi = 0;              // upper bound of the committed count
    ulspec_status enqueue_step();
    ulspec_status launch_step();
    ulspec_status launch_plain_step();
    ulspec_status sync_state();
};

ulspec_status ulspec_spec::launch_plain_step()
{
    hipStream_t stream = ctx->stream;
    hipLaunchKernelGGL(spec_plain_begin_kernel, dim3(1), dim3(64), 0, stream, st, seq, seed, k, unif, tok_t);
    ulspec_status r = t->forward(tok_t, 1, &st->n, -1, tlogits, 1);
    if (r == ULSPEC_OK) r = sample_launch(ctx, &s, 1, V, tlogits, unif, out_tok, ws_sample);
    if (r != ULSPEC_OK) return r;
    hipLaunchKernelGGL(spec_commit_kernel, dim3(1), dim3(64), 0, stream, st, seq, out_tok, (const int32_t*)zero, 0u);
    return check_launch(ctx, "plain step launch");
}

ulspec_status ulspec_spec::launch_step()
{
    if (k == 0) return launch_plain_step();
    hipStream_t stream = ctx->stream;
    hipLaunchKernelGGL(spec_begin_kernel, dim3(1), dim3(64), 0, stream, st, seq, seed, k, unif, tok_d);
    // draft: catch-up pair, then single tokens
    ulspec_status r = d->forward(tok_d, 2, &st->n, -2, dlogits, 1);
    if (r == ULSPEC_OK) r = sample_launch(ctx, &s, 1, V, dlogits, unif, dtok, ws_sample);
    for (uint32_t j = 1; j < k && r == ULSPEC_OK; ++j) {
        r = d->forward(dtok + j - 1, 1, &st->n, (int32_t)j - 1, dlogits + (size_t)j * V, 1);
        if (r == ULSPEC_OK) r = sample_launch(ctx, &s, 1, V, dlogits + (size_t)j * V, unif + j, dtok + j, ws_sample);
    }
    if (r != ULSPEC_OK) return r;
    hipLaunchKernelGGL(spec_verify_tokens_kernel, dim3(1), dim3(32), 0, stream, st, seq, dtok, k, tok_t);
    r = t->forward(tok_t, k + 1, &st->n, -1, tlogits, k + 1);
    if (r == ULSPEC_OK)
        r = accept_launch(ctx, &s, 1, k, V, tlogits, dlogits, dtok, unif + k, out_tok, nacc, ws_accept);
    if (r != ULSPEC_OK) return r;
    hipLaunchKernelGGL(spec_commit_kernel, dim3(1), dim3(64), 0, stream, st, seq, out_tok, nacc, k);
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
    hipError_t e = hipMemcpyAsync(host_st, st, sizeof(SpecState), hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "spec state sync");
    n_hi = (uint32_t)host_st->n;
    return ULSPEC_OK;
}

extern "C" ulspec_status ulspec_spec_create(ulspec_model* target, ulspec_model* draft, uint32_t k,
                                            const ulspec_sampling* s, uint64_t seed, ulspec_spec** out)
{
    if (!target || (!draft && k > 0)) return ULSPEC_EINVAL;
    ulspec_ctx* ctx = target->ctx;
    if (k == 0) draft = nullptr;  // plain decoding of the target: no draft model
    if (draft && draft->ctx != ctx) return fail(ctx, ULSPEC_EINVAL, "spec_create: models on different contexts");
    if (!s || !out) return fail(ctx, ULSPEC_EINVAL, "spec_create: null pointer");
    if (k > 16 || k + 1 > target->rows_max || (draft && draft->rows_max < 2))
        return fail(ctx, ULSPEC_EINVAL, "spec_create: k=%u (k <= 16, k + 1 <= %u rows of the target)", k,
                    target->rows_max);
    if (draft && target->cfg.vocab != draft->cfg.vocab)
        return fail(ctx, ULSPEC_EINVAL, "spec_create: vocabularies differ");
    if (!target->complete() || (draft && !draft->complete()))
        return fail(ctx, ULSPEC_EINVAL, "spec_create: model tensors missing");
    const uint32_t V = target->cfg.vocab;
    // the sampling parameters are validated by a dry check of the accept rule's limits
    if (!s->greedy) {
        if (!(s->temperature > 0.0f) || !(s->temperature < __builtin_inff()))
            return fail(ctx, ULSPEC_EINVAL, "spec_create: temperature must be positive and finite");
        if (s->top_k > 256 && s->top_k < V) return fail(ctx, ULSPEC_EUNSUPPORTED, "spec_create: top_k > 256");
        if (!(s->top_p == s->top_p)) return fail(ctx, ULSPEC_EINVAL, "spec_create: top_p is NaN");
    }
    (void)hipSetDevice(ctx->device);
    ulspec_spec* sp = new ulspec_spec;
    sp->ctx = ctx;
    sp->t = target;
    sp->d = draft;
    sp->k = k;
    sp->V = V;
    sp->s = *s;
    sp->seed = seed;
    sp->cap = draft ? std::min(target->cfg.max_ctx, draft->cfg.max_ctx) : target->cfg.max_ctx;
    struct Want {
        void** p;
        size_t bytes;
    } wants[] = {
        {(void**)&sp->st, sizeof(SpecState)},
        {(void**)&sp->seq, (size_t)sp->cap * 4},
        {(void**)&sp->tok_d, 16},
        {(void**)&sp->dtok, 64},
        {(void**)&sp->tok_t, 64},
        {(void**)&sp->out_tok, 64},
        {(void**)&sp->nacc, 16},
        {(void**)&sp->zero, 16},
        {(void**)&sp->unif, 4 * (2 * 16 + 1)},
        {(void**)&sp->dlogits, (size_t)k * V * 4},
        {(void**)&sp->tlogits, (size_t)(k + 1) * V * 4},
        {(void**)&sp->ws_accept, k ? accept_workspace_bytes(1, k) : 0},
        {(void**)&sp->ws_sample, sample_workspace_bytes(1)},
    };
    ulspec_status st = ULSPEC_OK;
    for (const Want& w : wants) {
        if (st != ULSPEC_OK) break;
        if (!w.bytes) continue;  // k = 0: no draft rows, no acceptance
        hipError_t e = hipMalloc(w.p, w.bytes);
        if (e != hipSuccess) st = hip_fail(ctx, e, "spec_create hipMalloc");
        else sp->allocs.push_back(*w.p);
    }
    if (st == ULSPEC_OK) {
        hipError_t e = hipMemset(sp->zero, 0, 16);
        if (e == hipSuccess) e = hipMemset(sp->nacc, 0, 16);
        if (e == hipSuccess) e = hipMemset(sp->st, 0, sizeof(SpecState));  // no tokens before the prefill
        if (e == hipSuccess) e = hipHostMalloc((void**)&sp->host_st, sizeof(SpecState), hipHostMallocDefault);
        if (e != hipSuccess) st = hip_fail(ctx, e, "spec_create hipHostMalloc");
    }
    if (st != ULSPEC_OK) {
        ulspec_spec_destroy(sp);
        return st;
    }
    *out = sp;
    return ULSPEC_OK;
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
    ulspec_ctx* ctx = sp->ctx;
    if (!prompt || n < 1) return fail(ctx, ULSPEC_EINVAL, "spec_prefill: need at least 1 prompt token");
    if ((uint64_t)n + sp->k + 1 > sp->cap) return fail(ctx, ULSPEC_EINVAL, "spec_prefill: %u tokens leave no room", n);
    for (uint32_t i = 0; i < n; ++i)
        if (prompt[i] < 0 || (uint32_t)prompt[i] >= sp->V)
            return fail(ctx, ULSPEC_EINVAL, "spec_prefill: token %d out of range", prompt[i]);
    (void)hipSetDevice(ctx->device);
    ulspec_status st = ULSPEC_OK;
    if (hipMemset(sp->nacc, 0, 16) != hipSuccess) return fail(ctx, ULSPEC_EDEVICE, "spec_prefill: reset");
    if (n > 1) {
        st = ulspec_model_forward(sp->t, prompt, n - 1, 0, nullptr, 0);
        if (st == ULSPEC_OK && sp->d) st = ulspec_model_forward(sp->d, prompt, n - 1, 0, nullptr, 0);
        if (st != ULSPEC_OK) return st;
    }
    hipError_t e = hipMemcpy(sp->seq, prompt, (size_t)n * 4, hipMemcpyHostToDevice);
    if (e != hipSuccess) return hip_fail(ctx, e, "spec_prefill copy");
    hipLaunchKernelGGL(spec_reset_kernel, dim3(1), dim3(1), 0, ctx->stream, sp->st, (int32_t)n);
    st = check_launch(ctx, "spec_prefill launch");
    if (st != ULSPEC_OK) return st;
    sp->prefilled = true;
    sp->plain_first = n == 1 && sp->k > 0;
    return sp->sync_state();
}

extern "C" ulspec_status ulspec_spec_steps(ulspec_spec* sp, uint32_t n_steps)
{
    if (!sp) return ULSPEC_EINVAL;
    ulspec_ctx* ctx = sp->ctx;
    if (!sp->prefilled) return fail(ctx, ULSPEC_EINVAL, "spec_steps: no prefill");
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
    const uint32_t start = (uint32_t)sp->host_st->n;
    uint32_t produced = 0;
    while (produced < n_new) {
        // as many steps as cannot pass n_new (each commits <= k+1), at least one
        const uint32_t r = std::max<uint32_t>(1, (n_new - produced) / (sp->k + 1));
        st = ulspec_spec_steps(sp, r);
        if (st != ULSPEC_OK) return st;
        st = sp->sync_state();
        if (st != ULSPEC_OK) return st;
        produced = (uint32_t)sp->host_st->n - start;
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
    if (n_tokens) *n_tokens = (uint32_t)sp->host_st->n;
    if (steps) *steps = sp->host_st->step;
    if (accepted) *accepted = sp->host_st->accepted;
    if (proposed) *proposed = sp->host_st->proposed;
    return ULSPEC_OK;
}

extern "C" ulspec_status ulspec_spec_tokens(ulspec_spec* sp, uint32_t start, uint32_t n, int32_t* out)
{
    if (!sp) return ULSPEC_EINVAL;
    ulspec_ctx* ctx = sp->ctx;
    ulspec_status st = sp->sync_state();
    if (st != ULSPEC_OK) return st;
    if (!out || (uint64_t)start + n > (uint64_t)sp->host_st->n)
        return fail(ctx, ULSPEC_EINVAL, "spec_tokens: %u+%u beyond %d committed", start, n, sp->host_st->n);
    hipError_t e = hipMemcpy(out, sp->seq + start, (size_t)n * 4, hipMemcpyDeviceToHost);
    return e == hipSuccess ? ULSPEC_OK : hip_fail(ctx, e, "spec_tokens copy");
}

extern "C" ulspec_status ulspec_spec_last_step(ulspec_spec* sp, float* target_logits, float* draft_logits,
                                               int32_t* draft_tokens, float* uniforms, int32_t* out_tokens,
                                               int32_t* n_accepted)
{
    if (!sp) return ULSPEC_EINVAL;
    ulspec_ctx* ctx = sp->ctx;
    (void)hipSetDevice(ctx->device);
    hipError_t e = hipStreamSynchronize(ctx->stream);
    const size_t k = sp->k, V = sp->V;
    struct Copy {
        void* dst;
        const void* src;
        size_t bytes;
    } copies[] = {
        {target_logits, sp->tlogits, (k + 1) * V * 4}, {draft_logits, sp->dlogits, k * V * 4},
        {draft_tokens, sp->dtok, k * 4},                {uniforms, sp->unif, (2 * k + 1) * 4},
        {out_tokens, sp->out_tok, (k + 1) * 4},         {n_accepted, sp->nacc, 4},
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
