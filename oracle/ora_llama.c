/* ora_llama.c -- CPU restatement of the Llama-shaped verify forward and the
 * speculative decoding loop.  TEST INFRASTRUCTURE ONLY (checker and timed CPU
 * baseline); nothing in the product links it.
 *
 * Block order: src/inference/inference_engine.cpp:602-682.  Weight names:
 * src/inference/model.cpp:190-246.  Formulas and the fp16 rounding points
 * (Q and the K/V cache only) are listed in oracle.h.  The speculative step replaces the host callback loop
 * of src/inference/speculative_decoder.cpp:25-71 with the draft / verify /
 * accept sequence documented in oracle.h; the cumulative counters follow
 * update_acceptance_stats (:112-116). */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "ora_internal.h"
#include "oracle.h"

typedef struct {
    uint8_t *wq, *wk, *wv, *wo, *wg, *wu, *wd;
    int tq, tk, tv, to, tg, tu, td;
    float *attn_norm, *ffn_norm;
    uint16_t *kc, *vc; /* [max_ctx][Hkv*D] */
} ora_layer;

struct ora_llama {
    ora_llama_cfg c;
    int64_t D;
    int nthreads;
    ora_layer* L;
    uint8_t* embed;
    int embed_type;
    float* out_norm;
    uint8_t* wout;
    int tout;
    float* rope; /* [max_ctx][D/2][2] */
};

void ora_llama_set_threads(ora_llama* m, int nthreads)
{
    if (m) m->nthreads = nthreads > 0 ? nthreads : 1;
}

ora_llama* ora_llama_create(const ora_llama_cfg* cfg, int nthreads)
{
    if (!cfg || cfg->n_heads <= 0 || cfg->n_kv_heads <= 0 || cfg->n_heads % cfg->n_kv_heads ||
        cfg->dim % cfg->n_heads || cfg->n_layers <= 0 || cfg->max_ctx < 2)
        return NULL;
    ora_llama* m = (ora_llama*)calloc(1, sizeof(ora_llama));
    m->c = *cfg;
    m->D = cfg->dim / cfg->n_heads;
    m->nthreads = nthreads > 0 ? nthreads : 1;
    m->L = (ora_layer*)calloc((size_t)cfg->n_layers, sizeof(ora_layer));
    size_t kv = (size_t)cfg->max_ctx * (size_t)(cfg->n_kv_heads * m->D);
    for (int64_t l = 0; l < cfg->n_layers; ++l) {
        m->L[l].kc = (uint16_t*)calloc(kv, sizeof(uint16_t));
        m->L[l].vc = (uint16_t*)calloc(kv, sizeof(uint16_t));
    }
    int64_t half = m->D / 2;
    m->rope = (float*)malloc(sizeof(float) * 2 * (size_t)(cfg->max_ctx * half));
    for (int64_t p = 0; p < cfg->max_ctx; ++p)
        for (int64_t i = 0; i < half; ++i) {
            double th = (double)p * pow((double)cfg->rope_base, -2.0 * (double)i / (double)m->D);
            m->rope[2 * (p * half + i)] = (float)cos(th);
            m->rope[2 * (p * half + i) + 1] = (float)sin(th);
        }
    return m;
}

void ora_llama_free(ora_llama* m)
{
    if (!m) return;
    for (int64_t l = 0; l < m->c.n_layers; ++l) {
        ora_layer* L = &m->L[l];
        free(L->wq); free(L->wk); free(L->wv); free(L->wo); free(L->wg); free(L->wu); free(L->wd);
        free(L->attn_norm); free(L->ffn_norm); free(L->kc); free(L->vc);
    }
    free(m->L); free(m->embed); free(m->out_norm); free(m->wout); free(m->rope);
    free(m);
}

static int ends_with(const char* s, const char* t)
{
    size_t a = strlen(s), b = strlen(t);
    return a >= b && strcmp(s + a - b, t) == 0;
}

int ora_llama_set_tensor(ora_llama* m, const char* name, int type, const void* data, size_t nbytes,
                         int64_t ne0, int64_t ne1)
{
    if (!m || !name || !data) return -1;
    const ora_llama_cfg* c = &m->c;
    int64_t H = c->n_heads, Hkv = c->n_kv_heads, D = m->D;
    void* copy = malloc(nbytes);
    memcpy(copy, data, nbytes);
    int64_t layer = -1;
    const char* base = name;
    if (strncmp(name, "blk.", 4) == 0) {
        layer = strtol(name + 4, (char**)&base, 10);
        if (*base != '.' || layer < 0 || layer >= c->n_layers) { free(copy); return -1; }
        ++base;
    }
    int is_norm = type == 0;
    size_t want = is_norm ? (size_t)(c->dim * 4) : ora_row_bytes(type, ne0) * (size_t)ne1;
    if (nbytes != want) { free(copy); return -1; }
    ora_layer* L = layer >= 0 ? &m->L[layer] : NULL;
#define SETW(ptr, tptr, e0, e1) do { if (ne0 != (e0) || ne1 != (e1)) { free(copy); return -1; } \
    free(ptr); ptr = (uint8_t*)copy; tptr = type; return 0; } while (0)
    if (!L) {
        if (strcmp(name, "token_embd.weight") == 0) {
            if (ne0 != c->dim || ne1 != c->vocab) { free(copy); return -1; }
            free(m->embed); m->embed = (uint8_t*)copy; m->embed_type = type; return 0;
        }
        if (strcmp(name, "output_norm.weight") == 0 && is_norm) { free(m->out_norm); m->out_norm = (float*)copy; return 0; }
        if (strcmp(name, "output.weight") == 0) SETW(m->wout, m->tout, c->dim, c->vocab);
        free(copy);
        return -1;
    }
    if (ends_with(base, "attn_norm.weight") && is_norm) { free(L->attn_norm); L->attn_norm = (float*)copy; return 0; }
    if (ends_with(base, "ffn_norm.weight") && is_norm) { free(L->ffn_norm); L->ffn_norm = (float*)copy; return 0; }
    if (strcmp(base, "attn_q.weight") == 0) SETW(L->wq, L->tq, c->dim, H * D);
    if (strcmp(base, "attn_k.weight") == 0) SETW(L->wk, L->tk, c->dim, Hkv * D);
    if (strcmp(base, "attn_v.weight") == 0) SETW(L->wv, L->tv, c->dim, Hkv * D);
    if (strcmp(base, "attn_output.weight") == 0) SETW(L->wo, L->to, H * D, c->dim);
    if (strcmp(base, "ffn_gate.weight") == 0) SETW(L->wg, L->tg, c->dim, c->ffn);
    if (strcmp(base, "ffn_up.weight") == 0) SETW(L->wu, L->tu, c->dim, c->ffn);
    if (strcmp(base, "ffn_down.weight") == 0) SETW(L->wd, L->td, c->ffn, c->dim);
#undef SETW
    free(copy);
    return -1;
}

/* one embedding row, dequantized exactly as the device kernel */
static void embed_row(const ora_llama* m, int32_t tok, float* h)
{
    int64_t dim = m->c.dim;
    if (tok < 0 || tok >= m->c.vocab) tok = 0;
    const uint8_t* row = m->embed + (size_t)tok * ora_row_bytes(m->embed_type, dim);
    ora_dequantize(m->embed_type, row, dim, h);
}

/* h += delta (if given); x = (h * r) * w */
static void add_rmsnorm(float* h, const float* delta, const float* w, int64_t M, int64_t dim, float eps, float* x)
{
    for (int64_t r = 0; r < M; ++r) {
        float* hr = h + r * dim;
        float ss = 0.0f;
        for (int64_t i = 0; i < dim; ++i) {
            if (delta) hr[i] = hr[i] + delta[r * dim + i];
            ss = fmaf(hr[i], hr[i], ss);
        }
        float rr = 1.0f / sqrtf(ss / (float)dim + eps);
        for (int64_t i = 0; i < dim; ++i) x[r * dim + i] = (hr[i] * rr) * w[i];
    }
}

static void rope_pair(const float* cs, float x0, float x1, uint16_t* y)
{
    float a = x0 * cs[0], b = x1 * cs[1];
    float c = x0 * cs[1], d = x1 * cs[0];
    y[0] = ora_f2h(a - b);
    y[1] = ora_f2h(c + d);
}

int ora_llama_forward(ora_llama* m, const int32_t* tokens, int64_t M, int64_t pos, float* logits, int64_t n_logits)
{
    const ora_llama_cfg* c = &m->c;
    int64_t dim = c->dim, H = c->n_heads, Hkv = c->n_kv_heads, D = m->D, F = c->ffn, V = c->vocab;
    if (M <= 0 || pos < 0 || pos + M > c->max_ctx || n_logits < 0 || n_logits > M || (n_logits && !logits)) return -1;
    int nt = m->nthreads;
    int64_t kvw = Hkv * D, xw = dim > F ? dim : F;
    float* h = (float*)malloc(sizeof(float) * (size_t)(M * dim));
    float* delta = (float*)malloc(sizeof(float) * (size_t)(M * dim));
    float* q = (float*)malloc(sizeof(float) * (size_t)(M * H * D));
    float* kk = (float*)malloc(sizeof(float) * (size_t)(M * kvw));
    float* vv = (float*)malloc(sizeof(float) * (size_t)(M * kvw));
    float* att = (float*)malloc(sizeof(float) * (size_t)(M * H * D));
    float* g = (float*)malloc(sizeof(float) * (size_t)(M * F));
    float* u = (float*)malloc(sizeof(float) * (size_t)(M * F));
    float* x = (float*)malloc(sizeof(float) * (size_t)(M * xw));
    uint16_t* q16 = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)(M * H * D));
    for (int64_t r = 0; r < M; ++r) embed_row(m, tokens[r], h + r * dim);
    float scale = 1.0f / sqrtf((float)D);
    for (int64_t l = 0; l < c->n_layers; ++l) {
        ora_layer* L = &m->L[l];
        add_rmsnorm(h, l ? delta : NULL, L->attn_norm, M, dim, c->rms_eps, x);
        ora_q4_gemm_x32(L->tq, L->wq, H * D, dim, x, M, q, nt);
        ora_q4_gemm_x32(L->tk, L->wk, kvw, dim, x, M, kk, nt);
        ora_q4_gemm_x32(L->tv, L->wv, kvw, dim, x, M, vv, nt);
        for (int64_t r = 0; r < M; ++r) {
            int64_t p = pos + r;
            const float* cs = m->rope + 2 * p * (D / 2);
            for (int64_t i = 0; i < H * D / 2; ++i)
                rope_pair(cs + 2 * (i % (D / 2)), q[r * H * D + 2 * i], q[r * H * D + 2 * i + 1], q16 + r * H * D + 2 * i);
            for (int64_t i = 0; i < kvw / 2; ++i)
                rope_pair(cs + 2 * (i % (D / 2)), kk[r * kvw + 2 * i], kk[r * kvw + 2 * i + 1], L->kc + p * kvw + 2 * i);
            for (int64_t i = 0; i < kvw; ++i) L->vc[p * kvw + i] = ora_f2h(vv[r * kvw + i]);
        }
        ora_attention_f32(q16, L->kc, L->vc, pos, M, NULL, H, Hkv, D, scale, att, nt);
        ora_q4_gemm_x32(L->to, L->wo, dim, H * D, att, M, delta, nt);
        add_rmsnorm(h, delta, L->ffn_norm, M, dim, c->rms_eps, x);
        ora_q4_gemm_x32(L->tg, L->wg, F, dim, x, M, g, nt);
        ora_q4_gemm_x32(L->tu, L->wu, F, dim, x, M, u, nt);
        for (int64_t i = 0; i < M * F; ++i) {
            float s = g[i] * (1.0f / (1.0f + ora_expf(-g[i])));
            x[i] = s * u[i];
        }
        ora_q4_gemm_x32(L->td, L->wd, dim, F, x, M, delta, nt);
    }
    add_rmsnorm(h, delta, m->out_norm, M, dim, c->rms_eps, x);
    if (n_logits) ora_q4_gemm_x32(m->tout, m->wout, V, dim, x + (M - n_logits) * dim, n_logits, logits, nt);
    free(h); free(delta); free(q); free(kk); free(vv); free(att); free(g); free(u); free(x); free(q16);
    return 0;
}

int ora_llama_kv_io(ora_llama* m, int64_t layer, int dir, int64_t pos0, int64_t n, uint16_t* k, uint16_t* v)
{
    if (!m || layer < 0 || layer >= m->c.n_layers || pos0 < 0 || n < 0 || pos0 + n > m->c.max_ctx) return -1;
    size_t row = (size_t)(m->c.n_kv_heads * m->D), bytes = (size_t)n * row * sizeof(uint16_t);
    uint16_t* kc = m->L[layer].kc + (size_t)pos0 * row;
    uint16_t* vc = m->L[layer].vc + (size_t)pos0 * row;
    if (dir == 0) { memcpy(k, kc, bytes); memcpy(v, vc, bytes); }
    else { memcpy(kc, k, bytes); memcpy(vc, v, bytes); }
    return 0;
}

int ora_spec_prefill(ora_llama* t, ora_llama* d, const int32_t* prompt, int64_t n, int32_t* seq, int64_t cap,
                     ora_spec_state* st)
{
    if (n < 1 || n > cap) return -1;
    if (n > 1 && (ora_llama_forward(t, prompt, n - 1, 0, NULL, 0) || (d && ora_llama_forward(d, prompt, n - 1, 0, NULL, 0))))
        return -1;
    memcpy(seq, prompt, sizeof(int32_t) * (size_t)n);
    st->n = n;
    st->step = st->accepted = st->proposed = 0;
    return 0;
}

int ora_spec_step(ora_llama* t, ora_llama* d, const ora_sampling* s, int64_t k, uint64_t seed, int32_t* seq,
                  int64_t cap, ora_spec_state* st)
{
    int64_t V = t->c.vocab, n = st->n;
    if (k < 0 || k > 15 || n < 1 || n + k + 1 > cap || (k > 0 && (!d || d->c.vocab != V))) return -1;
    if (k == 0 || n == 1) {
        /* plain step: t_n from warp(target logits of t_{n-1}) with counter step (2k+1) */
        float u0 = ora_uniform(seed, (uint64_t)(st->step * (2 * k + 1)));
        float* tl = (float*)malloc(sizeof(float) * (size_t)V);
        int32_t last = seq[n - 1], tok = 0;
        int rc = ora_llama_forward(t, &last, 1, n - 1, tl, 1);
        if (!rc) rc = ora_sample(s, 1, V, tl, &u0, &tok);
        free(tl);
        if (rc) return -1;
        seq[n] = tok;
        st->n = n + 1;
        st->step += 1;
        return 0;
    }
    float u[33];
    for (int64_t j = 0; j <= 2 * k; ++j) u[j] = ora_uniform(seed, (uint64_t)(st->step * (2 * k + 1) + j));
    float* dl = (float*)malloc(sizeof(float) * (size_t)(k * V));
    float* tl = (float*)malloc(sizeof(float) * (size_t)((k + 1) * V));
    int32_t dt[16], tt[16], out[16], nacc = 0;
    int32_t pair[2] = { seq[n - 2], seq[n - 1] };
    int rc = ora_llama_forward(d, pair, 2, n - 2, dl, 1);
    rc |= ora_sample(s, 1, V, dl, u, dt);
    for (int64_t j = 1; j < k && !rc; ++j) {
        rc |= ora_llama_forward(d, dt + j - 1, 1, n - 1 + j, dl + j * V, 1);
        rc |= ora_sample(s, 1, V, dl + j * V, u + j, dt + j);
    }
    tt[0] = seq[n - 1];
    for (int64_t j = 0; j < k; ++j) tt[j + 1] = dt[j];
    if (!rc) rc |= ora_llama_forward(t, tt, k + 1, n - 1, tl, k + 1);
    if (!rc) rc |= ora_accept(s, 1, k, V, tl, dl, dt, u + k, out, &nacc, 1);
    free(dl);
    free(tl);
    if (rc) return -1;
    for (int32_t i = 0; i <= nacc; ++i) seq[n + i] = out[i];
    st->n = n + nacc + 1;
    st->step += 1;
    st->accepted += nacc;
    st->proposed += k;
    return 0;
}

int64_t ora_spec_generate(ora_llama* t, ora_llama* d, const ora_sampling* s, int64_t k, uint64_t seed, int64_t n_new,
                          int32_t* seq, int64_t cap, ora_spec_state* st)
{
    int64_t start = st->n;
    while (st->n - start < n_new)
        if (ora_spec_step(t, d, s, k, seed, seq, cap, st)) return -1;
    return st->n - start;
}
