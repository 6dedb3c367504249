/*
 * ora_accept.c -- acceptance sampling of k drafted tokens (test infrastructure,
 * see oracle.h).
 *
 * Semantics (the device kernels implement the same arithmetic, operation for
 * operation, so tokens agree bit for bit on identical logits):
 *
 * Warp of one logit row l[0..V):
 *   lmax = max l;  invT = 1.0f / temperature (fp32 division);
 *   kept = all tokens, or the top_k by (logit desc, index asc) when 0 < top_k < V;
 *   e_i = expf_det((l_i - lmax) * invT)       -- temperature on max-subtracted
 *                                                logits, src/api/gguf_loader.cpp:98-100
 *   E_i = trunc(e_i * 2^S) (uint64) with S = 63 - bitlen(V) (48 at V = 32000,
 *   46 at V = 128256), so that Z = sum E_i < 2^63 is exact.
 *   top_p < 1: walk kept by (logit desc, index asc) accumulating C; keep up to
 *   and including the first token with (double)C >= (double)top_p * (double)Z;
 *   Z becomes the kept sum.
 *   Fixed-point sums are associative, so any reduction order gives the same Z.
 *
 * Inverse-CDF draw with uniform u over weights W with total Z (index order,
 * strict "<", fall back to the last index with nonzero weight; the convention of
 * src/inference/inference_engine.cpp:356-366):
 *   T = (uint64)((double)u * (double)Z); first i with T < cumsum_{j<=i} W_j.
 *
 * Speculative rule per sequence (Leviathan et al. 2023, Alg. 1): for i < k with
 * draft token x, p = warp(target row i), q = warp(draft row i):
 *   accept iff ((double)u_i * (double)Q_x) * (double)Zp < (double)P_x * (double)Zq
 *   (i.e. u_i * q(x) < p(x)).
 *   First rejection at i: residual r_j = max(0, P_j*Zq - Q_j*Zp) (double
 *   products and difference), scaled by 2^(62 - bitlen(Zp) - bitlen(Zq)) and
 *   truncated to uint64, then drawn with u_k; an all-zero residual draws from p.
 *   All k accepted: bonus token drawn from warp(target row k) with u_k.
 * Greedy: accept while argmax(target row i) == x_i (ties -> lowest index); emit
 * the argmax at the first mismatch, or argmax(target row k) as the bonus.
 * Output row: n_accepted + 1 tokens, then -1.
 */
#include "ora_internal.h"

#include <math.h>
#include <string.h>

typedef struct {
    float l;
    int32_t i;
} lk;

/* (logit desc, index asc) */
static inline int lk_before(lk a, lk b)
{
    return a.l > b.l || (a.l == b.l && a.i < b.i);
}

static int lk_cmp(const void* pa, const void* pb)
{
    lk a = *(const lk*)pa, b = *(const lk*)pb;
    if (lk_before(a, b)) return -1;
    if (lk_before(b, a)) return 1;
    return 0;
}

/* min-heap on "before": root is the element that comes last in the order */
static void heap_sift_down(lk* h, int n, int i)
{
    for (;;) {
        int l = 2 * i + 1, r = l + 1, m = i;
        if (l < n && lk_before(h[m], h[l])) m = l;
        if (r < n && lk_before(h[m], h[r])) m = r;
        if (m == i) return;
        lk t = h[i]; h[i] = h[m]; h[m] = t;
        i = m;
    }
}

static int bitlen64(uint64_t x)
{
    int n = 0;
    while (x) { ++n; x >>= 1; }
    return n;
}

/* fixed-point scale exponent of a row of V tokens */
int ora_warp_shift(int64_t V)
{
    return 63 - bitlen64((uint64_t)V);
}

static int64_t argmax_row(const float* l, int64_t V)
{
    int64_t a = 0;
    for (int64_t i = 1; i < V; ++i)
        if (l[i] > l[a]) a = i;
    return a;
}

int64_t ora_warp_row(const ora_sampling* s, const float* logits, int64_t V, uint64_t* E, uint64_t* Z)
{
    float lmax = logits[0];
    for (int64_t i = 1; i < V; ++i)
        if (logits[i] > lmax) lmax = logits[i];
    const float invT = 1.0f / s->temperature;
    memset(E, 0, sizeof(uint64_t) * (size_t)V);
    int64_t nk;
    lk* kept;
    if (s->top_k > 0 && (int64_t)s->top_k < V) {
        nk = s->top_k;
        kept = (lk*)malloc(sizeof(lk) * (size_t)nk);
        for (int64_t i = 0; i < nk; ++i) { kept[i].l = logits[i]; kept[i].i = (int32_t)i; }
        for (int64_t i = nk / 2 - 1; i >= 0; --i) heap_sift_down(kept, (int)nk, (int)i);
        for (int64_t i = nk; i < V; ++i) {
            lk c = { logits[i], (int32_t)i };
            if (lk_before(c, kept[0])) { kept[0] = c; heap_sift_down(kept, (int)nk, 0); }
        }
    } else {
        nk = V;
        kept = (lk*)malloc(sizeof(lk) * (size_t)nk);
        for (int64_t i = 0; i < V; ++i) { kept[i].l = logits[i]; kept[i].i = (int32_t)i; }
    }
    const float scale = ldexpf(1.0f, ora_warp_shift(V));
    uint64_t z = 0;
    for (int64_t t = 0; t < nk; ++t) {
        float e = ora_expf((kept[t].l - lmax) * invT);
        uint64_t q = (uint64_t)(e * scale);
        E[kept[t].i] = q;
        z += q;
    }
    if (s->top_p < 1.0f) {
        qsort(kept, (size_t)nk, sizeof(lk), lk_cmp);
        double thr = (double)s->top_p * (double)z;
        uint64_t c = 0;
        int64_t t = 0;
        for (; t < nk; ++t) {
            c += E[kept[t].i];
            if ((double)c >= thr) { ++t; break; }
        }
        for (int64_t r = t; r < nk; ++r) E[kept[r].i] = 0;
        z = c;
        nk = t;
    }
    free(kept);
    *Z = z;
    return nk;
}

int64_t ora_cdf_pick(const uint64_t* W, int64_t V, uint64_t Z, float u)
{
    uint64_t T = (uint64_t)((double)u * (double)Z);
    uint64_t c = 0;
    int64_t last = -1;
    for (int64_t i = 0; i < V; ++i) {
        if (W[i] == 0) continue;
        c += W[i];
        last = i;
        if (T < c) return i;
    }
    return last < 0 ? V - 1 : last;
}

typedef struct {
    const ora_sampling* s;
    int64_t k, V;
    const float *tl, *dl, *u;
    const int32_t* dt;
    int32_t *out, *nacc;
} accept_job;

static void accept_one(const accept_job* j, int64_t b, uint64_t* P, uint64_t* Q, uint64_t* R)
{
    const int64_t k = j->k, V = j->V;
    const float* tl = j->tl + (size_t)b * (size_t)(k + 1) * (size_t)V;
    const float* dl = j->dl ? j->dl + (size_t)b * (size_t)k * (size_t)V : NULL;
    const int32_t* x = j->dt + b * k;
    const float* u = j->u ? j->u + b * (k + 1) : NULL;
    int32_t* out = j->out + b * (k + 1);
    for (int64_t i = 0; i <= k; ++i) out[i] = -1;
    if (j->s->greedy) {
        for (int64_t i = 0; i < k; ++i) {
            int64_t a = argmax_row(tl + i * V, V);
            out[i] = (int32_t)a;
            if (a != x[i]) { j->nacc[b] = (int32_t)i; return; }
        }
        out[k] = (int32_t)argmax_row(tl + k * V, V);
        j->nacc[b] = (int32_t)k;
        return;
    }
    for (int64_t i = 0; i < k; ++i) {
        uint64_t Zp, Zq;
        ora_warp_row(j->s, tl + i * V, V, P, &Zp);
        ora_warp_row(j->s, dl + i * V, V, Q, &Zq);
        int32_t xi = x[i];
        uint64_t Px = (xi >= 0 && xi < V) ? P[xi] : 0;
        uint64_t Qx = (xi >= 0 && xi < V) ? Q[xi] : 0;
        double lhs = ((double)u[i] * (double)Qx) * (double)Zp;
        double rhs = (double)Px * (double)Zq;
        if (lhs < rhs) { out[i] = xi; continue; }
        int sh = 62 - bitlen64(Zp) - bitlen64(Zq);
        uint64_t SR = 0;
        for (int64_t t = 0; t < V; ++t) {
            double a = (double)P[t] * (double)Zq;
            double c = (double)Q[t] * (double)Zp;
            double r = a - c;
            R[t] = r > 0.0 ? (uint64_t)ldexp(r, sh) : 0;
            SR += R[t];
        }
        out[i] = (int32_t)(SR ? ora_cdf_pick(R, V, SR, u[k]) : ora_cdf_pick(P, V, Zp, u[k]));
        j->nacc[b] = (int32_t)i;
        return;
    }
    uint64_t Zp;
    ora_warp_row(j->s, tl + k * V, V, P, &Zp);
    out[k] = (int32_t)ora_cdf_pick(P, V, Zp, u[k]);
    j->nacc[b] = (int32_t)k;
}

static void accept_range(void* arg, int64_t lo, int64_t hi)
{
    accept_job* j = (accept_job*)arg;
    uint64_t* buf = (uint64_t*)malloc(sizeof(uint64_t) * 3u * (size_t)j->V);
    for (int64_t b = lo; b < hi; ++b) accept_one(j, b, buf, buf + j->V, buf + 2 * j->V);
    free(buf);
}

int ora_accept(const ora_sampling* s, int64_t B, int64_t k, int64_t V,
               const float* target_logits, const float* draft_logits,
               const int32_t* draft_tokens, const float* uniforms,
               int32_t* out_tokens, int32_t* out_n_accepted, int nthreads)
{
    if (B <= 0 || k < 0 || V <= 0 || !s || !target_logits || !out_tokens || !out_n_accepted) return -1;
    if (k > 0 && !draft_tokens) return -1;
    if (!s->greedy && (!uniforms || (k > 0 && !draft_logits) || !(s->temperature > 0.0f))) return -1;
    accept_job j = { s, k, V, target_logits, draft_logits, uniforms, draft_tokens, out_tokens, out_n_accepted };
    ora_parallel_for(nthreads, B, accept_range, &j);
    return 0;
}

typedef struct {
    const ora_sampling* s;
    int64_t V;
    const float *l, *u;
    int32_t* out;
} sample_job;

static void sample_range(void* arg, int64_t lo, int64_t hi)
{
    sample_job* j = (sample_job*)arg;
    uint64_t* P = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)j->V);
    for (int64_t r = lo; r < hi; ++r) {
        const float* l = j->l + (size_t)r * (size_t)j->V;
        if (j->s->greedy) {
            j->out[r] = (int32_t)argmax_row(l, j->V);
        } else {
            uint64_t Z;
            ora_warp_row(j->s, l, j->V, P, &Z);
            j->out[r] = (int32_t)ora_cdf_pick(P, j->V, Z, j->u[r]);
        }
    }
    free(P);
}

int ora_sample(const ora_sampling* s, int64_t R, int64_t V, const float* logits,
               const float* uniforms, int32_t* out_tokens)
{
    if (R <= 0 || V <= 0 || !s || !logits || !out_tokens) return -1;
    if (!s->greedy && (!uniforms || !(s->temperature > 0.0f))) return -1;
    sample_job j = { s, V, logits, uniforms, out_tokens };
    ora_parallel_for(1, R, sample_range, &j);
    return 0;
}

/*
 * Tree acceptance (multi-draft speculative sampling: SpecInfer, Miao et al.
 * 2024, Alg. 2, sibling drafts drawn with replacement from the draft row of
 * their parent).  Nodes 0 .. n-1, node 0 the root (the last committed token),
 * parent[i] < i for i >= 1.  Target row v = distribution after node v; draft
 * row v = the distribution node v's children were drawn from.  Walk from the
 * root; at node v, C = warp(target row v) with total Zc, q = warp(draft row v):
 * the children c of v, in index order, are tested with u[c-1]:
 *   accept iff ((double)u * (double)Q_x) * (double)Zc < (double)C_x * (double)Zq;
 *   on rejection C_j <- trunc(ldexp(max(0, C_j*Zq - Q_j*Zc), 62 - bitlen(Zc) -
 *   bitlen(Zq))) and Zc <- sum C (left unchanged when that sum is 0).
 * An accepted child becomes v; when no child is accepted (or v is a leaf) the
 * last token is drawn from C with u[n-1].  On a chain (parent[i] = i-1) this
 * is ora_accept's rule with the same uniforms.  Greedy: move to the first
 * child whose token is argmax(target row v), else emit that argmax.
 * Outputs: tokens [n] = the accepted children's tokens then the drawn one (-1
 * padded), path [n] = 0 then the accepted nodes (-1 padded), n_accepted.
 */
typedef struct {
    const ora_sampling* s;
    int64_t n, V;
    const int32_t* parent;
    const float *tl, *dl, *u;
    const int32_t* tok;
    int32_t *out, *path, *nacc;
} tree_job;

static void tree_one(const tree_job* j, int64_t b, uint64_t* C, uint64_t* Q)
{
    const int64_t n = j->n, V = j->V;
    const float* tl = j->tl + (size_t)b * (size_t)n * (size_t)V;
    const float* dl = j->dl ? j->dl + (size_t)b * (size_t)n * (size_t)V : NULL;
    const int32_t* tok = j->tok + b * n;
    const float* u = j->u ? j->u + b * n : NULL;
    int32_t* out = j->out + b * n;
    int32_t* path = j->path + b * n;
    for (int64_t i = 0; i < n; ++i) out[i] = path[i] = -1;
    path[0] = 0;
    int64_t v = 0, depth = 0;
    for (;;) {
        int64_t next = -1;
        if (j->s->greedy) {
            const int32_t a = (int32_t)argmax_row(tl + v * V, V);
            for (int64_t c = v + 1; c < n && next < 0; ++c)
                if (j->parent[c] == v && tok[c] == a) next = c;
            out[depth] = a;
            if (next < 0) break;
        } else {
            uint64_t Zc, Zq = 0;
            int have_q = 0;
            ora_warp_row(j->s, tl + v * V, V, C, &Zc);
            for (int64_t c = v + 1; c < n; ++c) {
                if (j->parent[c] != v) continue;
                if (!have_q) {
                    ora_warp_row(j->s, dl + v * V, V, Q, &Zq);
                    have_q = 1;
                }
                const int32_t x = tok[c];
                const uint64_t Cx = (x >= 0 && x < V) ? C[x] : 0;
                const uint64_t Qx = (x >= 0 && x < V) ? Q[x] : 0;
                const double lhs = ((double)u[c - 1] * (double)Qx) * (double)Zc;
                const double rhs = (double)Cx * (double)Zq;
                if (lhs < rhs) {
                    out[depth] = x;
                    next = c;
                    break;
                }
                const int sh = 62 - bitlen64(Zc) - bitlen64(Zq);
                uint64_t SR = 0;
                for (int64_t t = 0; t < V; ++t) {
                    const double r = (double)C[t] * (double)Zq - (double)Q[t] * (double)Zc;
                    SR += r > 0.0 ? (uint64_t)ldexp(r, sh) : 0;
                }
                if (SR) {
                    for (int64_t t = 0; t < V; ++t) {
                        const double r = (double)C[t] * (double)Zq - (double)Q[t] * (double)Zc;
                        C[t] = r > 0.0 ? (uint64_t)ldexp(r, sh) : 0;
                    }
                    Zc = SR;
                }
            }
            if (next < 0) {
                out[depth] = (int32_t)ora_cdf_pick(C, V, Zc, u[n - 1]);
                break;
            }
        }
        ++depth;
        path[depth] = (int32_t)next;
        v = next;
    }
    j->nacc[b] = (int32_t)depth;
}

static void tree_range(void* arg, int64_t lo, int64_t hi)
{
    tree_job* j = (tree_job*)arg;
    uint64_t* buf = (uint64_t*)malloc(sizeof(uint64_t) * 2u * (size_t)j->V);
    for (int64_t b = lo; b < hi; ++b) tree_one(j, b, buf, buf + j->V);
    free(buf);
}

int ora_accept_tree(const ora_sampling* s, int64_t B, int64_t n, int64_t V, const int32_t* parent,
                    const float* target_logits, const float* draft_logits, const int32_t* tokens,
                    const float* uniforms, int32_t* out_tokens, int32_t* out_path, int32_t* out_n_accepted,
                    int nthreads)
{
    if (B <= 0 || n <= 0 || V <= 0 || !s || !parent || !target_logits || !tokens || !out_tokens || !out_path ||
        !out_n_accepted)
        return -1;
    if (parent[0] != -1) return -1;
    for (int64_t i = 1; i < n; ++i)
        if (parent[i] < 0 || parent[i] >= i) return -1;
    if (!s->greedy && (!uniforms || !draft_logits || !(s->temperature > 0.0f))) return -1;
    tree_job j = { s, n, V, parent, target_logits, draft_logits, uniforms, tokens, out_tokens, out_path,
                   out_n_accepted };
    ora_parallel_for(nthreads, B, tree_range, &j);
    return 0;
}
