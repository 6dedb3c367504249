/*
 * ora_attn.c -- draft-verify attention on the CPU (test infrastructure, see
 * oracle.h).
 *
 * Query i (0 <= i < nq) sits at position n_prefix + i (causal) and sees every
 * prefix key j < n_prefix.  Among the nq new keys (rows n_prefix + a):
 *   causal (parent == NULL): a <= i, i.e. key position <= query position, the
 *     rule of src/shaders/attention/flash_attention_v2_fused.glsl:153-154;
 *   tree: a == i or a is an ancestor of i through parent[] (parent[a] < a, -1
 *     attaches a node to the prefix).
 * Score = scale * (q . k) (scale applied after the dot,
 * flash_attention_v2_fused.glsl:160); softmax over visible keys; output
 * sum_j p_j v_j.  Head h reads KV head h / (H / Hkv).
 */
#include "ora_internal.h"

#include <math.h>
#include <string.h>

static int visible(const int32_t* parent, int64_t i, int64_t a)
{
    if (!parent) return a <= i;
    if (a == i) return 1;
    int64_t p = parent[i];
    while (p >= 0) {
        if (p == a) return 1;
        p = parent[p];
    }
    return 0;
}

static int check_args(int64_t n_prefix, int64_t nq, const int32_t* parent, int64_t H, int64_t Hkv, int64_t D)
{
    if (n_prefix < 0 || nq <= 0 || H <= 0 || Hkv <= 0 || D <= 0 || H % Hkv) return -1;
    if (parent)
        for (int64_t i = 0; i < nq; ++i)
            if (parent[i] >= i || parent[i] < -1) return -1;
    return 0;
}

int ora_attention_f64(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                      int64_t n_prefix, int64_t nq, const int32_t* parent,
                      int64_t H, int64_t Hkv, int64_t D, float scale, double* out)
{
    if (check_args(n_prefix, nq, parent, H, Hkv, D)) return -1;
    const int64_t L = n_prefix + nq, G = H / Hkv;
    double* s = (double*)malloc(sizeof(double) * (size_t)L);
    double* qd = (double*)malloc(sizeof(double) * (size_t)D);
    for (int64_t h = 0; h < H; ++h) {
        const int64_t hk = h / G;
        for (int64_t i = 0; i < nq; ++i) {
            for (int64_t d = 0; d < D; ++d) qd[d] = (double)ora_h2f(q[(i * H + h) * D + d]);
            double mx = -INFINITY;
            for (int64_t j = 0; j < L; ++j) {
                if (j >= n_prefix && !visible(parent, i, j - n_prefix)) { s[j] = -INFINITY; continue; }
                const uint16_t* kr = k + (j * Hkv + hk) * D;
                double acc = 0.0;
                for (int64_t d = 0; d < D; ++d) acc += qd[d] * (double)ora_h2f(kr[d]);
                s[j] = (double)scale * acc;
                if (s[j] > mx) mx = s[j];
            }
            double den = 0.0;
            for (int64_t j = 0; j < L; ++j) {
                s[j] = s[j] == -INFINITY ? 0.0 : exp(s[j] - mx);
                den += s[j];
            }
            double* o = out + (i * H + h) * D;
            for (int64_t d = 0; d < D; ++d) o[d] = 0.0;
            for (int64_t j = 0; j < L; ++j) {
                if (s[j] == 0.0) continue;
                const uint16_t* vr = v + (j * Hkv + hk) * D;
                double p = s[j] / den;
                for (int64_t d = 0; d < D; ++d) o[d] += p * (double)ora_h2f(vr[d]);
            }
        }
    }
    free(qd);
    free(s);
    return 0;
}

typedef struct {
    const uint16_t *q, *k, *v;
    int64_t n_prefix, nq, H, Hkv, D;
    const int32_t* parent;
    float scale;
    float* out;
} attn_job;

/* fp32 online softmax, one (head, query) per iteration */
static void attn_range(void* arg, int64_t lo, int64_t hi)
{
    attn_job* j = (attn_job*)arg;
    const int64_t D = j->D, G = j->H / j->Hkv, L = j->n_prefix + j->nq;
    float* qf = (float*)malloc(sizeof(float) * (size_t)D);
    float* acc = (float*)malloc(sizeof(float) * (size_t)D);
    for (int64_t t = lo; t < hi; ++t) {
        int64_t h = t / j->nq, i = t % j->nq, hk = h / G;
        for (int64_t d = 0; d < D; ++d) { qf[d] = ora_h2f(j->q[(i * j->H + h) * D + d]); acc[d] = 0.0f; }
        float m = -INFINITY, l = 0.0f;
        for (int64_t key = 0; key < L; ++key) {
            if (key >= j->n_prefix && !visible(j->parent, i, key - j->n_prefix)) continue;
            const uint16_t* kr = j->k + (key * j->Hkv + hk) * D;
            float sdot = 0.0f;
            for (int64_t d = 0; d < D; ++d) sdot += qf[d] * ora_h2f(kr[d]);
            float sc = sdot * j->scale;
            float mn = sc > m ? sc : m;
            float alpha = expf(m - mn), p = expf(sc - mn);
            l = l * alpha + p;
            const uint16_t* vr = j->v + (key * j->Hkv + hk) * D;
            for (int64_t d = 0; d < D; ++d) acc[d] = acc[d] * alpha + p * ora_h2f(vr[d]);
            m = mn;
        }
        float* o = j->out + (i * j->H + h) * D;
        for (int64_t d = 0; d < D; ++d) o[d] = acc[d] / l;
    }
    free(acc);
    free(qf);
}

int ora_attention_f32(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                      int64_t n_prefix, int64_t nq, const int32_t* parent,
                      int64_t H, int64_t Hkv, int64_t D, float scale, float* out, int nthreads)
{
    if (check_args(n_prefix, nq, parent, H, Hkv, D)) return -1;
    attn_job j = { q, k, v, n_prefix, nq, H, Hkv, D, parent, scale, out };
    ora_parallel_for(nthreads, H * nq, attn_range, &j);
    return 0;
}
