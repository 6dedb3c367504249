/*
 * oracle.h -- CPU restatement of the speculative-decoding verification path.
 *
 * TEST INFRASTRUCTURE ONLY: the outputs the HIP path is tested against.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.  The
 * product (universal-loader_amd/) never links, imports or falls back to it.
 *
 * What it restates and where each part comes from:
 *   - GGUF Q4_0 / Q4_K block formats: type ids and block sizes of
 *     src/core/gguf_types.h:6-33,60-81 with the GGUF byte sizes (18 / 144 B);
 *     Q4_K byte offsets as read by src/inference/inference_engine.cpp:900-921.
 *   - F16 / Q8_0 / Q6_K rows (the types Q4_K_M files mix in): ggml's
 *     published block layouts (ggml is absent here; parity of the Q8_0 / Q6_K
 *     element order against ggml is unpinned, see ora_q4.c).
 *   - fp16 decode: src/inference/inference_engine.cpp:15-37 (half_to_float).
 *   - Weight orientation Y[m][n] = sum_k X[m][k] * W[n][k]:
 *     src/shaders/gemm/gemm_transposed_b_v2.glsl:23-29 with
 *     src/inference/inference_engine.cpp:550-566 (ne[0] = K contiguous).
 *   - Causal visibility (key j visible to query i iff j <= i, scale after the
 *     dot, online softmax): src/shaders/attention/flash_attention_v2_fused.glsl:153-166.
 *   - Inverse-CDF sampling (first i with u < cumsum, fall back to the last
 *     index): src/inference/inference_engine.cpp:340-367.
 *   - Temperature on max-subtracted logits: src/api/gguf_loader.cpp:98-100.
 *   - Softmax / SiLU: src/cpu_backend/activation_cpu.cpp:14-37.
 *   - RMSNorm: src/shaders/ffn/ffn_fused.glsl:23-33; RoPE (interleaved pairs,
 *     base 10000): src/shaders/rope.glsl:50-73; Llama block order:
 *     src/inference/inference_engine.cpp:602-682.
 *   - Speculative acceptance (p/q test, residual max(0, p-q), bonus token):
 *     Leviathan, Kalman & Matias, "Fast Inference from Transformers via
 *     Speculative Decoding", ICML 2023, Algorithm 1; Chen et al. 2023.  The
 *     reference's src/inference/speculative_decoder.cpp:89-110 only matches
 *     token ids and is deliberately not followed.
 *   - Tree acceptance (sibling drafts tested in turn against the running
 *     residual): Miao et al., "SpecInfer", ASPLOS 2024, Algorithm 2.  The
 *     reference's TreeSpeculation (src/inference/speculative_decoder.h:62-87,
 *     .cpp:118-176) builds no real tree and is not followed.
 *
 * Each function's test pin is listed in tests/ (closed forms, brute force,
 * numpy float64, the compiled reference functions under oracle/_ref).
 */
#ifndef ULSPEC_ORACLE_H
#define ULSPEC_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORA_F16 = 1, ORA_Q4_0 = 2, ORA_Q8_0 = 8, ORA_Q4_K = 12, ORA_Q6_K = 14 };

/* ---- fp16 ---------------------------------------------------------------- */
float    ora_h2f(uint16_t h);
uint16_t ora_f2h(float f); /* round to nearest even, overflow -> inf */
void     ora_h2f_array(const uint16_t* h, float* f, size_t n);
void     ora_f2h_array(const float* f, uint16_t* h, size_t n);

/* ---- deterministic random numbers ---------------------------------------- */
uint64_t ora_mix64(uint64_t x);
/* u = top 24 bits of mix64(seed + (idx+1)*golden) * 2^-24, in [0, 1) */
float ora_uniform(uint64_t seed, uint64_t idx);
void  ora_uniforms(uint64_t seed, uint64_t idx0, size_t n, float* out);
/* Box-Muller in double from the counter stream (seed, stream); fp32 output. */
void  ora_normals(uint64_t seed, uint64_t stream, size_t n, double mean, double std, float* out, int nthreads);

/* ---- deterministic exp shared (by algorithm) with the device ------------- */
float ora_expf(float x);

/* ---- GGUF Q4 formats ------------------------------------------------------ */
int    ora_blck_size(int type);          /* 32 / 256, 0 if unsupported */
int    ora_type_size(int type);          /* 18 / 144, 0 if unsupported */
size_t ora_row_bytes(int type, int64_t k);
int    ora_quantize(int type, const float* x, int64_t n, uint8_t* out);   /* n % blck == 0 */
int    ora_dequantize(int type, const uint8_t* in, int64_t n, float* out);
/* normals -> quantized rows, same stream layout as ora_normals(seed, stream) */
int    ora_synth_q4(int type, uint64_t seed, uint64_t stream, int64_t N, int64_t K, double std,
                    uint8_t* out, int nthreads);

/* ---- verify dequant-GEMM --------------------------------------------------- */
/* Y[M][N] (fp32) = X[M][K] (fp16) . W[N][K]^T, W in GGUF blocks.
 * f64: float64 accumulation of the exact products (the pinning reference).
 * f32: AVX2 + threads, per-block fp32 partials scaled in fp32 (the CPU baseline). */
int ora_q4_gemm_f64(int type, const uint8_t* W, int64_t N, int64_t K,
                    const uint16_t* X, int64_t M, double* Y);
int ora_q4_gemm_f32(int type, const uint8_t* W, int64_t N, int64_t K,
                    const uint16_t* X, int64_t M, float* Y, int nthreads);
/* The same with fp32 X (the model's activations). */
int ora_q4_gemm_x32(int type, const uint8_t* W, int64_t N, int64_t K,
                    const float* X, int64_t M, float* Y, int nthreads);

/* ---- verify attention ------------------------------------------------------ */
/* q: fp16 [nq][H][D]; k, v: fp16 [L][Hkv][D] with L = n_prefix + nq (the nq new
 * rows already appended); parent: NULL = causal chain, else int32 [nq] with
 * parent[i] < i or -1 (attach to the prefix); out fp32 [nq][H][D].  Softmax in
 * float64 (the pinning reference). */
int ora_attention_f64(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                      int64_t n_prefix, int64_t nq, const int32_t* parent,
                      int64_t H, int64_t Hkv, int64_t D, float scale, double* out);
/* Same semantics, fp32 online softmax with threads (the CPU baseline). */
int ora_attention_f32(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                      int64_t n_prefix, int64_t nq, const int32_t* parent,
                      int64_t H, int64_t Hkv, int64_t D, float scale, float* out, int nthreads);

/* ---- acceptance sampling --------------------------------------------------- */
typedef struct {
    float    temperature; /* > 0 */
    uint32_t top_k;       /* 0 = off */
    float    top_p;       /* >= 1 = off */
    int32_t  greedy;      /* != 0: argmax rule, uniforms and draft logits unused */
} ora_sampling;

/* Warped distribution of one logit row in exact fixed point.
 * E[i] = trunc(expf((l[i]-lmax)*invT) * 2^S) for kept i, 0 otherwise, with
 * S = ora_warp_shift(V) = 63 - bitlen(V); Z = sum E < 2^63.
 * Returns the number of kept tokens. */
int     ora_warp_shift(int64_t V);
int64_t ora_warp_row(const ora_sampling* s, const float* logits, int64_t V, uint64_t* E, uint64_t* Z);
/* Inverse-CDF draw over weights W[V] (index order), total Z, uniform u. */
int64_t ora_cdf_pick(const uint64_t* W, int64_t V, uint64_t Z, float u);
/* Sample one token per row from the warped distribution (greedy: argmax). */
int ora_sample(const ora_sampling* s, int64_t R, int64_t V, const float* logits,
               const float* uniforms, int32_t* out_tokens);
/* One verification per sequence.  target [B][k+1][V], draft [B][k][V],
 * draft_tokens [B][k], uniforms [B][k+1]; out_tokens [B][k+1] (-1 padded),
 * out_n_accepted [B]. */
int ora_accept(const ora_sampling* s, int64_t B, int64_t k, int64_t V,
               const float* target_logits, const float* draft_logits,
               const int32_t* draft_tokens, const float* uniforms,
               int32_t* out_tokens, int32_t* out_n_accepted, int nthreads);
/* One tree verification per sequence (rule in ora_accept.c): parent [n]
 * (parent[0] = -1, parent[i] in [0, i)), shared by the B trees; target and
 * draft [B][n][V] (row v: after node v / the children's draft distribution),
 * tokens [B][n], uniforms [B][n]; out_tokens [B][n] and out_path [B][n]
 * (-1 padded), out_n_accepted [B]. */
int ora_accept_tree(const ora_sampling* s, int64_t B, int64_t n, int64_t V, const int32_t* parent,
                    const float* target_logits, const float* draft_logits, const int32_t* tokens,
                    const float* uniforms, int32_t* out_tokens, int32_t* out_path, int32_t* out_n_accepted,
                    int nthreads);

/* ---- Llama-shaped model and the speculative loop ---------------------------
 * Block order of InferenceEngine::forward_layer_gpu
 * (src/inference/inference_engine.cpp:602-682): RMSNorm -> Q, K, V -> RoPE ->
 * attention -> O -> +residual -> RMSNorm -> gate, up -> SiLU(gate)*up -> down
 * -> +residual; final RMSNorm, LM head.  Activations are fp32 (the residual
 * stream and every GEMM input: normed activations, attention output, SiLU
 * product); only Q and the K/V cache are rounded to fp16 (round to nearest
 * even), the attention kernel's inputs.
 *   RMSNorm  x = (h * r) * w, r = 1 / sqrtf(sum(h^2) / dim + eps)
 *            (src/shaders/ffn/ffn_fused.glsl:23-33)
 *   RoPE     pairs (2i, 2i+1): y0 = x0 c - x1 s, y1 = x0 s + x1 c with
 *            (c, s) = fp32(cos, sin)(pos * base^(-2i/D)) evaluated in double
 *            (src/shaders/rope.glsl:50-73)
 *   SiLU     g * (1 / (1 + ora_expf(-g))) (src/cpu_backend/activation_cpu.cpp:14-20)
 *   attention ora_attention_f32, scale 1/sqrt(D), causal over the cache. */
typedef struct {
    int64_t dim, n_layers, n_heads, n_kv_heads, ffn, vocab, max_ctx;
    float rms_eps, rope_base;
} ora_llama_cfg;

typedef struct ora_llama ora_llama;
ora_llama* ora_llama_create(const ora_llama_cfg* cfg, int nthreads);
void       ora_llama_free(ora_llama* m);
/* Worker threads of the forward's GEMMs and attention (the results do not
 * depend on it). */
void       ora_llama_set_threads(ora_llama* m, int nthreads);
/* GGUF tensor by name (token_embd / output_norm / output / blk.<i>.{attn_norm,
 * attn_q, attn_k, attn_v, attn_output, ffn_norm, ffn_gate, ffn_up, ffn_down}
 * .weight); norms F32 (type 0), the rest Q4_0 / Q4_K; bytes are copied. */
int        ora_llama_set_tensor(ora_llama* m, const char* name, int type, const void* data, size_t nbytes,
                                int64_t ne0, int64_t ne1);
/* Forward M tokens at positions pos .. pos+M-1 (K/V appended); logits of the
 * last n_logits rows to logits [n_logits][vocab] (NULL when n_logits = 0). */
int        ora_llama_forward(ora_llama* m, const int32_t* tokens, int64_t M, int64_t pos, float* logits,
                             int64_t n_logits);
/* K/V rows pos0 .. pos0+n-1 of one layer out of (dir 0) / into (dir 1) the
 * model, fp16 bits [n][n_kv_heads * head_dim]. */
int        ora_llama_kv_io(ora_llama* m, int64_t layer, int dir, int64_t pos0, int64_t n, uint16_t* k, uint16_t* v);

/* Speculative decoding (one sequence).  seq holds the committed tokens
 * (capacity cap); st->n of them.  One step, as the device loop:
 *   u_j = ora_uniform(seed, step*(2k+1) + j), j = 0 .. 2k
 *   draft forward [seq[n-2], seq[n-1]] at n-2 -> d_1 = sample(row n-1, u_0);
 *   draft forward [d_j] at n-1+j -> d_{j+1} = sample(.., u_j), j = 1 .. k-1
 *   target forward [seq[n-1], d_1 .. d_k] at n-1 .. n-1+k
 *   ora_accept(.., uniforms u_k .. u_2k) -> n_acc + 1 tokens appended.
 * A plain step (k = 0, draft NULL: decoding of the target alone; or n = 1,
 * before the draft has the two tokens of its catch-up pair): target forward
 * [seq[n-1]] at n-1 -> seq[n] = sample(.., u_0); proposed unchanged. */
typedef struct {
    int64_t n, step, accepted, proposed;
} ora_spec_state;
/* Both models process prompt[0 .. n-2] (n >= 1); seq = prompt; counters zero. */
int     ora_spec_prefill(ora_llama* target, ora_llama* draft, const int32_t* prompt, int64_t n, int32_t* seq,
                         int64_t cap, ora_spec_state* st);
int     ora_spec_step(ora_llama* target, ora_llama* draft, const ora_sampling* s, int64_t k, uint64_t seed,
                      int32_t* seq, int64_t cap, ora_spec_state* st);
/* Steps until at least n_new tokens were committed by this call; returns the
 * number committed (< 0 on error). */
int64_t ora_spec_generate(ora_llama* target, ora_llama* draft, const ora_sampling* s, int64_t k, uint64_t seed,
                          int64_t n_new, int32_t* seq, int64_t cap, ora_spec_state* st);

#ifdef __cplusplus
}
#endif
#endif
