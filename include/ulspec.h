/*
 * ulspec.h -- C ABI of the MI355X (gfx950) speculative-decoding verification
 * path.  Plain C: opaque context, status codes, device pointers and sizes.
 *
 * The reference exposes this path through the C++ class py::InferenceAPI
 * (src/api/inference_api.h:52-123, pybind module `vulkangguf`,
 * src/api/inference_api.cpp:389-427) over inference::InferenceEngine and
 * inference::SpeculativeDecoder (src/inference/speculative_decoder.h:24-60).
 * Those classes are mirrored in C++ on top of this ABI
 * (universal-loader_amd/csrc/host/); each entry point below names the
 * reference interface whose work it takes over.
 *
 * Conventions
 *   - Every function returns ULSPEC_OK or an error code; no C++ exception
 *     crosses the ABI.  ulspec_last_error() gives the message of the last
 *     failure on a context.
 *   - Arguments are validated on the host before any launch, so invalid
 *     calls fail without touching the GPU.
 *   - A context owns one HIP stream (default priority) on one device; compute
 *     calls are asynchronous on that stream; ulspec_sync / ulspec_memcpy are
 *     the host fences.  A context is not thread-safe (one per host thread, as
 *     py::InferenceAPI serialises every call behind api_mutex_,
 *     src/api/inference_api.h:115).
 *   - Weights, KV caches and workspaces belong to the context; host buffers
 *     belong to the caller.  There is no CPU fallback: without a usable
 *     gfx950 device, ulspec_create fails with ULSPEC_EDEVICE.
 */
#ifndef ULSPEC_H
#define ULSPEC_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ulspec_ctx ulspec_ctx;

typedef enum {
    ULSPEC_OK = 0,
    ULSPEC_EINVAL = 1,       /* bad argument (checked before any launch) */
    ULSPEC_ENOMEM = 2,       /* device or host allocation failed */
    ULSPEC_EDEVICE = 3,      /* HIP runtime error / no gfx950 device */
    ULSPEC_EUNSUPPORTED = 4  /* valid request the library does not implement */
} ulspec_status;

/* GGUF type ids (src/core/gguf_types.h:6-33). */
enum { ULSPEC_GGML_F16 = 1, ULSPEC_GGML_Q4_0 = 2, ULSPEC_GGML_Q8_0 = 8, ULSPEC_GGML_Q4_K = 12, ULSPEC_GGML_Q6_K = 14 };

/* ---- library / context ---------------------------------------------------
 * Replaces the Vulkan bring-up of InferenceEngine::initialize
 * (src/inference/inference_engine.cpp:48-148). */
const char*   ulspec_version(void);
/* Block sizes of the GGUF types: elements per block and bytes per block
 * (Q4_0 32 / 18, Q4_K 256 / 144, Q6_K 256 / 210, Q8_0 32 / 34, F16 1 / 2, ...;
 * 0 for an unknown id).  Replaces ggml_blck_size / ggml_type_size
 * (src/core/gguf_types.h:35-81, whose Q4 byte sizes 6 / 12 are wrong).  The
 * kernels read Q4_0 and Q4_K weights only. */
int           ulspec_ggml_blck_size(uint32_t ggml_type);
int           ulspec_ggml_type_size(uint32_t ggml_type);
ulspec_status ulspec_create(int hip_device, ulspec_ctx** out);
void          ulspec_destroy(ulspec_ctx* ctx);
const char*   ulspec_last_error(const ulspec_ctx* ctx); /* valid until the next call on ctx */
const char*   ulspec_status_str(ulspec_status s);

/* ---- memory (device buffers owned by the caller through the context) ----- */
ulspec_status ulspec_alloc(ulspec_ctx* ctx, size_t bytes, void** dev_ptr);
ulspec_status ulspec_free(ulspec_ctx* ctx, void* dev_ptr);
/* kind: 0 host->device, 1 device->host, 2 device->device; ordered on the
 * context stream and synchronous for the host. */
ulspec_status ulspec_memcpy(ulspec_ctx* ctx, void* dst, const void* src, size_t bytes, int kind);
ulspec_status ulspec_sync(ulspec_ctx* ctx);

/* ---- stream capture and timing ---------------------------------------------
 * Record a sequence of compute calls on the context stream into a HIP graph
 * and replay it; mark HIP events on the stream and read the time between two
 * marks.  This is the launch-free replay of a fixed step (the reference
 * submits one command buffer and waits on a fence per dispatch,
 * src/vulkan_backend/compute.cpp:82-121) and the device-side timing behind
 * InferenceAPI::enable_profiling / get_performance_report
 * (src/api/inference_api.h:93-94).  Calls that allocate (weight uploads,
 * workspace growth) must not run while capturing. */
ulspec_status ulspec_capture_begin(ulspec_ctx* ctx);
ulspec_status ulspec_capture_end(ulspec_ctx* ctx, uint32_t* graph_id);
ulspec_status ulspec_graph_replay(ulspec_ctx* ctx, uint32_t graph_id, uint32_t times);
ulspec_status ulspec_graph_destroy(ulspec_ctx* ctx, uint32_t graph_id);
ulspec_status ulspec_timer_mark(ulspec_ctx* ctx, uint32_t slot /* < 16 */);
ulspec_status ulspec_timer_elapsed_ms(ulspec_ctx* ctx, uint32_t slot_a, uint32_t slot_b, float* ms);
/* Measurement kernel with no counterpart in the reference: reads every 16-byte
 * unit of the device buffer `buf` (bytes a multiple of 16) once, 256 threads
 * per workgroup and 4 << (variant & 3) loads per thread, all issued before the
 * first use; variants 4..7 load with the non-temporal cache policy (no
 * last-level cache allocation, as the verify GEMMs load their weights).  *sink (device) is written only by a thread whose loaded
 * words XOR to 0x5eed5eed, so the loads cannot be elided.  Its duration for a
 * given size is the streaming-read ceiling the verify kernels are compared
 * with. */
ulspec_status ulspec_stream_read(ulspec_ctx* ctx, const void* buf, size_t bytes, uint32_t variant, uint32_t* sink);
/* The context's HIP device and its compute-unit count. */
ulspec_status ulspec_device_info(ulspec_ctx* ctx, int* device, int* n_cu);
/* Kernel-route override, no counterpart in the reference (for tests that must
 * reach each route whatever the device's CU count).  ULSPEC_OPT_TOPK_ROUTE:
 * how the top-k (kept list, top_k <= 256) statistics run -- 0 chosen from the
 * rows and CUs (default), 1 one 1024-thread workgroup per row, 2 one
 * 512-thread workgroup per row, 3 the scanned chunk pipeline (scan,
 * threshold, collect, finish), 4 the sampled chunk pipeline (a threshold from
 * a sample of each row, collect, finish: the default past the one-workgroup
 * routes, for top_k <= 128); a route that cannot take the call (rows past
 * 32768 logits, or k past its kept maxima) falls back to a chunk pipeline.
 * Every route gives the same tokens. */
enum { ULSPEC_OPT_TOPK_ROUTE = 1 };
/* Measurement kernel with no counterpart in the reference: the cost of one
 * grid-wide barrier between co-resident workgroups (a persistent kernel's
 * alternative to a kernel boundary).  `workgroups` x `threads` (256, 512 or
 * 1024) run `rounds` rounds of: write 256 floats, barrier (a flag per
 * workgroup, all polled), read another workgroup's floats.  mode 0: agent-scope
 * release / acquire around the flags (L2 write-back and invalidate); mode 1:
 * data and flags through agent-scope relaxed accesses, no write-back.  Gives
 * the microseconds per round and the number of stale reads.  Allocates, and
 * synchronises the context stream; EDEVICE if a wait passed its bound. */
ulspec_status ulspec_sync_probe(ulspec_ctx* ctx, uint32_t mode, uint32_t workgroups, uint32_t threads,
                                uint32_t rounds, float* us_per_round, uint32_t* errors);
ulspec_status ulspec_set_option(ulspec_ctx* ctx, uint32_t option, int64_t value);

/* ---- K1: verify dequant-GEMM ------------------------------------------------
 * Upload one linear weight given as GGUF blocks (host memory, rows of K
 * elements, ne[0] = K contiguous; src/core/tensor.h:17-65).  The context keeps
 * a device copy re-tiled for the kernel: Q4_0 / Q4_K / Q6_K / Q8_0 in their
 * own 18 / 144 / 210 / 34 bytes per block (Q6_K: (q - 32) * scale formed in
 * fp16 in the kernel, rounded only where its magnitude exceeds 2048); F16 as
 * is.  K is a multiple of the block size, and of 32 for F16.  weight_info
 * reports the uploaded type.
 * Replaces the first-use repack + upload of run_linear_q4k
 * (src/inference/inference_engine.cpp:536-548, repack_q4k_tensor :891-927). */
ulspec_status ulspec_weight_upload(ulspec_ctx* ctx, uint32_t ggml_type, const void* gguf_blocks,
                                   size_t nbytes, uint32_t n_rows /* N */, uint32_t k /* K */,
                                   uint32_t* out_weight_id);
ulspec_status ulspec_weight_info(ulspec_ctx* ctx, uint32_t weight_id, uint32_t* ggml_type,
                                 uint32_t* n_rows, uint32_t* k, size_t* device_bytes);
/* Y[M][N] (fp32, row-major) = X[M][K] (fp16, row-major) . W[N][K]^T.
 * M >= 1 (any size; rows are processed in groups of up to 64).
 * Replaces the dequantize + gemm_transposed_b_v2 pair of run_linear_q4k
 * (src/inference/inference_engine.cpp:550-566). */
ulspec_status ulspec_verify_gemm(ulspec_ctx* ctx, uint32_t weight_id, const uint16_t* x_f16,
                                 uint32_t M, float* y_f32);

/* ---- K2: verify attention ---------------------------------------------------
 * q: fp16 [nq][H][D]; k_cache, v_cache: fp16 [L][Hkv][D] with L = n_prefix + nq
 * (the nq new rows already written); out: fp32 [nq][H][D] (device memory).
 * parent: NULL for a causal chain, else HOST int32 [nq] with parent[i] < i or
 * -1 (child of the prefix).  1 <= nq <= 16, D == 128 or 64, H % Hkv == 0.
 * Replaces the single-token attention dispatch of forward_layer_gpu
 * (src/inference/inference_engine.cpp:627-630; semantics of
 * src/shaders/attention/flash_attention_v2_fused.glsl:153-166). */
ulspec_status ulspec_verify_attention(ulspec_ctx* ctx, const uint16_t* q, const uint16_t* k_cache,
                                      const uint16_t* v_cache, uint32_t n_prefix, uint32_t nq,
                                      const int32_t* parent, uint32_t H, uint32_t Hkv, uint32_t D,
                                      float scale, float* out);

/* ---- K3: acceptance sampling ------------------------------------------------ */
typedef struct {
    float    temperature; /* > 0 (ignored when greedy) */
    uint32_t top_k;       /* 0 = off */
    float    top_p;       /* >= 1 = off */
    int32_t  greedy;      /* != 0: argmax-match rule */
} ulspec_sampling;

/* Per sequence b: p_i = warp(target[b][i]), q_i = warp(draft[b][i]); accept
 * draft token x_i while u[b][i] * q_i(x_i) < p_i(x_i); on the first rejection
 * draw from max(0, p_i - q_i) (renormalised) with u[b][k]; if all k pass, draw
 * the bonus token from p_k with u[b][k].  Greedy: accept while argmax p_i ==
 * x_i and emit the argmax.  out_tokens [B][k+1] holds n_accepted + 1 tokens
 * then -1.  All arrays are device memory.  1 <= k <= 16, any top_k (the
 * kept list path up to 256, a per-row bound over the whole vocabulary
 * beyond), B (2k+1) <= 65535 logit rows per call.
 * Replaces SpeculativeDecoder::verify_speculation and the sampling of
 * InferenceEngine::sample_token (src/inference/speculative_decoder.cpp:89-110,
 * src/inference/inference_engine.cpp:340-367). */
ulspec_status ulspec_accept(ulspec_ctx* ctx, const ulspec_sampling* s, uint32_t B, uint32_t k,
                            uint32_t V, const float* target_logits, const float* draft_logits,
                            const int32_t* draft_tokens, const float* uniforms,
                            int32_t* out_tokens, int32_t* out_n_accepted);
/* ulspec_accept that allocates nothing: no counterpart in the reference; for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops, harnesses that forbid hipMalloc).  Same arguments, rule and
 * results as ulspec_accept; its kernels keep their intermediate sums in a
 * static device scratch array of ULSPEC_ACCEPT_NOALLOC_SCRATCH bytes per GPU
 * (held until the process ends) instead of the context workspace.  Calls
 * whose scratch would exceed it (B (2k+1) logit rows; e.g. B = 16, k = 8 with
 * top-k fits) fail with ULSPEC_EUNSUPPORTED before any launch.  Every call on
 * one GPU shares the array: calls that overlap on one GPU (other streams or
 * contexts) race. */
#define ULSPEC_ACCEPT_NOALLOC_SCRATCH (32u << 20)
ulspec_status ulspec_accept_noalloc(ulspec_ctx* ctx, const ulspec_sampling* s, uint32_t B, uint32_t k,
                                    uint32_t V, const float* target_logits, const float* draft_logits,
                                    const int32_t* draft_tokens, const float* uniforms,
                                    int32_t* out_tokens, int32_t* out_n_accepted);
/* Tree verification, B trees of one shape: nodes 0 .. n-1 (n <= 16), node 0
 * the root (the last committed token), parent (HOST int32 [n]) with
 * parent[0] = -1 and parent[i] in [0, i).  target_logits [B][n][V]: row v is
 * the target's distribution after node v; draft_logits [B][n][V]: row v is the
 * distribution node v's children were drawn from (rows of leaves are not
 * read); tokens [B][n] (node 0's unused); uniforms [B][n].  From the root,
 * the children c of the current node are tested in index order with
 * u[c-1] against the running residual (multi-draft speculative sampling,
 * SpecInfer, Miao et al. 2024, Alg. 2): accept iff u q(x) < C(x), else C <-
 * norm(max(0, C - q)); an accepted child becomes the current node; otherwise
 * the last token is drawn from C with u[n-1].  Greedy: follow the first child
 * holding the argmax, else emit it.  On a chain (parent[i] = i-1) this is
 * ulspec_accept.  out_tokens [B][n]: n_accepted + 1 tokens then -1;
 * out_path [B][n]: node 0 then the accepted nodes, then -1 (the rows
 * ulspec_model_kv_compact keeps).  Device memory but parent.  Replaces
 * TreeSpeculation (src/inference/speculative_decoder.h:62-87, .cpp:118-176),
 * which builds no real tree. */
ulspec_status ulspec_accept_tree(ulspec_ctx* ctx, const ulspec_sampling* s, uint32_t B, uint32_t n, uint32_t V,
                                 const int32_t* parent, const float* target_logits, const float* draft_logits,
                                 const int32_t* tokens, const float* uniforms, int32_t* out_tokens,
                                 int32_t* out_path, int32_t* out_n_accepted);
/* One token per row from warp(logits[r]) with uniforms[r] (greedy: argmax);
 * R <= 65535 rows per call.
 * Replaces InferenceEngine::sample_token (src/inference/inference_engine.cpp:340-367). */
ulspec_status ulspec_sample(ulspec_ctx* ctx, const ulspec_sampling* s, uint32_t R, uint32_t V,
                            const float* logits, const float* uniforms, int32_t* out_tokens);
/* uniforms[i] = top 24 bits of splitmix64(seed + (idx0 + i + 1) * golden) * 2^-24 */
ulspec_status ulspec_uniforms(ulspec_ctx* ctx, uint64_t seed, uint64_t idx0, uint32_t n, float* out);

/* ---- synthetic GGUF weights ---------------------------------------------
 * Writes N rows of K elements as raw GGUF blocks (Q4_0 / Q4_K) into device
 * memory `out` (N * K / blck * type_size bytes): element (n, k) is normal
 * number n*K + k of the counter-based stream (seed, stream) -- Box-Muller in
 * double on splitmix64 counters, then the GGUF quantizer.  For synthetic
 * random-init models (no checkpoint is loaded). */
ulspec_status ulspec_synth_q4(ulspec_ctx* ctx, uint32_t ggml_type, uint64_t seed, uint64_t stream, uint32_t N,
                              uint32_t K, float std_dev, void* out);

/* ---- Llama-shaped model (target or draft) ---------------------------------
 * Device weights, fp16 KV cache [max_ctx][n_kv_heads][head_dim] per layer and
 * activation buffers for up to 16 rows.  Block order of
 * InferenceEngine::forward_layer_gpu (src/inference/inference_engine.cpp:602-682):
 * RMSNorm -> QKV -> RoPE -> attention -> O -> +residual -> RMSNorm -> gate/up
 * -> SiLU(gate) * up -> down -> +residual; final RMSNorm and LM head.
 * Activations, the residual stream and logits are fp32 (GEMM inputs reach the
 * fp16 MFMAs as split (hi, lo) pairs); Q and the K/V cache are fp16.  Replaces Model /
 * KVCache (src/inference/model.h:49-115) and forward_layer_gpu (:475-692). */
typedef struct ulspec_model ulspec_model;
typedef struct {
    uint32_t dim, n_layers, n_heads, n_kv_heads, ffn, vocab;
    uint32_t max_ctx;    /* KV-cache positions */
    float    rms_eps;    /* RMSNorm epsilon */
    float    rope_base;  /* RoPE theta base (10000 in src/shaders/rope.glsl) */
} ulspec_model_cfg;
ulspec_status ulspec_model_create(ulspec_ctx* ctx, const ulspec_model_cfg* cfg, ulspec_model** out);
/* A model with n_seq <= 8 sequence slots, each with its own K/V cache of
 * max_ctx positions (one set of weights): the batch of the reference's
 * generate_batch (src/api/inference_api.h:63) for the device loop of
 * ulspec_spec_create_batch.  ulspec_model_create is n_seq = 1; the other
 * model entry points work on slot 0. */
ulspec_status ulspec_model_create_batch(ulspec_ctx* ctx, const ulspec_model_cfg* cfg, uint32_t n_seq,
                                        ulspec_model** out);
void          ulspec_model_destroy(ulspec_model* m);
/* One GGUF tensor by its GGUF name (token_embd.weight, output_norm.weight,
 * output.weight, blk.<i>.{attn_norm,attn_q,attn_k,attn_v,attn_output,ffn_norm,
 * ffn_gate,ffn_up,ffn_down}.weight), as the weight map of Model::load_from_gguf
 * (src/inference/model.cpp:190-246).  Norms are F32 (type 0), matrices and the
 * embedding Q4_0, Q4_K, Q6_K, Q8_0 or F16.  The parts of a fused weight (Q | K
 * | V, gate | up) of one type are fused as they are; parts of mixed types are
 * fused as fp16 rows.  ne0 = elements per row (contiguous), ne1 = rows.
 * `data` is host memory, or device memory when on_device != 0. */
ulspec_status ulspec_model_set_tensor(ulspec_model* m, const char* name, uint32_t ggml_type, const void* data,
                                      size_t nbytes, uint64_t ne0, uint64_t ne1, int on_device);
/* Forward M tokens (host ids) at positions pos .. pos+M-1, appending their K/V;
 * copies the logits of the last n_logits (<= 16) rows to host memory `logits`
 * (n_logits = 0: none).  Synchronous.  Serves InferenceAPI::get_token_logits
 * (src/api/inference_api.cpp:277-280) and prefill. */
ulspec_status ulspec_model_forward(ulspec_model* m, const int32_t* tokens, uint32_t M, uint32_t pos,
                                   float* logits, uint32_t n_logits);
/* ulspec_model_forward on sequence slot seq (its own K/V cache). */
ulspec_status ulspec_model_forward_seq(ulspec_model* m, uint32_t seq, const int32_t* tokens, uint32_t M,
                                       uint32_t pos, float* logits, uint32_t n_logits);
/* Forward a draft tree of M nodes (host ids; M <= 16 and at most the model's
 * row limit) whose K/V go to slots pos .. pos+M-1: node i (parent[i] in [-1,
 * i), host array; -1 = child of the prefix) takes RoPE position pos +
 * depth(i) and attends to positions 0 .. pos-1, its ancestors and itself
 * (the mask of ulspec_verify_attention).  Logits of all M nodes to host
 * memory logits [M][vocab].  Synchronous.  Each node's outputs equal those of
 * a causal forward of its root-to-node path at positions pos, pos+1, .. */
ulspec_status ulspec_model_forward_tree(ulspec_model* m, const int32_t* tokens, const int32_t* parent, uint32_t M,
                                        uint32_t pos, float* logits);
/* One linear layer of the model, alone, as a forward runs it: which = 0
 * Q|K|V (RMSNorm prologue; RoPE, fp16 Q and the K/V append at positions pos
 * .. pos + M - 1 of sequence slot 0), 1 O (residual epilogue and the next
 * norm's input), 2 gate|up (RMSNorm prologue, SiLU * up epilogue), 3 down
 * (residual epilogue), 4 the LM head (final RMSNorm, logits to the model's
 * own buffer; layer ignored), over the M <= 16 rows the model's activation
 * buffers hold from its last forward.  The verify GEMM of one linear of
 * InferenceEngine::forward_layer_gpu (src/inference/inference_engine.cpp:
 * 602-682) with its neighbours fused; for timing the GEMMs in the
 * configuration a speculative step runs them.  Asynchronous. */
ulspec_status ulspec_model_linear(ulspec_model* m, uint32_t layer, uint32_t which, uint32_t M, uint32_t pos);
/* Commit an accepted tree path: K/V rows pos + path[j] -> pos + j for j = 1
 * .. min(*n_accepted + 1, n_max) - 1 in every layer (row pos, the root,
 * stays).  path and n_accepted are DEVICE memory, as written by
 * ulspec_accept_tree for one tree (path strictly increasing from 0);
 * entries outside [0, n_max) are skipped.  Asynchronous on the context
 * stream.  The rows past the kept ones are stale and are overwritten by the
 * next forward. */
ulspec_status ulspec_model_kv_compact(ulspec_model* m, uint32_t pos, const int32_t* path, const int32_t* n_accepted,
                                      uint32_t n_max);
/* Copy K/V cache rows pos0 .. pos0+n-1 of one layer to (dir 0) or from (dir 1)
 * host arrays [n][n_kv_heads][head_dim] of fp16 bits.  Synchronous. */
ulspec_status ulspec_model_kv_io(ulspec_model* m, uint32_t layer, int dir, uint32_t pos0, uint32_t n, uint16_t* k,
                                 uint16_t* v);
/* ulspec_model_kv_io on sequence slot seq. */
ulspec_status ulspec_model_kv_io_seq(ulspec_model* m, uint32_t seq, uint32_t layer, int dir, uint32_t pos0,
                                     uint32_t n, uint16_t* k, uint16_t* v);

/* ---- GGUF files -------------------------------------------------------------
 * Read-only memory map of a GGUF v2/v3 file: header, metadata and tensor
 * table parsed with bounds checks; tensor data handed out as pointers into the
 * mapping.  No device work (usable without a GPU).  Replaces GGUFParser
 * (src/core/gguf_parser.h:37-90; parse / read_tensor_infos / read_tensor_data_direct,
 * src/core/gguf_parser.cpp:230-290,348-361, whose byte sizes are wrong, A2). */
typedef struct ulspec_gguf ulspec_gguf;
/* metadata value types (src/core/gguf_parser.h:12-26) */
enum {
    ULSPEC_GGUF_U8 = 0, ULSPEC_GGUF_I8 = 1, ULSPEC_GGUF_U16 = 2, ULSPEC_GGUF_I16 = 3, ULSPEC_GGUF_U32 = 4,
    ULSPEC_GGUF_I32 = 5, ULSPEC_GGUF_F32 = 6, ULSPEC_GGUF_BOOL = 7, ULSPEC_GGUF_STRING = 8, ULSPEC_GGUF_ARRAY = 9,
    ULSPEC_GGUF_U64 = 10, ULSPEC_GGUF_I64 = 11, ULSPEC_GGUF_F64 = 12
};
/* On failure *out is NULL and err (if given) holds the reason. */
ulspec_status ulspec_gguf_open(const char* path, ulspec_gguf** out, char* err, size_t err_len);
void          ulspec_gguf_close(ulspec_gguf* g);
const char*   ulspec_gguf_last_error(const ulspec_gguf* g);
ulspec_status ulspec_gguf_header(const ulspec_gguf* g, uint32_t* version, uint64_t* n_tensors, uint64_t* n_kv,
                                 uint64_t* alignment, uint64_t* data_offset);
/* Tensor i: ne[0] = elements per row (contiguous); offset relative to the data
 * section; nbytes = ne0 / blck * type_size * ne1 * ne2 * ne3, or 0 (and data
 * NULL) for a type without a fixed block layout.  name / data live until close. */
ulspec_status ulspec_gguf_tensor(const ulspec_gguf* g, uint64_t i, const char** name, uint32_t* ggml_type,
                                 uint32_t* n_dims, uint64_t ne[4], uint64_t* offset, uint64_t* nbytes,
                                 const void** data);
ulspec_status ulspec_gguf_find_tensor(const ulspec_gguf* g, const char* name, uint64_t* index);
/* Metadata entry i (array_type / array_len for ULSPEC_GGUF_ARRAY). */
ulspec_status ulspec_gguf_kv(const ulspec_gguf* g, uint64_t i, const char** key, uint32_t* value_type,
                             uint32_t* array_type, uint64_t* array_len);
/* The encoded value bytes of entry i (arrays: from the first element on), for
 * a caller that decodes string arrays such as tokenizer.ggml.tokens itself. */
ulspec_status ulspec_gguf_kv_bytes(const ulspec_gguf* g, uint64_t i, const void** data, uint64_t* nbytes);
/* Scalar lookups by key: integers and bools as int64, floats (and integers)
 * as double, strings as (pointer, length) into the mapping. */
ulspec_status ulspec_gguf_get_int(const ulspec_gguf* g, const char* key, int64_t* v);
ulspec_status ulspec_gguf_get_float(const ulspec_gguf* g, const char* key, double* v);
ulspec_status ulspec_gguf_get_str(const ulspec_gguf* g, const char* key, const char** v, uint64_t* len);
/* Llama configuration from the metadata (llama.embedding_length, block_count,
 * attention.head_count[_kv], feed_forward_length, context_length,
 * attention.layer_norm_rms_epsilon, rope.freq_base) and the vocabulary from
 * token_embd.weight; max_ctx 0 = llama.context_length. */
ulspec_status ulspec_gguf_llama_cfg(const ulspec_gguf* g, uint32_t max_ctx, ulspec_model_cfg* cfg);
/* Model from a GGUF file: every tensor by name through ulspec_model_set_tensor
 * (Model::load_from_gguf, src/inference/model.cpp:190-246).  Matrices may be
 * Q4_0, Q4_K, Q6_K, Q8_0 or F16 (what Q4_K_M files mix); a tensor of another
 * type fails with ULSPEC_EUNSUPPORTED naming it.  The file may be closed
 * afterwards. */
ulspec_status ulspec_model_load_gguf(ulspec_ctx* ctx, const ulspec_gguf* g, uint32_t max_ctx, ulspec_model** out);
/* The same with K/V caches for n_seq sequences (1 .. 8; a batch model as
 * ulspec_model_create_batch makes), for InferenceAPI::generate_batch
 * (src/api/inference_api.h:63) over the batched loop. */
ulspec_status ulspec_model_load_gguf_batch(ulspec_ctx* ctx, const ulspec_gguf* g, uint32_t max_ctx, uint32_t n_seq,
                                           ulspec_model** out);

/* ---- speculative decoding loop --------------------------------------------
 * One step (all on the device, captured once into a HIP graph and replayed):
 * the draft model takes the last two committed tokens (positions n-2, n-1),
 * then k-1 single-token forwards, sampling d_1 .. d_k from warp(draft logits)
 * with uniforms u(seed, s*(2k+1) + j); the target scores [t_{n-1}, d_1 .. d_k]
 * at positions n-1 .. n-1+k; ulspec_accept's rule with uniforms
 * u(seed, s*(2k+1) + k + j) emits n_accepted + 1 tokens, which are committed
 * (stale K/V rows past them are overwritten by the next step).  Replaces
 * SpeculativeDecoder::generate_with_speculation
 * (src/inference/speculative_decoder.cpp:25-71).
 * k = 0 (draft may be NULL): plain decoding of the target, the reference's
 * path with speculation off -- a step forwards t_{n-1} and samples t_n from
 * warp(target logits) with u(seed, s).  k <= 15 (k + 1 verify rows of the
 * 16 one forward takes). */
typedef struct ulspec_spec ulspec_spec;
ulspec_status ulspec_spec_create(ulspec_model* target, ulspec_model* draft, uint32_t k, const ulspec_sampling* s,
                                 uint64_t seed, ulspec_spec** out);
/* The same loop over n_seq <= 8 sequences at once (models created with at
 * least n_seq slots, (k+1) n_seq <= 48): every forward takes one group of
 * rows per sequence (M = (k+1) n_seq verify rows through the target), each
 * sequence on its own cache slot and positions; the accept rule runs over
 * the n_seq sequences.  Sequence b of step s uses uniforms
 * u(seed, (s n_seq + b)(2k+1) + j) (n_seq = 1: the counters above).  The
 * batch of the reference's generate_batch (src/api/inference_api.h:63). */
ulspec_status ulspec_spec_create_batch(ulspec_model* target, ulspec_model* draft, uint32_t k,
                                       const ulspec_sampling* s, uint64_t seed, uint32_t n_seq, ulspec_spec** out);
/* Tree steps over a fixed draft tree (one sequence): n <= 16 nodes in
 * breadth-first order (parent, HOST int32 [n]: parent[0] = -1, parent[i] in
 * [0, i), depths non-decreasing, each node's children consecutive; node 0 is
 * the last committed token).  Per step the draft runs one tree-masked forward
 * per level over [t_{n-2}, root, nodes so far] and draws the children of each
 * level from their parent's logits (sampling: i.i.d. with node i's uniform
 * u(seed, s(2n-1) + i - 1); greedy: the parent's best tokens in order), the
 * target scores the n nodes in one tree forward, ulspec_accept_tree's rule
 * (uniforms u(seed, s(2n-1) + n - 1 + j)) picks the path, both K/V caches are
 * compacted along it and path + final token are committed (a chain of k+1
 * nodes is the chain loop, counters included).  Replaces
 * TreeSpeculation::generate_tree_speculation / verify_tree
 * (src/inference/speculative_decoder.h:62-87, .cpp:118-176).  Prompts need
 * at least 2 tokens; ulspec_spec_state's `proposed` counts the tree depth per
 * step. */
ulspec_status ulspec_spec_create_tree(ulspec_model* target, ulspec_model* draft, uint32_t n, const int32_t* parent,
                                      const ulspec_sampling* s, uint64_t seed, ulspec_spec** out);
/* The last tree step's target logits [n][V], draft logits of nodes 0 .. n-2
 * [n-1][V] (rows of leaf nodes are not written), node tokens [n], uniforms
 * [2n-1], ulspec_accept_tree's tokens [n] and path [n], and n_accepted.
 * Synchronous. */
ulspec_status ulspec_spec_tree_last_step(ulspec_spec* sp, float* target_logits, float* draft_logits,
                                         int32_t* tokens, float* uniforms, int32_t* out_tokens, int32_t* path,
                                         int32_t* n_accepted);
void          ulspec_spec_destroy(ulspec_spec* sp);
/* Commit the prompt (n >= 1): both models process tokens 0 .. n-2; token n-1
 * is pending.  Resets the counters.  With n = 1 and k > 0 the first step is a
 * plain step (u(seed, 0)): the draft's catch-up pair needs two tokens.
 * Synchronous. */
ulspec_status ulspec_spec_prefill(ulspec_spec* sp, const int32_t* prompt, uint32_t n);
/* Prefill of a batch loop: the n_seq prompts concatenated, lens[b] >= 2
 * tokens each (>= 1 for k = 0). */
ulspec_status ulspec_spec_prefill_batch(ulspec_spec* sp, const int32_t* prompts, const uint32_t* lens);
/* Enqueue n_steps steps (asynchronous); EINVAL if they could overrun the
 * context (each step commits at most k+1 tokens). */
ulspec_status ulspec_spec_steps(ulspec_spec* sp, uint32_t n_steps);
/* Steps until at least n_new tokens were committed by this call (by every
 * sequence); *n_out = the number committed (the fewest of any sequence, up to
 * n_new + k).  Synchronous. */
ulspec_status ulspec_spec_generate(ulspec_spec* sp, uint32_t n_new, uint32_t* n_out);
/* Synchronises, then reports committed tokens (prompt included), steps,
 * accepted draft tokens and proposed draft tokens since the prefill (sums
 * over the sequences of a batch). */
ulspec_status ulspec_spec_state(ulspec_spec* sp, uint32_t* n_tokens, uint64_t* steps, uint64_t* accepted,
                                uint64_t* proposed);
/* The same for sequence seq of a batch. */
ulspec_status ulspec_spec_seq_state(ulspec_spec* sp, uint32_t seq, uint32_t* n_tokens, uint64_t* accepted,
                                    uint64_t* proposed);
/* Committed tokens start .. start+n-1 (of sequence 0) to host memory.  Synchronous. */
ulspec_status ulspec_spec_tokens(ulspec_spec* sp, uint32_t start, uint32_t n, int32_t* out);
ulspec_status ulspec_spec_seq_tokens(ulspec_spec* sp, uint32_t seq, uint32_t start, uint32_t n, int32_t* out);
/* Inputs and outputs of the last step, copied to host arrays (any may be
 * NULL), sequence-major for a batch of B: target logits [B][k+1][V], draft
 * logits [B][k][V], draft tokens [B][k], uniforms [B][2k+1], emitted tokens
 * [B][k+1] (-1 padded), n_accepted [B].  Synchronous.  For checking a step
 * against a CPU restatement. */
ulspec_status ulspec_spec_last_step(ulspec_spec* sp, float* target_logits, float* draft_logits,
                                    int32_t* draft_tokens, float* uniforms, int32_t* out_tokens,
                                    int32_t* n_accepted);
/* use_graph != 0 (default): replay the step captured as a HIP graph;
 * 0: launch the step's kernels directly on the stream. */
ulspec_status ulspec_spec_set_graph(ulspec_spec* sp, int use_graph);

#ifdef __cplusplus
}
#endif
#endif
