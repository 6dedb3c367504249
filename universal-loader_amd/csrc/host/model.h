// model.h -- device state of one Llama-shaped model and its forward pass
// (shared by the model and speculative-loop translation units).
#pragma once

#include <map>
#include <string>
#include <vector>

#include "../ulspec_internal.h"

struct ulspec_model {
    // One fused weight assembled from several GGUF tensors (Q | K | V rows
    // concatenated, gate / up rows interleaved); each part is kept as given
    // until all have arrived.
    struct Pending {
        struct Part {
            uint8_t* dev = nullptr;  // the part's GGUF blocks (device)
            uint32_t type = 0;
            uint64_t rows = 0;
        };
        Part part[3];             // Q, K, V or gate, up
        uint32_t have = 0;        // bitmask of parts received
        uint32_t need = 0;
    };
    struct Layer {
        uint32_t wqkv = ~0u, wo = ~0u, wgu = ~0u, wdown = ~0u;  // context weight ids
        float* attn_norm = nullptr;
        float* ffn_norm = nullptr;
        _Float16* kc = nullptr;  // [max_ctx][Hkv][D]
        _Float16* vc = nullptr;
    };

    ulspec_ctx* ctx = nullptr;
    ulspec_model_cfg cfg{};
    uint32_t head_dim = 0;
    std::vector<Layer> layers;
    std::map<std::string, Pending> pending;
    uint8_t* embed = nullptr;  // raw GGUF [vocab][dim]
    uint32_t embed_type = 0;
    size_t embed_bytes = 0;    // its allocation
    float* out_norm = nullptr;
    uint32_t w_out = ~0u;
    float2* rope = nullptr;    // [max_ctx][head_dim / 2] (cos, sin)

    // activations, up to kRows rows per forward.  GEMM inputs are fp32
    // activations held as split fp16 pairs [2 rows][width] (high parts, then
    // low parts): the attention output and SiLU(gate) * up.
    static constexpr uint32_t kRows = 16;
    uint32_t rows_max = 0;
    float* h = nullptr;        // [kRows][dim] residual stream (fp32)
    float* pss = nullptr;      // [kRows][pss_stride] RMSNorm partial sums of h^2
    uint32_t pss_stride = 0;
    float* logits = nullptr;   // [kRows][vocab]
    _Float16* q16 = nullptr;   // [kRows][H D] (attention queries, fp16)
    _Float16* att = nullptr;   // split [2 kRows][H D]
    _Float16* act = nullptr;   // split [2 kRows][F]
    _Float16* xn = nullptr;    // split [2 kRows][dim]: h times the next RMSNorm's weights (the next GEMM's X)
    float* part = nullptr;     // split-K slice partials
    size_t part_bytes = 0;
    int32_t* tok = nullptr;    // [kRows]
    int32_t* pos = nullptr;    // [1]
    float* attn_part = nullptr;
    _Float16** kv_tab = nullptr;  // device [2][n_layers]: every layer's K cache, then every V cache
    std::vector<void*> allocs;

    bool complete() const;
    // Forward M <= rows_max tokens read from device memory at positions
    // *pos_dev + pos_add ...; logits of the last n_logits rows to `logits`
    // (device).  With `parent` (host [M], parent[i] in [-1, i)) the rows are
    // a tree: row i keeps its K/V slot (pos + i) but takes RoPE position pos +
    // depth(i) and attends to the prefix and its ancestors only.
    // Asynchronous, never allocates or synchronises.
    ulspec_status forward(const int32_t* tok_dev, uint32_t M, const int32_t* pos_dev, int32_t pos_add,
                          float* logits_dev, uint32_t n_logits, const int32_t* parent = nullptr);
};

namespace ulspec {
void launch_set_i32(hipStream_t st, int32_t* p, int32_t v);
// K/V rows pos + path[j] -> pos + j, j = 1 .. min(*n_acc + 1, n_max) - 1, in
// every layer (pos = *pos_dev + pos_add); see kv_compact_kernel.
void launch_kv_compact(hipStream_t st, _Float16* const* kv_tab, uint32_t n_layers, uint32_t kvdim, uint32_t max_ctx,
                       const int32_t* pos_dev, int32_t pos_add, const int32_t* path, const int32_t* n_acc,
                       uint32_t n_max);
}
