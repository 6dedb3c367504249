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
        _Float16* kc = nullptr;  // [n_seq][max_ctx][Hkv][D]
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

    // activations, up to rows_cap rows per forward (kRows per sequence;
    // n_seq sequence slots, each with its own K / V cache).  GEMM inputs are
    // fp32 activations held as split fp16 pairs [2 rows][width] (high parts,
    // then low parts): the attention output and SiLU(gate) * up.
    static constexpr uint32_t kRows = 16;
    static constexpr uint32_t kBatchRows = 48;  // rows of a batched forward (8 sequences x 6)
    uint32_t rows_max = 0;     // rows of one sequence per forward
    uint32_t rows_cap = 0;     // rows of all sequences of one forward
    uint32_t n_seq = 1;
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
    int32_t* lin_pos = nullptr;  // [1] the position of ulspec_model_linear calls
    int64_t lin_pos_set = -1;    // the value last written there (-1: none)
    float* attn_part = nullptr;
    size_t attn_part_bytes = 0;
    _Float16* xg = nullptr;    // split [2 rows_cap][dim]: the LM head's rows gathered from xn
    float* pg = nullptr;       // [rows_cap][pss_stride]: their row-scale partials
    _Float16** kv_tab = nullptr;  // device [2][n_layers]: every layer's K cache, then every V cache
    std::vector<void*> allocs;

    // The rows of one forward (see forward): M = nseq groups of r rows,
    // group b on sequence slot seq0 + b from position pos_dev[b] + pos_add;
    // a tree's rows take RoPE position pos + depth (4 bits per row).
    struct Rows {
        uint32_t M, r, nseq, seq0;
        const int32_t* pos_dev;
        int32_t pos_add;
        bool tree;
        uint64_t depth_bits;
    };
    enum { kLinQkv = 0, kLinO = 1, kLinGateUp = 2, kLinDown = 3, kLinHead = 4 };

    bool complete() const;
    ulspec::GemmFuse fuse_base() const;
    void normed(ulspec::GemmFuse& f, const float* pss_rows, int P) const;
    // One linear of layer l with its fused prologue / epilogue, on the
    // model's activation buffers (P: RMSNorm partials per row of h).
    ulspec_status linear(uint32_t l, int which, const Rows& rows, int P);
    // Forward M tokens read from device memory: nseq groups of r = M / nseq
    // <= rows_max rows, group b on sequence slot seq0 + b at positions
    // pos_dev[b] + pos_add ... (pos_dev: nseq device ints); logits of the
    // last n_logits rows of every group to `logits` (device, [nseq][n_logits]
    // [vocab]).  With `parent` (host [M], parent[i] in [-1, i); one sequence)
    // the rows are a tree: row i keeps its K/V slot (pos + i) but takes RoPE
    // position pos + depth(i) and attends to the prefix and its ancestors
    // only.  Asynchronous, never allocates or synchronises.
    ulspec_status forward(const int32_t* tok_dev, uint32_t M, const int32_t* pos_dev, int32_t pos_add,
                          float* logits_dev, uint32_t n_logits, const int32_t* parent = nullptr, uint32_t nseq = 1,
                          uint32_t seq0 = 0);
    // Host tokens on sequence slot seq (chunks of rows_max rows), logits of the
    // last n_logits rows to host memory.  Synchronous.
    ulspec_status forward_host(const int32_t* tokens, uint32_t M, uint32_t pos, float* logits, uint32_t n_logits,
                               uint32_t seq);
};

namespace ulspec {
void launch_set_i32(hipStream_t st, int32_t* p, int32_t v);
// K/V rows pos + path[j] -> pos + j, j = 1 .. min(*n_acc + 1, n_max) - 1, in
// every layer (pos = *pos_dev + pos_add); see kv_compact_kernel.
void launch_kv_compact(hipStream_t st, _Float16* const* kv_tab, uint32_t n_layers, uint32_t kvdim, uint32_t max_ctx,
                       const int32_t* pos_dev, int32_t pos_add, const int32_t* path, const int32_t* n_acc,
                       uint32_t n_max);
}
