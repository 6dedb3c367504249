// ref_shim.cpp -- C entry points over the reference's own CPU functions for
// this path, compiled from their sources under /root/reference by the `ref`
// target of oracle/Makefile into oracle/_ref/libref.so.  Test infrastructure:
// used only to cross-check the oracle.
//   cpu::softmax_f32 / cpu::silu_f32   src/cpu_backend/activation_cpu.cpp:14-37
//   SpeculativeDecoder stats          src/inference/speculative_decoder.cpp:8-13,112-116
//   ggml_blck_size / ggml_type_size   src/core/gguf_types.h:35-81 (header only)
#include <cstddef>
#include <cstdint>

#include "activation_cpu.h"
#include "gguf_types.h"
#include "speculative_decoder.h"

extern "C" {

void ref_softmax_f32(float* dst, const float* src, size_t n) { cpu::softmax_f32(dst, src, n); }
void ref_silu_f32(float* dst, const float* src, size_t n) { cpu::silu_f32(dst, src, n); }

void* ref_specdec_create(uint32_t vocab, uint32_t max_spec_len, float threshold)
{
    return new inference::SpeculativeDecoder(vocab, max_spec_len, threshold);
}
void ref_specdec_update(void* d, uint32_t accepted, uint32_t total)
{
    static_cast<inference::SpeculativeDecoder*>(d)->update_acceptance_stats(accepted, total);
}
float ref_specdec_rate(void* d) { return static_cast<inference::SpeculativeDecoder*>(d)->get_acceptance_rate(); }
void ref_specdec_free(void* d) { delete static_cast<inference::SpeculativeDecoder*>(d); }

int ref_ggml_blck_size(uint32_t t) { return ggml::ggml_blck_size(static_cast<ggml::GGMLType>(t)); }
size_t ref_ggml_type_size(uint32_t t) { return ggml::ggml_type_size(static_cast<ggml::GGMLType>(t)); }
}
