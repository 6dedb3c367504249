// ulspec_inference.hpp -- C++ host classes over the C ABI of ulspec.h, with the
// shapes of the reference's speculative-decoding classes, so that
// src/inference and src/api can call the gfx950 path in place of their own:
//
//   ulspec_inference::SpeculationResult   <- inference::SpeculationResult
//                                            (src/inference/speculative_decoder.h:17-22)
//   ulspec_inference::SpeculativeDecoder  <- inference::SpeculativeDecoder
//                                            (src/inference/speculative_decoder.h:24-60)
//   ulspec_inference::InferenceAPI        <- the speculative-decoding and sampling
//                                            subset of py::InferenceAPI
//                                            (src/api/inference_api.h:52-123)
//
// Header only; link against libulspec.so.  Errors: the reference returns bool
// or throws from its parser (src/core/gguf_parser.cpp:23,63,69); here every
// failing ABI call throws ulspec_inference::Error carrying the status and the
// context's message.  Not thread-safe: one object per host thread, as the
// reference serialises every InferenceAPI call behind api_mutex_
// (src/api/inference_api.h:115) -- InferenceAPI below does the same.
#pragma once

#include <cstdint>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include "ulspec.h"

namespace ulspec_inference {

class Error : public std::runtime_error {
public:
    Error(ulspec_status st, const std::string& msg) : std::runtime_error(msg), status(st) {}
    ulspec_status status;
};

inline void check(ulspec_ctx* ctx, ulspec_status st, const char* what)
{
    if (st != ULSPEC_OK)
        throw Error(st, std::string(what) + ": " + (ctx ? ulspec_last_error(ctx) : ulspec_status_str(st)));
}

// One device context (one HIP stream on one gfx950 GPU).
class Context {
public:
    explicit Context(int device = 0)
    {
        check(nullptr, ulspec_create(device, &ctx_), "ulspec_create");
    }
    ~Context() { ulspec_destroy(ctx_); }
    Context(const Context&) = delete;
    Context& operator=(const Context&) = delete;
    ulspec_ctx* get() const { return ctx_; }

private:
    ulspec_ctx* ctx_ = nullptr;
};

// A memory-mapped GGUF file (GGUFParser, src/core/gguf_parser.h:37-90, with
// the GGUF block sizes); host only.
class GGUFFile {
public:
    explicit GGUFFile(const std::string& path)
    {
        char err[512] = {0};
        const ulspec_status st = ulspec_gguf_open(path.c_str(), &g_, err, sizeof(err));
        if (st != ULSPEC_OK) throw Error(st, std::string("ulspec_gguf_open: ") + err);
    }
    ~GGUFFile() { ulspec_gguf_close(g_); }
    GGUFFile(const GGUFFile&) = delete;
    GGUFFile& operator=(const GGUFFile&) = delete;
    const ulspec_gguf* get() const { return g_; }
    ulspec_model_cfg llama_cfg(uint32_t max_ctx = 0) const
    {
        ulspec_model_cfg c{};
        const ulspec_status st = ulspec_gguf_llama_cfg(g_, max_ctx, &c);
        if (st != ULSPEC_OK) throw Error(st, std::string("ulspec_gguf_llama_cfg: ") + ulspec_gguf_last_error(g_));
        return c;
    }

private:
    ulspec_gguf* g_ = nullptr;
};

// A Llama-shaped model whose tensors are given by GGUF name and raw block bytes
// (the weight map of Model::load_from_gguf, src/inference/model.cpp:190-246),
// or read from a GGUF file.
class Model {
public:
    Model(Context& ctx, const ulspec_model_cfg& cfg) : ctx_(ctx.get()), cfg_(cfg)
    {
        check(ctx_, ulspec_model_create(ctx_, &cfg, &m_), "ulspec_model_create");
    }
    // InferenceEngine::load_model (src/inference/inference_engine.cpp:150-181)
    Model(Context& ctx, const GGUFFile& file, uint32_t max_ctx = 0) : ctx_(ctx.get()), cfg_(file.llama_cfg(max_ctx))
    {
        check(ctx_, ulspec_model_load_gguf(ctx_, file.get(), max_ctx, &m_), "ulspec_model_load_gguf");
    }
    ~Model() { ulspec_model_destroy(m_); }
    Model(const Model&) = delete;
    Model& operator=(const Model&) = delete;

    void set_tensor(const std::string& name, uint32_t ggml_type, const void* data, size_t nbytes, uint64_t ne0,
                    uint64_t ne1)
    {
        check(ctx_, ulspec_model_set_tensor(m_, name.c_str(), ggml_type, data, nbytes, ne0, ne1, 0),
              "ulspec_model_set_tensor");
    }
    // Logits of the last token (InferenceEngine::get_token_logits,
    // src/inference/inference_engine.cpp:818-820, which returns nothing).
    std::vector<float> token_logits(const std::vector<uint32_t>& tokens, uint32_t pos = 0)
    {
        std::vector<int32_t> t(tokens.begin(), tokens.end());
        std::vector<float> out(cfg_.vocab);
        check(ctx_, ulspec_model_forward(m_, t.data(), (uint32_t)t.size(), pos, out.data(), 1), "ulspec_model_forward");
        return out;
    }
    ulspec_model* get() const { return m_; }
    ulspec_ctx* ctx() const { return ctx_; }
    const ulspec_model_cfg& cfg() const { return cfg_; }

private:
    ulspec_ctx* ctx_;
    ulspec_model_cfg cfg_;
    ulspec_model* m_ = nullptr;
};

struct SpeculationResult {
    std::vector<uint32_t> accepted_tokens;  // accepted drafts + the corrected / bonus token
    std::vector<uint32_t> rejected_tokens;  // drafts after the first rejection
    uint32_t num_accepted = 0;              // accepted drafts
    float acceptance_rate = 0.0f;           // num_accepted / k for this step
};

// The reference's class shape (ctor arguments, set_speculation_length,
// update_acceptance_stats, get_acceptance_rate starting at 0.5 and cumulative
// afterwards); drafting and verification run on the device instead of host
// callbacks.  acceptance_threshold is kept for the signature: the
// speculative-sampling rule has no threshold.
class SpeculativeDecoder {
public:
    SpeculativeDecoder(uint32_t vocab_size, uint32_t max_spec_len, float acceptance_threshold)
        : vocab_(vocab_size), k_(max_spec_len), threshold_(acceptance_threshold)
    {
    }
    ~SpeculativeDecoder() { ulspec_spec_destroy(sp_); }
    SpeculativeDecoder(const SpeculativeDecoder&) = delete;
    SpeculativeDecoder& operator=(const SpeculativeDecoder&) = delete;

    void set_speculation_length(uint32_t len)
    {
        k_ = len;
        reset_device();
    }
    // Bind the target (verifier) and draft models and the sampling rule.
    void attach(Model& target, Model& draft, const ulspec_sampling& s, uint64_t seed)
    {
        if (target.cfg().vocab != vocab_) throw Error(ULSPEC_EINVAL, "vocabulary size differs from the decoder's");
        target_ = &target;
        draft_ = &draft;
        s_ = s;
        seed_ = seed;
        reset_device();
    }
    void prefill(const std::vector<uint32_t>& prompt)
    {
        ensure();
        std::vector<int32_t> p(prompt.begin(), prompt.end());
        check(ctx(), ulspec_spec_prefill(sp_, p.data(), (uint32_t)p.size()), "ulspec_spec_prefill");
    }
    // One step: k drafts, one verification, commit
    // (SpeculativeDecoder::generate_with_speculation, speculative_decoder.cpp:25-71).
    SpeculationResult generate_with_speculation()
    {
        ensure();
        check(ctx(), ulspec_spec_steps(sp_, 1), "ulspec_spec_steps");
        std::vector<int32_t> drafts(k_), out(k_ + 1);
        int32_t nacc = 0;
        check(ctx(), ulspec_spec_last_step(sp_, nullptr, nullptr, drafts.data(), nullptr, out.data(), &nacc),
              "ulspec_spec_last_step");
        SpeculationResult r;
        for (int32_t i = 0; i <= nacc; ++i) r.accepted_tokens.push_back((uint32_t)out[i]);
        for (uint32_t i = (uint32_t)nacc; i < k_; ++i) r.rejected_tokens.push_back((uint32_t)drafts[i]);
        r.num_accepted = (uint32_t)nacc;
        r.acceptance_rate = k_ ? (float)nacc / (float)k_ : 0.0f;
        update_acceptance_stats((uint32_t)nacc, k_);
        return r;
    }
    // Generate at least n_new tokens; returns the committed sequence after the prompt.
    std::vector<uint32_t> generate(uint32_t n_new)
    {
        ensure();
        uint32_t n0 = 0, n1 = 0;
        uint64_t acc0 = 0, prop0 = 0, acc1 = 0, prop1 = 0;
        check(ctx(), ulspec_spec_state(sp_, &n0, nullptr, &acc0, &prop0), "ulspec_spec_state");
        uint32_t got = 0;
        check(ctx(), ulspec_spec_generate(sp_, n_new, &got), "ulspec_spec_generate");
        check(ctx(), ulspec_spec_state(sp_, &n1, nullptr, &acc1, &prop1), "ulspec_spec_state");
        update_acceptance_stats((uint32_t)(acc1 - acc0), (uint32_t)(prop1 - prop0));
        std::vector<int32_t> t(n1 - n0);
        if (!t.empty()) check(ctx(), ulspec_spec_tokens(sp_, n0, (uint32_t)t.size(), t.data()), "ulspec_spec_tokens");
        return std::vector<uint32_t>(t.begin(), t.end());
    }
    void update_acceptance_stats(uint32_t accepted, uint32_t total)
    {
        total_ += total;
        accepted_ += accepted;
        if (total_) rate_ = (float)accepted_ / (float)total_;
    }
    float get_acceptance_rate() const { return rate_; }
    float acceptance_threshold() const { return threshold_; }

private:
    ulspec_ctx* ctx() const { return target_ ? target_->ctx() : nullptr; }
    void reset_device()
    {
        ulspec_spec_destroy(sp_);
        sp_ = nullptr;
    }
    void ensure()
    {
        if (!target_ || !draft_) throw Error(ULSPEC_EINVAL, "attach() the target and draft models first");
        if (!sp_) check(ctx(), ulspec_spec_create(target_->get(), draft_->get(), k_, &s_, seed_, &sp_), "ulspec_spec_create");
    }

    uint32_t vocab_, k_;
    float threshold_;
    float rate_ = 0.5f;  // as the reference's constructor (speculative_decoder.cpp:10)
    uint64_t total_ = 0, accepted_ = 0;
    Model* target_ = nullptr;
    Model* draft_ = nullptr;
    ulspec_sampling s_{1.0f, 0, 1.0f, 1};
    uint64_t seed_ = 0;
    ulspec_spec* sp_ = nullptr;
};

// The speculative-decoding and sampling entry points of py::InferenceAPI.
class InferenceAPI {
public:
    InferenceAPI(Model& target, Model& draft, uint32_t max_spec_len = 4, uint64_t seed = 0)
        : target_(target), draft_(draft), dec_(target.cfg().vocab, max_spec_len, 0.0f), k_(max_spec_len), seed_(seed)
    {
    }
    void enable_speculative_decoding(bool enable)  // inference_api.cpp:214-216
    {
        std::lock_guard<std::mutex> lock(mu_);
        spec_ = enable;
    }
    float get_acceptance_rate() const  // inference_api.cpp:222-225
    {
        std::lock_guard<std::mutex> lock(mu_);
        return dec_.get_acceptance_rate();
    }
    void set_temperature(float t)  // inference_api.cpp:232-245
    {
        std::lock_guard<std::mutex> lock(mu_);
        s_.temperature = t;
    }
    void set_top_p(float p)
    {
        std::lock_guard<std::mutex> lock(mu_);
        s_.top_p = p;
    }
    void set_top_k(uint32_t k)
    {
        std::lock_guard<std::mutex> lock(mu_);
        s_.top_k = k;
    }
    void set_greedy(bool g)
    {
        std::lock_guard<std::mutex> lock(mu_);
        s_.greedy = g ? 1 : 0;
    }
    std::vector<float> get_token_logits(const std::vector<uint32_t>& tokens)  // inference_api.cpp:277-280
    {
        std::lock_guard<std::mutex> lock(mu_);
        return target_.token_logits(tokens);
    }
    // Token-level generation: the prompt, then at least max_tokens tokens
    // (speculative when enabled; otherwise k = 1 steps of the same loop).
    std::vector<uint32_t> generate_tokens(const std::vector<uint32_t>& prompt, uint32_t max_tokens)
    {
        std::lock_guard<std::mutex> lock(mu_);
        dec_.set_speculation_length(spec_ ? k_ : 1);
        dec_.attach(target_, draft_, s_, seed_);
        dec_.prefill(prompt);
        std::vector<uint32_t> out = dec_.generate(max_tokens);
        if (out.size() > max_tokens) out.resize(max_tokens);
        return out;
    }

private:
    Model& target_;
    Model& draft_;
    SpeculativeDecoder dec_;
    ulspec_sampling s_{1.0f, 0, 1.0f, 0};
    uint32_t k_;
    uint64_t seed_;
    bool spec_ = false;
    mutable std::mutex mu_;
};

}  // namespace ulspec_inference
