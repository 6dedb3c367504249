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
//                                            (src/api/inference_api.h:52-123),
//                                            with GenerationConfig / GenerationResult
//                                            (inference_api.h:14-30)
//
// Header only; link against libulspec.so.  Errors: the reference returns bool
// or throws from its parser (src/core/gguf_parser.cpp:23,63,69); here every
// failing ABI call throws ulspec_inference::Error carrying the status and the
// context's message.  Not thread-safe: one object per host thread, as the
// reference serialises every InferenceAPI call behind api_mutex_
// (src/api/inference_api.h:115) -- InferenceAPI below does the same.
#pragma once

#include <algorithm>
#include <chrono>
#include <cstdint>
#include <cstring>
#include <functional>
#include <memory>
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
    // The strings of an array-of-strings entry (tokenizer.ggml.tokens); empty if absent.
    std::vector<std::string> str_array(const std::string& key) const
    {
        uint64_t n_kv = 0;
        std::vector<std::string> out;
        if (ulspec_gguf_header(g_, nullptr, nullptr, &n_kv, nullptr, nullptr) != ULSPEC_OK) return out;
        for (uint64_t i = 0; i < n_kv; ++i) {
            const char* k = nullptr;
            uint32_t t = 0, at = 0;
            uint64_t n = 0;
            if (ulspec_gguf_kv(g_, i, &k, &t, &at, &n) != ULSPEC_OK || key != k) continue;
            if (t != ULSPEC_GGUF_ARRAY || at != ULSPEC_GGUF_STRING) return out;
            const void* data = nullptr;
            uint64_t nb = 0;
            if (ulspec_gguf_kv_bytes(g_, i, &data, &nb) != ULSPEC_OK) return out;
            const uint8_t* b = (const uint8_t*)data;
            uint64_t pos = 0;
            for (uint64_t j = 0; j < n && pos + 8 <= nb; ++j) {
                uint64_t len = 0;
                std::memcpy(&len, b + pos, 8);
                if (len > nb - pos - 8) break;
                out.emplace_back((const char*)b + pos + 8, (size_t)len);
                pos += 8 + len;
            }
            return out;
        }
        return out;
    }
    uint64_t data_bytes() const
    {
        uint64_t n_t = 0, total = 0;
        if (ulspec_gguf_header(g_, nullptr, &n_t, nullptr, nullptr, nullptr) != ULSPEC_OK) return 0;
        for (uint64_t i = 0; i < n_t; ++i) {
            uint64_t nb = 0, ne[4];
            uint32_t t, nd;
            uint64_t off;
            const char* name;
            const void* d;
            if (ulspec_gguf_tensor(g_, i, &name, &t, &nd, ne, &off, &nb, &d) == ULSPEC_OK) total += nb;
        }
        return total;
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
        : vocab_(vocab_size), k_(max_spec_len), max_len_(max_spec_len), threshold_(acceptance_threshold)
    {
    }
    ~SpeculativeDecoder() { ulspec_spec_destroy(sp_); }
    SpeculativeDecoder(const SpeculativeDecoder&) = delete;
    SpeculativeDecoder& operator=(const SpeculativeDecoder&) = delete;

    // 0: plain decoding of the target (the draft model is not used).
    void set_speculation_length(uint32_t len)
    {
        k_ = len;
        max_len_ = len;
        reset_device();
    }
    // Bind the target (verifier) and draft models and the sampling rule.
    void attach(Model& target, Model* draft, const ulspec_sampling& s, uint64_t seed)
    {
        if (target.cfg().vocab != vocab_) throw Error(ULSPEC_EINVAL, "vocabulary size differs from the decoder's");
        target_ = &target;
        draft_ = draft;
        s_ = s;
        seed_ = seed;
        reset_device();
    }
    void attach(Model& target, Model& draft, const ulspec_sampling& s, uint64_t seed) { attach(target, &draft, s, seed); }
    void prefill(const std::vector<uint32_t>& prompt)
    {
        ensure();
        std::vector<int32_t> p(prompt.begin(), prompt.end());
        check(ctx(), ulspec_spec_prefill(sp_, p.data(), (uint32_t)p.size()), "ulspec_spec_prefill");
        started_ = true;
    }
    // One step: k drafts, one verification, commit
    // (SpeculativeDecoder::generate_with_speculation, speculative_decoder.cpp:25-71).
    SpeculationResult generate_with_speculation()
    {
        ensure();
        check(ctx(), ulspec_spec_steps(sp_, 1), "ulspec_spec_steps");
        return step_result();
    }
    SpeculationResult step_result()
    {
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
    // The reference's call shape (speculative_decoder.h:32-35): one step from
    // context_token with num_speculative_tokens drafts, capped at the
    // decoder's speculation length as the reference caps it.  The step
    // continues the committed sequence when context_token is its last token;
    // otherwise a new sequence starts from context_token alone (its first
    // step is plain: one target draw, no drafts).  Without attached models it
    // returns context_token, as the reference does without callbacks.
    SpeculationResult generate_with_speculation(uint32_t context_token, uint32_t num_speculative_tokens = 4)
    {
        SpeculationResult r;
        if (!target_ || !draft_) {
            r.accepted_tokens.push_back(context_token);
            return r;
        }
        const uint32_t k = std::max<uint32_t>(1, std::min(num_speculative_tokens, max_len_));
        if (k != k_) {
            k_ = k;
            reset_device();
        }
        ensure();
        uint32_t n = 0;
        uint64_t prop0 = 0, prop1 = 0;
        int32_t last = -1;
        if (started_) {
            check(ctx(), ulspec_spec_state(sp_, &n, nullptr, nullptr, &prop0), "ulspec_spec_state");
            if (n) check(ctx(), ulspec_spec_tokens(sp_, n - 1, 1, &last), "ulspec_spec_tokens");
        }
        if (!started_ || last != (int32_t)context_token) {
            const int32_t t = (int32_t)context_token;
            check(ctx(), ulspec_spec_prefill(sp_, &t, 1), "ulspec_spec_prefill");
            started_ = true;
            check(ctx(), ulspec_spec_state(sp_, &n, nullptr, nullptr, &prop0), "ulspec_spec_state");
        }
        check(ctx(), ulspec_spec_steps(sp_, 1), "ulspec_spec_steps");
        check(ctx(), ulspec_spec_state(sp_, nullptr, nullptr, nullptr, &prop1), "ulspec_spec_state");
        if (prop1 == prop0) {  // a plain step: one token, no drafts
            int32_t t = -1;
            check(ctx(), ulspec_spec_tokens(sp_, n, 1, &t), "ulspec_spec_tokens");
            r.accepted_tokens.push_back((uint32_t)t);
            return r;
        }
        return step_result();
    }
    // One step of the loop; the tokens it committed (any step kind).
    std::vector<uint32_t> step_tokens()
    {
        ensure();
        uint32_t n0 = 0, n1 = 0;
        uint64_t acc0 = 0, prop0 = 0, acc1 = 0, prop1 = 0;
        check(ctx(), ulspec_spec_state(sp_, &n0, nullptr, &acc0, &prop0), "ulspec_spec_state");
        check(ctx(), ulspec_spec_steps(sp_, 1), "ulspec_spec_steps");
        check(ctx(), ulspec_spec_state(sp_, &n1, nullptr, &acc1, &prop1), "ulspec_spec_state");
        update_acceptance_stats((uint32_t)(acc1 - acc0), (uint32_t)(prop1 - prop0));
        std::vector<int32_t> t(n1 - n0);
        if (n1 > n0) check(ctx(), ulspec_spec_tokens(sp_, n0, n1 - n0, t.data()), "ulspec_spec_tokens");
        return std::vector<uint32_t>(t.begin(), t.end());
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
    uint64_t accepted() const { return accepted_; }
    uint64_t proposed() const { return total_; }

private:
    ulspec_ctx* ctx() const { return target_ ? target_->ctx() : nullptr; }
    void reset_device()
    {
        ulspec_spec_destroy(sp_);
        sp_ = nullptr;
        started_ = false;
    }
    void ensure()
    {
        if (!target_ || (k_ && !draft_)) throw Error(ULSPEC_EINVAL, "attach() the target and draft models first");
        if (!sp_)
            check(ctx(), ulspec_spec_create(target_->get(), k_ && draft_ ? draft_->get() : nullptr, k_, &s_, seed_, &sp_),
                  "ulspec_spec_create");
    }

    uint32_t vocab_, k_, max_len_;
    bool started_ = false;
    float threshold_;
    float rate_ = 0.5f;  // as the reference's constructor (speculative_decoder.cpp:10)
    uint64_t total_ = 0, accepted_ = 0;
    Model* target_ = nullptr;
    Model* draft_ = nullptr;
    ulspec_sampling s_{1.0f, 0, 1.0f, 1};
    uint64_t seed_ = 0;
    ulspec_spec* sp_ = nullptr;
};

// py::GenerationConfig (src/api/inference_api.h:14-22) with the defaults of
// the InferenceAPI constructor (src/api/inference_api.cpp:9-17).
struct GenerationConfig {
    uint32_t max_tokens = 100;
    float temperature = 1.0f;
    float top_p = 0.9f;
    uint32_t top_k = 40;
    float frequency_penalty = 0.0f;
    float presence_penalty = 0.0f;
    bool do_sample = true;
};

// py::GenerationResult (src/api/inference_api.h:24-30).
struct GenerationResult {
    std::vector<uint32_t> tokens;
    std::string text;
    uint32_t num_tokens = 0;
    float time_ms = 0.0f;
    float tokens_per_second = 0.0f;
};

// py::GenerationProgress (src/api/inference_api.h:32-40).
struct GenerationProgress {
    uint32_t current_step = 0;
    uint32_t total_steps = 0;
    float progress_pct = 0.0f;
    float time_elapsed_ms = 0.0f;
    float estimated_remaining_ms = 0.0f;
    float tokens_per_second = 0.0f;
    std::string last_token;
};

// The speculative-decoding and sampling entry points of py::InferenceAPI.
// Models come from GGUF files (load_model / load_draft_model, on a Context)
// or from the caller (the Model& constructor).  Generation with speculation
// off is plain decoding of the target (one row, one draw per token); on, it
// is the device loop with max_spec_len drafts per step.
class InferenceAPI {
public:
    InferenceAPI(Model& target, Model& draft, uint32_t max_spec_len = 4, uint64_t seed = 0)
        : target_(&target), draft_(&draft), k_(max_spec_len), seed_(seed)
    {
    }
    // The reference's shape (inference_api.cpp:9-17): no model until load_model.
    explicit InferenceAPI(Context& ctx, uint32_t max_ctx = 0, uint32_t max_spec_len = 4, uint64_t seed = 0)
        : ctx_(&ctx), max_ctx_(max_ctx), k_(max_spec_len), seed_(seed)
    {
    }
    // InferenceAPI::load_model (inference_api.cpp:21-43): false on failure,
    // the reason in last_error().  Replaces any loaded target and draft.
    bool load_model(const std::string& path)
    {
        std::lock_guard<std::mutex> lock(mu_);
        if (!ctx_) return fail_("load_model needs the Context constructor");
        try {
            GGUFFile f(path);
            std::unique_ptr<Model> m(new Model(*ctx_, f, max_ctx_));
            drop_models_();
            own_target_ = std::move(m);
            target_ = own_target_.get();
            vocab_ = f.str_array("tokenizer.ggml.tokens");
            model_bytes_ = f.data_bytes();
            model_path_ = path;
            return true;
        } catch (const Error& e) {
            return fail_(e.what());
        }
    }
    // A draft model for speculative decoding (same vocabulary as the target).
    bool load_draft_model(const std::string& path)
    {
        std::lock_guard<std::mutex> lock(mu_);
        if (!ctx_ || !target_) return fail_("load the target model first");
        try {
            GGUFFile f(path);
            std::unique_ptr<Model> m(new Model(*ctx_, f, max_ctx_));
            if (m->cfg().vocab != target_->cfg().vocab) return fail_("draft and target vocabularies differ");
            own_draft_ = std::move(m);
            draft_ = own_draft_.get();
            return true;
        } catch (const Error& e) {
            return fail_(e.what());
        }
    }
    bool unload_model()  // inference_api.cpp:45-54
    {
        std::lock_guard<std::mutex> lock(mu_);
        if (own_target_) drop_models_();
        return true;
    }
    const std::string& last_error() const { return err_; }
    const std::string& model_path() const { return model_path_; }
    uint64_t model_size_bytes() const { return model_bytes_; }

    void enable_speculative_decoding(bool enable)  // inference_api.cpp:214-216
    {
        std::lock_guard<std::mutex> lock(mu_);
        spec_ = enable;
    }
    // Cumulative accepted / proposed drafts; 0.5 before any speculative step
    // (inference_api.cpp:222-225, the decoder's initial value).
    float get_acceptance_rate() const
    {
        std::lock_guard<std::mutex> lock(mu_);
        return proposed_ ? (float)accepted_ / (float)proposed_ : 0.5f;
    }
    float get_throughput() const
    {
        std::lock_guard<std::mutex> lock(mu_);
        return throughput_;
    }
    void set_temperature(float t)  // inference_api.cpp:232-245
    {
        std::lock_guard<std::mutex> lock(mu_);
        s_.temperature = t;
        config_.temperature = t;
    }
    void set_top_p(float p)
    {
        std::lock_guard<std::mutex> lock(mu_);
        s_.top_p = p;
        config_.top_p = p;
    }
    void set_top_k(uint32_t k)
    {
        std::lock_guard<std::mutex> lock(mu_);
        s_.top_k = k;
        config_.top_k = k;
    }
    void set_greedy(bool g)
    {
        std::lock_guard<std::mutex> lock(mu_);
        s_.greedy = g ? 1 : 0;
    }
    // str -> token ids for generate()'s text prompts (inference_api.cpp:368-370).
    void register_custom_tokenizer(std::function<std::vector<uint32_t>(const std::string&)> f)
    {
        std::lock_guard<std::mutex> lock(mu_);
        tokenizer_ = std::move(f);
    }
    std::vector<float> get_token_logits(const std::vector<uint32_t>& tokens)  // inference_api.cpp:277-280
    {
        std::lock_guard<std::mutex> lock(mu_);
        if (!target_) return {};
        return target_->token_logits(tokens);
    }
    // The GGUF vocabulary strings of the tokens joined ("▁" read as a space).
    std::string token_text(const std::vector<uint32_t>& tokens) const
    {
        std::string out;
        for (uint32_t t : tokens) {
            if (t >= vocab_.size()) continue;
            const std::string& w = vocab_[t];
            for (size_t i = 0; i < w.size();) {
                if (w.compare(i, 3, "\xe2\x96\x81") == 0) {
                    out += ' ';
                    i += 3;
                } else {
                    out += w[i++];
                }
            }
        }
        return out;
    }
    // Token-level generation with the API's sampling (set_temperature /
    // top_p / top_k / greedy): the prompt, then at least max_tokens tokens.
    std::vector<uint32_t> generate_tokens(const std::vector<uint32_t>& prompt, uint32_t max_tokens)
    {
        std::lock_guard<std::mutex> lock(mu_);
        return run_(prompt, max_tokens, s_);
    }
    // With a GenerationConfig (do_sample false: greedy); penalties are not
    // implemented and throw ULSPEC_EUNSUPPORTED.
    GenerationResult generate_tokens(const std::vector<uint32_t>& prompt, const GenerationConfig& config)
    {
        std::lock_guard<std::mutex> lock(mu_);
        const auto t0 = std::chrono::steady_clock::now();
        GenerationResult r;
        r.tokens = run_(prompt, config.max_tokens, sampling_(config));
        const float ms = std::chrono::duration<float, std::milli>(std::chrono::steady_clock::now() - t0).count();
        r.text = token_text(r.tokens);
        r.num_tokens = (uint32_t)r.tokens.size();
        r.time_ms = ms;
        r.tokens_per_second = ms > 0.0f ? r.num_tokens / (ms * 1e-3f) : 0.0f;
        throughput_ = r.tokens_per_second;
        return r;
    }
    // InferenceAPI::generate (inference_api.cpp:56-78): text in (through the
    // registered tokenizer), text out; "Error: No model loaded" without a model.
    std::string generate(const std::string& prompt, const GenerationConfig& config)
    {
        std::vector<uint32_t> ids;
        {
            std::lock_guard<std::mutex> lock(mu_);
            if (!target_) return "Error: No model loaded";
            if (!tokenizer_) throw Error(ULSPEC_EUNSUPPORTED, "text prompts need register_custom_tokenizer()");
            ids = tokenizer_(prompt);
        }
        return generate_tokens(ids, config).text;
    }
    // InferenceAPI::generate_streaming (inference_api.cpp:96-125): the
    // callback gets each new token's text as the loop commits it (one step,
    // then a host fence); returns the whole text.
    std::string generate_streaming(const std::string& prompt, const GenerationConfig& config,
                                   std::function<void(const std::string&)> token_callback)
    {
        return stream_(prompt, config, [&](const std::string& piece, uint32_t, float) {
            if (token_callback) token_callback(piece);
        });
    }
    // InferenceAPI::generate_with_progress (inference_api.cpp:127-162): a
    // GenerationProgress after each committed token; returns the text (the
    // reference returns an empty string: its result is never filled).
    std::string generate_with_progress(const std::string& prompt, const GenerationConfig& config,
                                       std::function<void(const GenerationProgress&)> progress_callback)
    {
        const uint32_t total = config.max_tokens;
        return stream_(prompt, config, [&](const std::string& piece, uint32_t done, float sec) {
            if (!progress_callback) return;
            GenerationProgress p;
            p.current_step = done;
            p.total_steps = total;
            p.progress_pct = total ? 100.0f * (float)done / (float)total : 100.0f;
            p.time_elapsed_ms = sec * 1e3f;
            p.tokens_per_second = sec > 0.0f ? (float)done / sec : 0.0f;
            p.estimated_remaining_ms = p.tokens_per_second > 0.0f ? (float)(total - done) / p.tokens_per_second * 1e3f
                                                                  : 0.0f;
            p.last_token = piece;
            progress_callback(p);
        });
    }
    // InferenceAPI::generate_batch (inference_api.cpp:164-175): generate()
    // for each prompt, in order, as the reference does (the Python module's
    // generate_batch steps the prompts together on the batched loop).
    std::vector<std::string> generate_batch(const std::vector<std::string>& prompts, const GenerationConfig& config)
    {
        std::vector<std::string> out;
        out.reserve(prompts.size());
        for (const auto& p : prompts) out.push_back(generate(p, config));
        return out;
    }
    GenerationResult generate_default(const std::string& prompt)  // inference_api.cpp:80-95
    {
        GenerationConfig c;
        {
            std::lock_guard<std::mutex> lock(mu_);
            c = config_;
        }
        std::vector<uint32_t> ids;
        {
            std::lock_guard<std::mutex> lock(mu_);
            if (!target_) {
                GenerationResult r;
                r.text = "Error: No model loaded";
                return r;
            }
            if (!tokenizer_) throw Error(ULSPEC_EUNSUPPORTED, "text prompts need register_custom_tokenizer()");
            ids = tokenizer_(prompt);
        }
        return generate_tokens(ids, c);
    }

private:
    bool fail_(const std::string& why)
    {
        err_ = why;
        return false;
    }
    void drop_models_()
    {
        draft_ = nullptr;
        target_ = nullptr;
        own_draft_.reset();
        own_target_.reset();
        vocab_.clear();
        model_bytes_ = 0;
        model_path_.clear();
    }
    static ulspec_sampling sampling_(const GenerationConfig& c)
    {
        if (c.frequency_penalty != 0.0f || c.presence_penalty != 0.0f)
            throw Error(ULSPEC_EUNSUPPORTED, "frequency / presence penalties are not implemented");
        ulspec_sampling s{1.0f, 0, 1.0f, 1};
        if (c.do_sample) s = ulspec_sampling{c.temperature, c.top_k, c.top_p, 0};
        return s;
    }
    // The loop one step at a time for the streaming entry points (the lock is
    // held throughout, as the reference holds api_mutex_); on(text of the
    // token, tokens so far, seconds) per committed token, up to max_tokens.
    std::string stream_(const std::string& prompt, const GenerationConfig& config,
                        const std::function<void(const std::string&, uint32_t, float)>& on)
    {
        std::lock_guard<std::mutex> lock(mu_);
        if (!target_) return "Error: No model loaded";
        if (!tokenizer_) throw Error(ULSPEC_EUNSUPPORTED, "text prompts need register_custom_tokenizer()");
        const std::vector<uint32_t> ids = tokenizer_(prompt);
        const bool spec = spec_ && draft_;
        SpeculativeDecoder dec(target_->cfg().vocab, spec ? k_ : 0, 0.0f);
        dec.attach(*target_, spec ? draft_ : nullptr, sampling_(config), seed_);
        const auto t0 = std::chrono::steady_clock::now();
        dec.prefill(ids);
        std::string text;
        uint32_t done = 0;
        while (done < config.max_tokens) {
            for (uint32_t t : dec.step_tokens()) {
                if (done == config.max_tokens) break;
                ++done;
                const std::string piece = token_text({t});
                text += piece;
                on(piece, done, std::chrono::duration<float>(std::chrono::steady_clock::now() - t0).count());
            }
        }
        const float sec = std::chrono::duration<float>(std::chrono::steady_clock::now() - t0).count();
        throughput_ = sec > 0.0f ? (float)done / sec : 0.0f;
        if (spec) {
            accepted_ += dec.accepted();
            proposed_ += dec.proposed();
        }
        return text;
    }
    std::vector<uint32_t> run_(const std::vector<uint32_t>& prompt, uint32_t max_tokens, const ulspec_sampling& s)
    {
        if (!target_) throw Error(ULSPEC_EINVAL, "no model loaded");
        const bool spec = spec_ && draft_;
        SpeculativeDecoder dec(target_->cfg().vocab, spec ? k_ : 0, 0.0f);
        dec.attach(*target_, spec ? draft_ : nullptr, s, seed_);
        dec.prefill(prompt);
        std::vector<uint32_t> out = dec.generate(max_tokens);
        if (out.size() > max_tokens) out.resize(max_tokens);
        if (spec) {
            accepted_ += dec.accepted();
            proposed_ += dec.proposed();
        }
        return out;
    }

    Context* ctx_ = nullptr;
    uint32_t max_ctx_ = 0;
    Model* target_ = nullptr;
    Model* draft_ = nullptr;
    std::unique_ptr<Model> own_target_, own_draft_;
    std::vector<std::string> vocab_;
    uint64_t model_bytes_ = 0;
    std::string model_path_, err_;
    ulspec_sampling s_{1.0f, 0, 1.0f, 0};
    GenerationConfig config_;
    std::function<std::vector<uint32_t>(const std::string&)> tokenizer_;
    uint32_t k_;
    uint64_t seed_;
    bool spec_ = false;
    uint64_t accepted_ = 0, proposed_ = 0;
    float throughput_ = 0.0f;
    mutable std::mutex mu_;
};

}  // namespace ulspec_inference
