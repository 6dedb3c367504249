// Drives the C++ host classes of include/ulspec_inference.hpp on a small
// random model: greedy speculative generation must equal greedy plain
// decoding (speculation off; both are the target's argmax chain), the
// acceptance rate starts at 0.5, a step reports n_accepted + 1 committed
// tokens, and the reference's generate_with_speculation(context_token, n)
// shape, started from one token, follows the argmax chain.  With two GGUF
// paths (target, draft; vocabulary strings "▁w<i>") it also loads them
// through InferenceAPI::load_model / load_draft_model and generates text.
// Prints "OK" and exits 0 on success.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "ulspec_inference.hpp"

using namespace ulspec_inference;

static uint64_t mix(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

// Q4_0 rows with pseudo-random nibbles and a fixed scale of 1/64.
static std::vector<uint8_t> q4_0(uint64_t seed, uint64_t rows, uint64_t k)
{
    std::vector<uint8_t> b(rows * (k / 32) * 18);
    for (size_t i = 0; i < b.size(); i += 18) {
        b[i] = 0x00;
        b[i + 1] = 0x24;  // fp16 0x2400 = 1/64
        for (int j = 0; j < 16; ++j) b[i + 2 + j] = (uint8_t)mix(seed * 0x9e3779b97f4a7c15ull + i + j);
    }
    return b;
}

static void load(Model& m, uint64_t seed)
{
    const ulspec_model_cfg& c = m.cfg();
    const uint64_t D = c.dim / c.n_heads;
    auto put = [&](const std::string& name, uint64_t ne0, uint64_t ne1) {
        std::vector<uint8_t> b = q4_0(seed++, ne1, ne0);
        m.set_tensor(name, ULSPEC_GGML_Q4_0, b.data(), b.size(), ne0, ne1);
    };
    std::vector<float> ones(c.dim, 1.0f);
    put("token_embd.weight", c.dim, c.vocab);
    put("output.weight", c.dim, c.vocab);
    m.set_tensor("output_norm.weight", 0, ones.data(), ones.size() * 4, c.dim, 1);
    for (uint32_t l = 0; l < c.n_layers; ++l) {
        const std::string p = "blk." + std::to_string(l) + ".";
        put(p + "attn_q.weight", c.dim, c.n_heads * D);
        put(p + "attn_k.weight", c.dim, c.n_kv_heads * D);
        put(p + "attn_v.weight", c.dim, c.n_kv_heads * D);
        put(p + "attn_output.weight", c.n_heads * D, c.dim);
        put(p + "ffn_gate.weight", c.dim, c.ffn);
        put(p + "ffn_up.weight", c.dim, c.ffn);
        put(p + "ffn_down.weight", c.ffn, c.dim);
        m.set_tensor(p + "attn_norm.weight", 0, ones.data(), ones.size() * 4, c.dim, 1);
        m.set_tensor(p + "ffn_norm.weight", 0, ones.data(), ones.size() * 4, c.dim, 1);
    }
}

// The target's greedy continuation of seq by n tokens (full re-forward each token).
static std::vector<uint32_t> argmax_chain(Model& m, std::vector<uint32_t> seq, size_t n)
{
    for (size_t i = 0; i < n; ++i) {
        std::vector<float> lg = m.token_logits(seq);
        seq.push_back((uint32_t)(std::max_element(lg.begin(), lg.end()) - lg.begin()));
    }
    return seq;
}

static int files_part(Context& ctx, const char* target_path, const char* draft_path)
{
    InferenceAPI api(ctx, 128, 4, 3);
    if (api.generate("w1", GenerationConfig{}) != "Error: No model loaded") {
        std::printf("no-model message\n");
        return 1;
    }
    if (api.load_model("/nonexistent/model.gguf") || api.last_error().empty()) {
        std::printf("load_model of a missing file\n");
        return 1;
    }
    if (!api.load_model(target_path) || !api.load_draft_model(draft_path)) {
        std::printf("load_model: %s\n", api.last_error().c_str());
        return 1;
    }
    api.register_custom_tokenizer([](const std::string& text) {
        std::vector<uint32_t> ids;
        for (size_t i = 0; (i = text.find('w', i)) != std::string::npos; ++i) ids.push_back((uint32_t)std::atoi(&text[i + 1]));
        return ids;
    });
    GenerationConfig c;
    c.max_tokens = 16;
    c.do_sample = false;
    api.enable_speculative_decoding(true);
    const std::string spec = api.generate("w1 w2 w3 w4", c);
    api.enable_speculative_decoding(false);
    const std::string plain = api.generate("w1 w2 w3 w4", c);
    GenerationResult r = api.generate_tokens(std::vector<uint32_t>{1, 2, 3, 4}, c);
    if (spec != plain || r.text != plain || r.num_tokens != 16 || std::count(plain.begin(), plain.end(), ' ') != 16) {
        std::printf("text generation: '%s' vs '%s'\n", spec.c_str(), plain.c_str());
        return 1;
    }
    const std::vector<std::string> batch = api.generate_batch({"w1 w2 w3 w4", "w5 w6"}, c);
    if (batch.size() != 2 || batch[0] != plain || batch[1] != api.generate("w5 w6", c)) {
        std::printf("generate_batch\n");
        return 1;
    }
    for (bool sp : {true, false}) {
        api.enable_speculative_decoding(sp);
        std::string pieces;
        uint32_t calls = 0, last_step = 0;
        const std::string streamed = api.generate_streaming("w1 w2 w3 w4", c, [&](const std::string& t) {
            pieces += t;
            ++calls;
        });
        const std::string progressed = api.generate_with_progress("w1 w2 w3 w4", c, [&](const GenerationProgress& p) {
            last_step = p.current_step;
        });
        if (streamed != plain || pieces != plain || calls != 16 || progressed != plain || last_step != 16) {
            std::printf("streaming: '%s' (%u calls), progress %u\n", streamed.c_str(), calls, last_step);
            return 1;
        }
    }
    const float rate = api.get_acceptance_rate();
    if (!(rate >= 0.0f && rate <= 1.0f)) {
        std::printf("acceptance rate %f\n", rate);
        return 1;
    }
    return 0;
}

int main(int argc, char** argv)
{
    try {
        Context ctx(0);
        ulspec_model_cfg tc{256, 2, 4, 4, 512, 1000, 160, 1e-5f, 10000.0f};
        ulspec_model_cfg dc = tc;
        dc.n_layers = 1;
        Model target(ctx, tc), draft(ctx, dc);
        load(target, 100);
        load(draft, 900);
        std::vector<uint32_t> prompt;
        for (uint32_t i = 0; i < 20; ++i) prompt.push_back((uint32_t)(mix(i) % tc.vocab));

        InferenceAPI api(target, draft, 4, 7);
        if (api.get_acceptance_rate() != 0.5f) { std::printf("initial rate\n"); return 1; }
        api.set_greedy(true);
        api.enable_speculative_decoding(true);
        std::vector<uint32_t> spec = api.generate_tokens(prompt, 40);
        api.enable_speculative_decoding(false);
        std::vector<uint32_t> plain = api.generate_tokens(prompt, 40);
        if (spec.size() != 40 || spec != plain) { std::printf("greedy speculative != greedy\n"); return 1; }
        std::vector<float> lg = api.get_token_logits(prompt);
        if (lg.size() != tc.vocab) { std::printf("logits size\n"); return 1; }

        SpeculativeDecoder dec(tc.vocab, 3, 0.0f);
        ulspec_sampling s{0.8f, 0, 1.0f, 0};
        dec.attach(target, draft, s, 11);
        dec.prefill(prompt);
        SpeculationResult r = dec.generate_with_speculation();
        if (r.accepted_tokens.size() != r.num_accepted + 1 || r.rejected_tokens.size() != 3 - r.num_accepted) {
            std::printf("step result sizes\n");
            return 1;
        }
        // the reference's call shape from a single context token: a plain
        // first step, then speculative steps on the committed sequence
        SpeculativeDecoder d2(tc.vocab, 3, 0.0f);
        d2.attach(target, draft, ulspec_sampling{1.0f, 0, 1.0f, 1}, 5);
        SpeculationResult a = d2.generate_with_speculation(prompt[0], 4);
        if (a.accepted_tokens.size() != 1 || a.num_accepted != 0 || !a.rejected_tokens.empty()) {
            std::printf("first step from one token\n");
            return 1;
        }
        std::vector<uint32_t> chain{prompt[0], a.accepted_tokens[0]};
        for (int i = 0; i < 6; ++i) {
            SpeculationResult b = d2.generate_with_speculation(chain.back());
            if (b.accepted_tokens.size() != b.num_accepted + 1) {
                std::printf("overload step sizes\n");
                return 1;
            }
            chain.insert(chain.end(), b.accepted_tokens.begin(), b.accepted_tokens.end());
        }
        if (chain != argmax_chain(target, {prompt[0]}, chain.size() - 1)) {
            std::printf("overload chain != argmax chain\n");
            return 1;
        }
        if (argc >= 3 && files_part(ctx, argv[1], argv[2])) return 1;
        std::printf("OK rate %.3f\n", dec.get_acceptance_rate());
        return 0;
    } catch (const Error& e) {
        std::printf("error %d: %s\n", (int)e.status, e.what());
        return 1;
    }
}
