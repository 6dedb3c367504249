// Drives the C++ host classes of include/ulspec_inference.hpp on a small
// random model: greedy speculative generation must equal greedy generation
// with k = 1 (both are the target's argmax chain), the acceptance rate starts
// at 0.5, and a step reports n_accepted + 1 committed tokens.
// Prints "OK" and exits 0 on success.
#include <cstdio>
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

int main()
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
        std::printf("OK rate %.3f\n", dec.get_acceptance_rate());
        return 0;
    } catch (const Error& e) {
        std::printf("error %d: %s\n", (int)e.status, e.what());
        return 1;
    }
}
