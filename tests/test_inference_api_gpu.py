"""The vulkangguf-compatible InferenceAPI (universal-loader_amd/inference_api.py)
over GGUF files: token-level generation with and without the draft model,
live acceptance rate and logits."""
import importlib

import numpy as np
import pytest

import gguf_io as G
from llama_util import make_tensors

pytestmark = pytest.mark.gpu

CFG = dict(dim=256, n_layers=2, n_heads=4, n_kv_heads=4, ffn=512, vocab=1000, max_ctx=128, rms_eps=1e-5,
           rope_base=10000.0)


@pytest.fixture(scope="module")
def files(ora, tmp_path_factory):
    d = tmp_path_factory.mktemp("api")
    out = []
    for name, seed, layers in (("target", 31, 2), ("draft", 32, 1)):
        cfg = dict(CFG, n_layers=layers)
        kv = G.llama_kv(cfg)
        kv = [e if e[0] != "tokenizer.ggml.tokens" else
              ("tokenizer.ggml.tokens", G.ARRAY, (G.STRING, [f"▁w{i}" for i in range(CFG["vocab"])])) for e in kv]
        p = d / f"{name}.gguf"
        G.write(p, kv, G.model_tensors(make_tensors(ora, cfg, 12, seed=seed)))
        out.append(str(p))
    return out


@pytest.fixture(scope="module")
def api_mod(pkg):
    return importlib.import_module(pkg.__name__ + ".inference_api")


def test_greedy_generation_with_and_without_speculation(pkg, ctx, api_mod, files):
    target, draft = files
    api = api_mod.InferenceAPI(ctx=ctx, seed=7)
    assert api.generate([1, 2, 3]) == "Error: No model loaded"
    assert api.load_model(target) and api.load_draft_model(draft)
    info = api.get_model_info()
    assert (info.vocab_size, info.num_layers, info.hidden_dim, info.context_len, info.architecture) == \
        (1000, 2, 256, 128, "llama")
    prompt = list(np.random.default_rng(4).integers(0, 1000, 10))
    cfg = api_mod.GenerationConfig(max_tokens=20, do_sample=False)
    assert api.get_acceptance_rate() == 0.5
    plain = api.generate_tokens(prompt, cfg)
    api.enable_speculative_decoding(True)
    spec = api.generate_tokens(prompt, cfg)
    assert plain.tokens == spec.tokens and spec.num_tokens == 20
    assert 0.0 <= api.get_acceptance_rate() <= 1.0 and api.get_throughput() > 0
    # greedy = argmax chain of the target's own logits
    seq = list(prompt)
    for _ in range(4):
        seq.append(int(np.argmax(api.get_token_logits(seq))))
    assert seq[len(prompt):] == spec.tokens[:4]
    assert spec.text == "".join(f" w{t}" for t in spec.tokens)
    api.register_custom_tokenizer(lambda s: [int(x) for x in s.split()])
    assert api.generate(" ".join(str(t) for t in prompt), cfg) == spec.text
    api.unload_model()
    assert api.get_model_architecture() == ""


def test_sampled_generation_is_seeded(pkg, ctx, api_mod, files):
    target, draft = files
    res = []
    for _ in range(2):
        api = api_mod.InferenceAPI(ctx=ctx, seed=99)
        api.load_model(target)
        api.load_draft_model(draft)
        api.enable_speculative_decoding(True)
        api.set_temperature(0.8)
        api.set_top_k(40)
        api.set_top_p(0.9)
        res.append(api.generate_default([5, 6, 7, 8]).tokens)
        api.unload_model()
    assert res[0] == res[1] and len(res[0]) == 100


def test_generate_batch(pkg, ctx, api_mod, files):
    """generate_batch: the prompts stepped together on the batched loop (groups
    of up to 8 sequences), greedy outputs equal to one-prompt generation, with
    and without speculation; text prompts through the tokenizer; the
    reference's no-model string per prompt."""
    target, draft = files
    api = api_mod.InferenceAPI(ctx=ctx, seed=5)
    assert api.generate_batch(["1 2", "3 4"]) == ["Error: No model loaded"] * 2
    api.load_model(target)
    api.load_draft_model(draft)
    rng = np.random.default_rng(12)
    prompts = [list(rng.integers(0, 1000, n)) for n in (9, 4, 17, 6, 12, 3, 8, 15, 5, 11)]
    cfg = api_mod.GenerationConfig(max_tokens=12, do_sample=False)
    pair = None
    for spec in (True, False):
        api.enable_speculative_decoding(spec)
        one = [api.generate_tokens(p, cfg).tokens for p in prompts]
        batch = api.generate_tokens_batch(prompts, cfg)  # a group of 8, then one of 2
        assert [r.tokens for r in batch] == one, spec
        assert all(r.num_tokens == 12 for r in batch) and api.get_throughput() > 0
        pair = pair or api._batch
    api.register_custom_tokenizer(lambda s: [int(x) for x in s.split()])
    texts = api.generate_batch([" ".join(str(t) for t in p) for p in prompts[:3]], cfg)
    assert texts == [api.generate_tokens(p, cfg).text for p in prompts[:3]]
    # groups of 8, 2 and 3 sequences all ran on one target / draft pair of 8-slot models
    assert api._batch is pair and all(m.n_seq == api.MAX_BATCH for m in pair)
    api.unload_model()
    assert api._batch is None


def test_streaming_and_progress(pkg, ctx, api_mod, files):
    """generate_streaming / generate_with_progress: one callback per committed
    token, in order, the texts joining to generate()'s output."""
    target, draft = files
    api = api_mod.InferenceAPI(ctx=ctx, seed=5)
    assert api.generate_streaming([1, 2], None, print) == "Error: No model loaded"
    api.load_model(target)
    api.load_draft_model(draft)
    cfg = api_mod.GenerationConfig(max_tokens=14, do_sample=False)
    prompt = [3, 1, 4, 1, 5, 9]
    for spec in (True, False):
        api.enable_speculative_decoding(spec)
        want = api.generate_tokens(prompt, cfg)
        pieces, prog = [], []
        assert api.generate_streaming(prompt, cfg, pieces.append) == want.text
        assert pieces == [api.token_text([t]) for t in want.tokens]
        assert api.generate_with_progress(prompt, cfg, prog.append) == want.text
        assert [p.current_step for p in prog] == list(range(1, 15)) and prog[-1].progress_pct == 100.0
        assert [p.last_token for p in prog] == pieces and all(p.total_steps == 14 for p in prog)
    api.unload_model()
