"""InferenceAPI configuration types (no device)."""
import importlib


def test_generation_config_defaults_match_the_reference(pkg):
    m = importlib.import_module(pkg.__name__ + ".inference_api")
    c = m.GenerationConfig()
    # InferenceAPI::InferenceAPI (src/api/inference_api.cpp:8-16)
    assert (c.max_tokens, c.temperature, c.top_p, c.top_k, c.frequency_penalty, c.presence_penalty, c.do_sample) == \
        (100, 1.0, 0.9, 40, 0.0, 0.0, True)
    r = m.GenerationResult()
    assert (r.tokens, r.text, r.num_tokens) == ([], "", 0)
