"""The speculative-decoding subset of the reference's Python module
`vulkangguf` (pybind11, src/api/inference_api.cpp:389-473), over the gfx950
library: same class and method names, argument meaning and result types.

    api = InferenceAPI()
    api.load_model("target.gguf")            # InferenceAPI::load_model (:21-43)
    api.load_draft_model("draft.gguf")       # no counterpart: the reference has no draft model
    api.enable_speculative_decoding(True)    # :214-216 (a no-op there)
    res = api.generate_tokens(prompt_ids, GenerationConfig(max_tokens=64))
    texts = api.generate_batch(prompts)      # :164-175 (a loop of generate there; the batched loop here)
    api.generate_streaming(p, cfg, print)    # :96-125, token texts as they are committed
    api.get_acceptance_rate()                # :222-225 (0.0 there; live here)
    api.get_token_logits(ids)                # :277-280 (empty there; live here)

Token ids in, token ids out.  Text goes through a tokenizer registered with
register_custom_tokenizer (:368-370); output text joins the GGUF vocabulary
strings (tokenizer.ggml.tokens, "▁" read as a space).  Every model call
runs the HIP kernels of lib/libulspec.so; without a gfx950 device the calls
raise (no CPU path).  Methods of the reference outside this path (adapters,
multi-GPU, pipeline caches, quantization switches) are not provided.
"""
import threading
import time
from dataclasses import dataclass, field

import numpy as np

from . import (EUNSUPPORTED, GGUFFile, Speculative, UlspecError, load_gguf_model, sampling)


@dataclass
class GenerationConfig:
    """py::GenerationConfig (src/api/inference_api.h:14-22); defaults of the
    InferenceAPI constructor (inference_api.cpp:8-16)."""
    max_tokens: int = 100
    temperature: float = 1.0
    top_p: float = 0.9
    top_k: int = 40
    frequency_penalty: float = 0.0
    presence_penalty: float = 0.0
    do_sample: bool = True


@dataclass
class GenerationResult:
    """py::GenerationResult (inference_api.h:24-30)."""
    tokens: list = field(default_factory=list)
    text: str = ""
    num_tokens: int = 0
    time_ms: float = 0.0
    tokens_per_second: float = 0.0


@dataclass
class GenerationProgress:
    """py::GenerationProgress (inference_api.h:32-40)."""
    current_step: int = 0
    total_steps: int = 0
    progress_pct: float = 0.0
    time_elapsed_ms: float = 0.0
    estimated_remaining_ms: float = 0.0
    tokens_per_second: float = 0.0
    last_token: str = ""


@dataclass
class ModelMetrics:
    """py::ModelMetrics (inference_api.h:42-50)."""
    vocab_size: int = 0
    num_layers: int = 0
    hidden_dim: int = 0
    context_len: int = 0
    num_heads: int = 0
    model_size_bytes: int = 0
    architecture: str = ""


class InferenceAPI:
    """py::InferenceAPI (inference_api.h:52-123), speculative-decoding subset.
    Every public method holds one lock, as the reference's api_mutex_."""

    SPEC_LENGTH = 5  # drafts per step (k)

    def __init__(self, ctx=None, max_ctx=0, seed=0):
        from . import Context
        self._ctx = ctx if ctx is not None else Context(0)
        self._max_ctx = max_ctx
        self._seed = seed
        self._lock = threading.RLock()
        self._config = GenerationConfig()
        self._target = self._draft = None
        self._batch = None  # (target, draft) with MAX_BATCH sequence slots, for generate_batch
        self._vocab = None
        self._model_path = self._draft_path = ""
        self._model_bytes = 0
        self._spec = False
        self._tokenizer = None
        self._accepted = self._proposed = 0
        self._throughput = 0.0

    # -- models ---------------------------------------------------------------
    def load_model(self, model_path):
        """Target model from a GGUF file (InferenceAPI::load_model, :21-43)."""
        with self._lock:
            self.unload_model()
            with GGUFFile(model_path) as g:
                self._target = load_gguf_model(self._ctx, g, self._max_ctx)
                self._model_bytes = sum(t.nbytes for t in g.tensors())
                try:
                    self._vocab = self._read_vocab(g)
                except UlspecError:
                    self._vocab = None
            self._model_path = model_path
            return True

    def load_draft_model(self, model_path):
        """Draft model for speculative decoding (same vocabulary as the target)."""
        with self._lock:
            if self._target is None:
                raise UlspecError(EUNSUPPORTED, "load the target model first")
            d = load_gguf_model(self._ctx, model_path, self._max_ctx)
            if d.cfg.vocab != self._target.cfg.vocab:
                d.close()
                raise ValueError("draft and target vocabularies differ")
            if self._draft is not None:
                self._draft.close()
            self._drop_batch()
            self._draft, self._draft_path = d, model_path
            return True

    def unload_model(self):
        with self._lock:
            self._drop_batch()
            for m in (self._draft, self._target):
                if m is not None:
                    m.close()
            self._target = self._draft = None
            self._model_path, self._draft_path, self._vocab, self._model_bytes = "", "", None, 0
            return True

    def _drop_batch(self):
        for m in self._batch or ():
            if m is not None:
                m.close()
        self._batch = None

    def _batch_models(self, spec):
        """One target (and draft) model pair with MAX_BATCH sequence slots,
        loaded from the same files on first use (a second copy of the weights)
        and kept; every group of 2 .. MAX_BATCH prompts runs on it (a loop of
        B sequences uses slots 0 .. B - 1).  The draft is added when a later
        call first needs it."""
        if self._batch is None:
            t = load_gguf_model(self._ctx, self._model_path, self._max_ctx, n_seq=self.MAX_BATCH)
            self._batch = (t, None)
        if spec and self._batch[1] is None:
            d = load_gguf_model(self._ctx, self._draft_path, self._max_ctx, n_seq=self.MAX_BATCH)
            self._batch = (self._batch[0], d)
        return self._batch

    @staticmethod
    def _read_vocab(g):
        return g.get_str_array("tokenizer.ggml.tokens")

    # -- configuration -------------------------------------------------------
    def enable_speculative_decoding(self, enable):
        with self._lock:
            self._spec = bool(enable)

    def set_temperature(self, temp):
        with self._lock:
            self._config.temperature = float(temp)

    def set_top_p(self, top_p):
        with self._lock:
            self._config.top_p = float(top_p)

    def set_top_k(self, top_k):
        with self._lock:
            self._config.top_k = int(top_k)

    def enable_gpu(self, enable):
        """The path runs on the GPU only: enabling succeeds, disabling does not."""
        return bool(enable)

    def is_gpu_enabled(self):
        return True

    def register_custom_tokenizer(self, tokenizer_func):
        """str -> list of token ids, used by generate() for text prompts (:368-370)."""
        with self._lock:
            self._tokenizer = tokenizer_func

    # -- queries ---------------------------------------------------------------
    def get_acceptance_rate(self):
        """Cumulative accepted / proposed drafts; 0.5 before any speculative
        step (SpeculativeDecoder's initial value, speculative_decoder.cpp:10)."""
        with self._lock:
            return self._accepted / self._proposed if self._proposed else 0.5

    def get_throughput(self):
        with self._lock:
            return self._throughput

    def get_model_info(self):
        with self._lock:
            if self._target is None:
                return ModelMetrics()
            c = self._target.cfg
            return ModelMetrics(c.vocab, c.n_layers, c.dim, c.max_ctx, c.n_heads, self._model_bytes, "llama")

    def get_model_architecture(self):
        with self._lock:
            return "llama" if self._target is not None else ""

    def get_token_logits(self, tokens):
        """Target logits after `tokens` (positions 0..len-1), as a list of
        floats (InferenceAPI::get_token_logits, :277-280)."""
        with self._lock:
            if self._target is None:
                return []
            return self._target.forward(np.asarray(tokens, np.int32), 0, n_logits=1)[0].tolist()

    # -- generation ------------------------------------------------------------
    def _sampling(self, config):
        if config.frequency_penalty or config.presence_penalty:
            raise UlspecError(EUNSUPPORTED, "frequency / presence penalties are not implemented")
        if not config.do_sample:
            return sampling(greedy=True)
        return sampling(temperature=config.temperature, top_k=config.top_k, top_p=config.top_p)

    def generate_tokens(self, prompt_ids, config=None):
        """max_tokens new token ids after prompt_ids: speculative steps with the
        draft model when enabled, otherwise plain decoding of the target (the
        device loop with k = 0: one target row and one draw per token)."""
        with self._lock:
            if self._target is None:
                raise UlspecError(EUNSUPPORTED, "no model loaded")
            config = config or self._config
            s = self._sampling(config)
            spec = self._spec and self._draft is not None
            k = self.SPEC_LENGTH if spec else 0
            loop = Speculative(self._target, self._draft if spec else None, k, s, self._seed)
            try:
                t0 = time.perf_counter()
                loop.prefill(np.asarray(prompt_ids, np.int32))
                n0 = loop.state()["n"]
                loop.generate(int(config.max_tokens))
                st = loop.state()
                toks = loop.tokens(n0, min(int(config.max_tokens), st["n"] - n0)).tolist()
                dt = time.perf_counter() - t0
            finally:
                loop.close()
            if spec:
                self._accepted += st["accepted"]
                self._proposed += st["proposed"]
            self._throughput = len(toks) / dt if dt > 0 else 0.0
            return GenerationResult(toks, self.token_text(toks), len(toks), dt * 1e3, self._throughput)

    def _stream(self, prompt, config, on_token):
        """The device loop one step at a time (a host fence per step): on_token
        (token id, text, tokens so far, seconds) for each committed token, up
        to max_tokens.  Returns the generated text."""
        config = config or self._config
        s = self._sampling(config)
        spec = self._spec and self._draft is not None
        loop = Speculative(self._target, self._draft if spec else None, self.SPEC_LENGTH if spec else 0, s,
                           self._seed)
        want, done, text = int(config.max_tokens), 0, ""
        try:
            t0 = time.perf_counter()
            loop.prefill(np.asarray(self._tokenize(prompt), np.int32))
            st = loop.state()
            n = st["n"]
            while done < want:
                loop.steps(1)
                st = loop.state()
                for t in loop.tokens(n, st["n"] - n).tolist()[:want - done]:
                    done += 1
                    piece = self.token_text([t])
                    text += piece
                    on_token(t, piece, done, time.perf_counter() - t0)
                n = st["n"]
            dt = time.perf_counter() - t0
        finally:
            loop.close()
        if spec:
            self._accepted += st["accepted"]
            self._proposed += st["proposed"]
        self._throughput = done / dt if dt > 0 else 0.0
        return text

    def generate_streaming(self, prompt, config, token_callback):
        """InferenceAPI::generate_streaming (inference_api.cpp:96-125): the
        callback gets each new token's text as it is committed; returns the
        whole text ("Error: No model loaded" without a model)."""
        with self._lock:
            if self._target is None:
                return "Error: No model loaded"
            return self._stream(prompt, config,
                                lambda t, piece, done, sec: token_callback(piece) if token_callback else None)

    def generate_with_progress(self, prompt, config, progress_callback):
        """InferenceAPI::generate_with_progress (inference_api.cpp:127-162): a
        GenerationProgress after each committed token.  Returns the generated
        text (the reference returns an empty string: its result is never
        filled)."""
        with self._lock:
            if self._target is None:
                return "Error: No model loaded"
            config = config or self._config
            total = int(config.max_tokens)

            def on_token(t, piece, done, sec):
                if progress_callback is None:
                    return
                rate = done / sec if sec > 0 else 0.0
                progress_callback(GenerationProgress(done, total, 100.0 * done / total if total else 100.0,
                                                     sec * 1e3, (total - done) / rate * 1e3 if rate > 0 else 0.0,
                                                     rate, piece))
            return self._stream(prompt, config, on_token)

    MAX_BATCH = 8  # sequences per batched loop (ulspec_model_create_batch)

    def generate_tokens_batch(self, prompts, config=None):
        """A GenerationResult per prompt (token ids in), the prompts stepped
        together in groups of up to MAX_BATCH sequences on the batched device
        loop: one verify forward of (k + 1) rows per sequence per step
        (speculative when enabled with a draft model, else target-only
        decoding).  Greedy results equal generate_tokens() prompt by prompt;
        sampled ones draw from the batch's uniform stream (sequence b of step
        s: u(seed, (s B + b)(2k + 1) + j)), not the one-prompt stream.
        time_ms and tokens_per_second are those of the prompt's group."""
        with self._lock:
            if self._target is None:
                raise UlspecError(EUNSUPPORTED, "no model loaded")
            config = config or self._config
            s = self._sampling(config)
            spec = self._spec and self._draft is not None
            k = self.SPEC_LENGTH if spec else 0
            want = int(config.max_tokens)
            results, n_tok, t_all = [], 0, 0.0
            for g0 in range(0, len(prompts), self.MAX_BATCH):
                group = [np.asarray(p, np.int32) for p in prompts[g0:g0 + self.MAX_BATCH]]
                if len(group) == 1:
                    results.append(self.generate_tokens(group[0], config))
                    n_tok += results[-1].num_tokens
                    t_all += results[-1].time_ms * 1e-3
                    continue
                tgt, dft = self._batch_models(spec)
                loop = Speculative(tgt, dft if spec else None, k, s, self._seed, n_seq=len(group))
                try:
                    t0 = time.perf_counter()
                    loop.prefill(group)
                    n0 = [loop.seq_state(b)["n"] for b in range(len(group))]
                    loop.generate(want)
                    dt = time.perf_counter() - t0
                    for b in range(len(group)):
                        st = loop.seq_state(b)
                        toks = loop.tokens(n0[b], min(want, st["n"] - n0[b]), seq=b).tolist()
                        results.append(GenerationResult(toks, self.token_text(toks), len(toks), dt * 1e3,
                                                        len(toks) / dt if dt > 0 else 0.0))
                        n_tok += len(toks)
                        if spec:
                            self._accepted += st["accepted"]
                            self._proposed += st["proposed"]
                    t_all += dt
                finally:
                    loop.close()
            self._throughput = n_tok / t_all if t_all > 0 else 0.0
            return results

    def generate_batch(self, prompts, config=None):
        """InferenceAPI::generate_batch (inference_api.cpp:164-175): an output
        text per prompt (text through the registered tokenizer, or token ids),
        "Error: No model loaded" for each without a model; the prompts run
        together on the batched loop (generate_tokens_batch)."""
        with self._lock:
            if self._target is None:
                return ["Error: No model loaded" for _ in prompts]
            ids = [self._tokenize(p) for p in prompts]
            return [r.text for r in self.generate_tokens_batch(ids, config)]

    def _tokenize(self, prompt):
        if isinstance(prompt, str):
            if self._tokenizer is None:
                raise UlspecError(EUNSUPPORTED, "text prompts need register_custom_tokenizer()")
            return self._tokenizer(prompt)
        return prompt

    def generate(self, prompt, config=None):
        """Text (with a registered tokenizer) or token ids in, text out
        (InferenceAPI::generate, :45-63, including its error string)."""
        with self._lock:
            if self._target is None:
                return "Error: No model loaded"
            return self.generate_tokens(self._tokenize(prompt), config).text

    def generate_default(self, prompt):
        """generate() with the API's own configuration (:65-77)."""
        with self._lock:
            return self.generate_tokens(self._tokenize(prompt), self._config)

    def token_text(self, tokens):
        """Decoded text when the GGUF vocabulary covers the ids, else the ids."""
        if self._vocab is None or any(t >= len(self._vocab) for t in tokens):
            return " ".join(str(t) for t in tokens)
        return "".join(self._vocab[t] for t in tokens).replace("\u2581", " ")
