"""The oracle's Llama forward and speculative loop, pinned on the CPU:
  - against an independent float64 numpy forward (same fp16 rounding points),
    so a wrong RoPE pairing / sign, a transposed weight, a missing residual or
    a misplaced norm fails;
  - batching: a forward of M tokens equals M single-token forwards bitwise;
  - greedy speculative decoding emits exactly the target's autoregressive
    argmax sequence (the defining property of the greedy rule);
  - with the draft equal to the target, every draft token is accepted
    (p == q makes u * q(x) < p(x) hold for every u < 1).
"""
import numpy as np
import pytest

from llama_util import NumpyLlama, load, make_tensors

TOL = 2e-3
TINY = dict(dim=128, n_layers=2, n_heads=2, n_kv_heads=1, ffn=96, vocab=300, max_ctx=96, rms_eps=1e-5,
            rope_base=10000.0)


def _oracle(ora, cfg, tensors):
    m = ora.Llama(**cfg, nthreads=4)
    load(m, tensors)
    return m


@pytest.mark.parametrize("wtype", [2])
def test_forward_matches_numpy_float64(ora, wtype):
    t = make_tensors(ora, TINY, wtype, seed=11, std=0.05, norm_std=0.1)
    m = _oracle(ora, TINY, t)
    ref = NumpyLlama(ora, t, TINY)
    rng = np.random.default_rng(5)
    toks = rng.integers(0, TINY["vocab"], 9)
    lo = m.forward(toks[:6], 0, n_logits=6)
    lr = ref.forward(toks[:6], 0)
    # fp16 rounding points see float32 vs float64 inputs, so an fp16 element
    # now and then lands one ulp apart; that stays far below the tolerance
    scale = np.sqrt((lr ** 2).mean())
    assert np.abs(lo - lr).max() <= TOL * scale, np.abs(lo - lr).max() / scale
    lo2 = m.forward(toks[6:], 6, n_logits=3)  # continues on the cache
    lr2 = ref.forward(toks[6:], 6)
    assert np.abs(lo2 - lr2).max() <= TOL * scale
    _check_cache(ora, m, ref, 9)


def _check_cache(ora, m, ref, n, tol=TOL):
    for l in range(m.cfg.n_layers):
        k, v = m.kv_io(l, 0, 0, n)
        for got, want in ((k, ref.kc[l][:n]), (v, ref.vc[l][:n])):
            want = want.reshape(n, -1)
            err = np.abs(ora.h2f_fast(got).astype(np.float64) - want).max()
            assert err <= tol * np.sqrt((want ** 2).mean()), (l, err)


def test_forward_q4k_matches_numpy(ora):
    cfg = dict(TINY, dim=256, n_heads=4, n_kv_heads=4, ffn=512)
    t = make_tensors(ora, cfg, 12, seed=3, std=0.05, norm_std=0.1)
    m = _oracle(ora, cfg, t)
    ref = NumpyLlama(ora, t, cfg)
    toks = [5, 17, 250, 3]
    lo, lr = m.forward(toks, 0, n_logits=4), ref.forward(toks, 0)
    scale = np.sqrt((lr ** 2).mean())
    assert np.abs(lo - lr).max() <= TOL * scale
    _check_cache(ora, m, ref, 4)


def test_rope_mistake_is_caught(ora):
    """The cache check is sensitive: a different RoPE base moves the rotated
    keys far beyond the tolerance."""
    t = make_tensors(ora, TINY, 2, seed=11, std=0.05, norm_std=0.1)
    m = _oracle(ora, TINY, t)
    bad = NumpyLlama(ora, t, dict(TINY, rope_base=5000.0))
    toks = [1, 2, 3, 4, 5, 6]
    m.forward(toks, 0)
    bad.forward(toks, 0)
    with pytest.raises(AssertionError):
        _check_cache(ora, m, bad, 6, tol=20 * TOL)


def test_batched_forward_equals_single_token_forwards(ora):
    t = make_tensors(ora, TINY, 2, seed=2)
    a, b = _oracle(ora, TINY, t), _oracle(ora, TINY, t)
    toks = np.arange(10, 20)
    la = a.forward(toks, 0, n_logits=10)
    lb = np.concatenate([b.forward(toks[i:i + 1], i, n_logits=1) for i in range(10)])
    assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    for l in range(TINY["n_layers"]):
        ka, va = a.kv_io(l, 0, 0, 10)
        kb, vb = b.kv_io(l, 0, 0, 10)
        assert np.array_equal(ka, kb) and np.array_equal(va, vb)


def test_greedy_speculation_equals_target_argmax_chain(ora):
    cfg_t, cfg_d = TINY, dict(TINY, n_layers=1)
    tt, td = make_tensors(ora, cfg_t, 2, seed=21), make_tensors(ora, cfg_d, 2, seed=22)
    tgt, dft = _oracle(ora, cfg_t, tt), _oracle(ora, cfg_d, td)
    prompt = np.random.default_rng(3).integers(0, TINY["vocab"], 12).astype(np.int32)
    sp = ora.Speculative(tgt, dft, 3, ora.sampling(greedy=True), seed=9)
    sp.prefill(prompt)
    n = sp.generate(30)
    got = sp.tokens()
    # autoregressive greedy on a fresh copy of the target
    ref = _oracle(ora, cfg_t, tt)
    seq = list(prompt)
    ref.forward(np.array(seq[:-1], np.int32), 0)
    while len(seq) < len(got):
        lg = ref.forward(np.array(seq[-1:], np.int32), len(seq) - 1, n_logits=1)[0]
        seq.append(int(np.argmax(lg)))
    assert n >= 30 and list(got) == seq


def test_draft_equal_to_target_accepts_everything(ora):
    t = make_tensors(ora, TINY, 2, seed=31)
    tgt, dft = _oracle(ora, TINY, t), _oracle(ora, TINY, t)
    sp = ora.Speculative(tgt, dft, 4, ora.sampling(temperature=0.8), seed=4)
    sp.prefill(np.arange(8, dtype=np.int32))
    sp.generate(25)
    st = sp.state()
    assert st["accepted"] == st["proposed"] == 4 * st["steps"]
    assert st["n"] == 8 + 5 * st["steps"]
