"""Batched speculative decoding on the GPU (B sequences at once: one group of
rows per sequence in every forward, a K/V cache slot per sequence, the
acceptance rule over B sequences) against the oracle, through the C ABI.

Bars:
  - the K/V a batch model writes for a sequence's prefill equal, bit for
    bit, a one-sequence model's on the same prompt;
  - greedy, free-running: every sequence's committed tokens and acceptance
    counters equal the oracle's own loop on that sequence's prompt;
  - temperature 0.8, full vocabulary and top-k 40 / top-p 0.9: every step's
    uniforms follow u(seed, (s B + b)(2k+1) + j), and every draft draw and
    accept decision of every sequence is bit-exact with the oracle's rule on
    the step's logits; the batched logits of each sequence agree with a
    one-sequence GPU model's for the same tokens within LOGIT_TOL of their
    RMS (batched rows take the split-K GEMM path and the cache rows of earlier
    batched steps, so fp32 order and some fp16 K/V roundings differ);
  - Q4_K, 8 sequences x 6 verify rows (48): every verify row's target logits
    within LOGIT_TOL_ORACLE of their RMS of the oracle's forward, and the
    greedy tokens equal to the oracle's loop.
"""
import numpy as np
import pytest

from llama_util import load, make_tensors

pytestmark = pytest.mark.gpu

TARGET = dict(dim=512, n_layers=8, n_heads=8, n_kv_heads=8, ffn=1376, vocab=32000, max_ctx=256, rms_eps=1e-5,
              rope_base=10000.0)
DRAFT = dict(TARGET, n_layers=2)
LOGIT_TOL = 2e-3


@pytest.fixture(scope="module")
def weights(ora):
    return make_tensors(ora, TARGET, 2, seed=101), make_tensors(ora, DRAFT, 2, seed=202)


@pytest.fixture(scope="module")
def prompts():
    rng = np.random.default_rng(91)
    return [rng.integers(0, 32000, n).astype(np.int32) for n in (20, 33, 47, 64, 9, 28, 51, 40)]


def _gpu(pkg, ctx, cfg, tensors, n_seq=1):
    m = pkg.Model(ctx, **cfg, n_seq=n_seq)
    load(m, tensors)
    return m


def _ora(ora, cfg, tensors):
    m = ora.Llama(**cfg, nthreads=ora.nthreads_default())
    load(m, tensors)
    return m


def test_batch_model_prefill_equals_single_sequence(pkg, ctx, weights, prompts):
    tw, _ = weights
    mb = _gpu(pkg, ctx, TARGET, tw, n_seq=4)
    m1 = _gpu(pkg, ctx, TARGET, tw)
    for b in range(4):
        p = prompts[b]
        lb = mb.forward(p, 0, n_logits=2, seq=b)
        l1 = m1.forward(p, 0, n_logits=2)
        assert np.array_equal(lb, l1), b
        for layer in (0, 7):
            kb, vb = mb.kv_io(layer, 0, 0, len(p), seq=b)
            k1, v1 = m1.kv_io(layer, 0, 0, len(p))
            assert np.array_equal(kb, k1) and np.array_equal(vb, v1), (b, layer)
    with pytest.raises(pkg.UlspecError) as e:
        mb.forward(prompts[0], 0, seq=4)
    assert e.value.status == pkg.EINVAL
    mb.close()
    m1.close()


@pytest.mark.parametrize("B,k", [(4, 4), (8, 5)])
def test_batch_greedy_tokens_bit_exact_with_oracle(pkg, ctx, ora, weights, prompts, B, k):
    tw, dw = weights
    gt, gd = _gpu(pkg, ctx, TARGET, tw, n_seq=B), _gpu(pkg, ctx, DRAFT, dw, n_seq=B)
    sp = pkg.Speculative(gt, gd, k, pkg.sampling(greedy=True), 7, n_seq=B)
    sp.prefill(prompts[:B])
    sp.generate(24)
    ot, od = _ora(ora, TARGET, tw), _ora(ora, DRAFT, dw)
    steps = sp.state()["steps"]
    for b in range(B):
        osp = ora.Speculative(ot, od, k, ora.sampling(greedy=True), 7)
        osp.prefill(prompts[b])
        for _ in range(steps):
            osp.step()
        got, want = sp.tokens(seq=b), osp.tokens()
        st = sp.seq_state(b)
        print(f"  B={B} seq {b}: {st['n'] - len(prompts[b])} tokens, accepted {st['accepted']}/{st['proposed']}")
        assert np.array_equal(got, want), b
        assert (st["n"], st["accepted"], st["proposed"]) == (osp.state()["n"], osp.state()["accepted"],
                                                             osp.state()["proposed"])
    for m in (sp, gt, gd, ot, od):
        m.close()


# Q4_K (256-element super-blocks: FFN 1536), 8 sequences x (k + 1) = 48 verify
# rows: the target's GEMMs take the split-K kernel at 6 column tiles of split
# X (the min term from X sub-block sums, low-part rows bank-offset in LDS)
TARGET_K = dict(TARGET, n_layers=4, ffn=1536)
DRAFT_K = dict(TARGET_K, n_layers=2)
Q4_K = 12
LOGIT_TOL_ORACLE = 1e-3  # measured 2.5e-4


def test_batch_q4_k_48_rows_against_oracle(pkg, ctx, ora, prompts):
    tw, dw = make_tensors(ora, TARGET_K, Q4_K, seed=303), make_tensors(ora, DRAFT_K, Q4_K, seed=404)
    B, k = 8, 5
    gt, gd = _gpu(pkg, ctx, TARGET_K, tw, n_seq=B), _gpu(pkg, ctx, DRAFT_K, dw, n_seq=B)
    sp = pkg.Speculative(gt, gd, k, pkg.sampling(greedy=True), 7, n_seq=B)
    sp.prefill(prompts[:B])
    ot, od = _ora(ora, TARGET_K, tw), _ora(ora, DRAFT_K, dw)
    seqs = [list(p) for p in prompts[:B]]
    worst = 0.0
    for step in range(3):
        ns = [len(q) for q in seqs]
        sp.steps(1)
        r = sp.last_step()
        for b in range(B):
            # every verify row's target logits against the oracle's forward
            n = ns[b]
            toks = np.concatenate([[seqs[b][n - 1]], r["draft_tokens"][b]]).astype(np.int32)
            ot.forward(np.array(seqs[b][:n - 1], np.int32), 0)
            want = ot.forward(toks, n - 1, n_logits=k + 1).astype(np.float64)
            err = float(np.abs(r["target_logits"][b].astype(np.float64) - want).max() /
                        np.sqrt((want ** 2).mean()))
            worst = max(worst, err)
            seqs[b] += list(r["out_tokens"][b][:r["n_accepted"][b] + 1])
    print(f"  Q4_K, 48 verify rows: target logits max err / rms vs the oracle {worst:.2e}")
    assert worst <= LOGIT_TOL_ORACLE
    # greedy tokens: each sequence equals the oracle's own loop on its prompt
    steps = sp.state()["steps"]
    for b in range(B):
        osp = ora.Speculative(ot, od, k, ora.sampling(greedy=True), 7)
        osp.prefill(prompts[b])
        for _ in range(steps):
            osp.step()
        assert np.array_equal(sp.tokens(seq=b), osp.tokens()), b
        assert np.array_equal(sp.tokens(seq=b), np.array(seqs[b], np.int32)), b
    for m in (sp, gt, gd, ot, od):
        m.close()


@pytest.mark.parametrize("mode", ["full", "topk_topp"])
def test_batch_sampling_steps_bit_exact_with_oracle(pkg, ctx, ora, weights, prompts, mode):
    tw, dw = weights
    B, k, seed = 4, 4, 2024
    args = dict(temperature=0.8) if mode == "full" else dict(temperature=0.8, top_k=40, top_p=0.9)
    s_gpu, s_ora = pkg.sampling(**args), ora.sampling(**args)
    gt, gd = _gpu(pkg, ctx, TARGET, tw, n_seq=B), _gpu(pkg, ctx, DRAFT, dw, n_seq=B)
    ref = _gpu(pkg, ctx, TARGET, tw)  # one-sequence model: the batched logits' reference
    sp = pkg.Speculative(gt, gd, k, s_gpu, seed, n_seq=B)
    sp.prefill(prompts[:B])
    seqs = [list(p) for p in prompts[:B]]
    worst = 0.0
    for step in range(6):
        ns = [len(q) for q in seqs]
        sp.steps(1)
        r = sp.last_step()
        for b in range(B):
            want_u = ora.uniforms(seed, (step * B + b) * (2 * k + 1), 2 * k + 1)
            assert np.array_equal(r["uniforms"][b].view(np.uint32), want_u.view(np.uint32)), (step, b)
            u, d = r["uniforms"][b], r["draft_tokens"][b]
            for j in range(k):
                assert ora.sample(s_ora, r["draft_logits"][b, j:j + 1], u[j:j + 1])[0] == d[j], (step, b, j)
        out, nacc = ora.accept(s_ora, r["target_logits"], r["draft_logits"], r["draft_tokens"], r["uniforms"][:, k:])
        assert np.array_equal(nacc, r["n_accepted"]) and np.array_equal(out, r["out_tokens"]), step
        for b in range(B):
            n = ns[b]
            toks = np.concatenate([[seqs[b][n - 1]], r["draft_tokens"][b]]).astype(np.int32)
            ref.forward(np.array(seqs[b][:n - 1], np.int32), 0)
            tl = ref.forward(toks, n - 1, n_logits=k + 1)
            a = r["target_logits"][b].astype(np.float64)
            worst = max(worst, float(np.abs(a - tl).max() / np.sqrt((tl.astype(np.float64) ** 2).mean())))
            seqs[b] += list(r["out_tokens"][b][:r["n_accepted"][b] + 1])
    for b in range(B):
        assert np.array_equal(sp.tokens(seq=b), np.array(seqs[b], np.int32))
    print(f"  {mode}: batched vs one-sequence target logits, max err / rms {worst:.2e}")
    assert worst <= LOGIT_TOL
    for m in (sp, gt, gd, ref):
        m.close()


def test_batch_argument_errors(pkg, ctx, weights, prompts):
    tw, dw = weights
    gt, gd = _gpu(pkg, ctx, TARGET, tw, n_seq=2), _gpu(pkg, ctx, DRAFT, dw, n_seq=2)
    with pytest.raises(pkg.UlspecError) as e:  # more sequences than the models' slots
        pkg.Speculative(gt, gd, 4, pkg.sampling(greedy=True), 1, n_seq=3)
    assert e.value.status == pkg.EINVAL
    sp = pkg.Speculative(gt, gd, 4, pkg.sampling(greedy=True), 1, n_seq=2)
    with pytest.raises(pkg.UlspecError) as e:  # a batch prefill needs two tokens per sequence
        sp.prefill([prompts[0], prompts[1][:1]])
    assert e.value.status == pkg.EINVAL
    with pytest.raises(pkg.UlspecError) as e:
        pkg.Model(ctx, **TARGET, n_seq=9)
    assert e.value.status == pkg.EINVAL
    for m in (sp, gt, gd):
        m.close()
