"""End-to-end speculative decoding on the GPU (model forward, device loop,
graph replay) against the oracle, through the C ABI.

Bar: the committed token sequences and acceptance counters are bit-exact with
the oracle's loop on the same weights, prompt and seed.  Model logits agree
within LOGIT_TOL of their RMS (max |error| / RMS): activations are fp32 on both
sides (split fp16 pairs into the GPU's MFMAs), only Q and the K/V cache are
fp16, so the two differ by fp32 summation order and the fp16 roundings of Q,
K and V that it moves (measured 2e-4 on this model).
"""
import numpy as np
import pytest

from llama_util import load, make_tensors

pytestmark = pytest.mark.gpu

# tiny Llama: dim 512, 8 layers, 8 heads x 64, FFN 1376, vocab 32000, Q4_0;
# draft: 2 layers of the same dims
TARGET = dict(dim=512, n_layers=8, n_heads=8, n_kv_heads=8, ffn=1376, vocab=32000, max_ctx=256, rms_eps=1e-5,
              rope_base=10000.0)
DRAFT = dict(TARGET, n_layers=2)
LOGIT_TOL = 2e-3


@pytest.fixture(scope="module")
def weights(ora):
    return make_tensors(ora, TARGET, 2, seed=101), make_tensors(ora, DRAFT, 2, seed=202)


@pytest.fixture(scope="module")
def prompt():
    return np.random.default_rng(77).integers(0, 32000, 64).astype(np.int32)


def _gpu_model(pkg, ctx, cfg, tensors):
    m = pkg.Model(ctx, **cfg)
    load(m, tensors)
    return m


def _ora_model(ora, cfg, tensors):
    m = ora.Llama(**cfg, nthreads=ora.nthreads_default())
    load(m, tensors)
    return m


def test_model_forward_logits_and_cache(pkg, ctx, ora, weights, prompt):
    tw, _ = weights
    g, o = _gpu_model(pkg, ctx, TARGET, tw), _ora_model(ora, TARGET, tw)
    lg = g.forward(prompt[:40], 0, n_logits=16)  # chunks of 16 and a final chunk of 16
    lo = o.forward(prompt[:40], 0, n_logits=16)
    scale = np.sqrt((lo.astype(np.float64) ** 2).mean())
    err = np.abs(lg.astype(np.float64) - lo).max() / scale
    print(f"  logits max err / rms = {err:.2e}, mean {np.abs(lg - lo).mean() / scale:.2e}")
    assert err <= LOGIT_TOL
    assert np.array_equal(np.argmax(lg, axis=1), np.argmax(lo, axis=1))
    for l in (0, TARGET["n_layers"] - 1):
        kg, vg = g.kv_io(l, 0, 0, 40)
        ko, vo = o.kv_io(l, 0, 0, 40)
        for a, b in ((kg, ko), (vg, vo)):
            a, b = ora.h2f_fast(a).astype(np.float64), ora.h2f_fast(b).astype(np.float64)
            # fp16 cache entries: one ulp (2^-10 relative) where the fp32 values
            # on either side of a rounding boundary differ in the last bits
            assert (np.abs(a - b) <= np.abs(b) * 2.0 ** -10 + 1e-3 * np.sqrt((b ** 2).mean())).all()
    g.close()


def test_forward_rows_are_batch_invariant(pkg, ctx, weights, prompt):
    tw, _ = weights
    a, b = _gpu_model(pkg, ctx, TARGET, tw), _gpu_model(pkg, ctx, TARGET, tw)
    la = a.forward(prompt[:6], 0, n_logits=6)
    lb = np.concatenate([b.forward(prompt[i:i + 1], i, n_logits=1) for i in range(6)])
    assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    a.close()
    b.close()


def test_greedy_tokens_bit_exact_with_oracle(pkg, ctx, ora, weights, prompt):
    """Free-running greedy decoding: the whole committed sequence and the
    counters equal the oracle's (argmax decisions are robust to the fp32
    summation order)."""
    tw, dw = weights
    k, n_new, seed = 4, 128, 2024
    gt, gd = _gpu_model(pkg, ctx, TARGET, tw), _gpu_model(pkg, ctx, DRAFT, dw)
    sp = pkg.Speculative(gt, gd, k, pkg.sampling(greedy=True), seed)
    sp.prefill(prompt)
    n = sp.generate(n_new)
    got, st = sp.tokens(), sp.state()
    ot, od = _ora_model(ora, TARGET, tw), _ora_model(ora, DRAFT, dw)
    osp = ora.Speculative(ot, od, k, ora.sampling(greedy=True), seed)
    osp.prefill(prompt)
    on = osp.generate(n_new)
    print(f"  greedy: {n} tokens in {st['steps']} steps, accepted {st['accepted']}/{st['proposed']}")
    assert n == on and n >= n_new
    assert np.array_equal(got, osp.tokens())
    assert st == osp.state()
    for m in (sp, gt, gd):
        m.close()


@pytest.mark.parametrize("top_p", [1.0, 0.9])
def test_sampling_steps_bit_exact_with_oracle(pkg, ctx, ora, weights, prompt, top_p):
    """Temperature 0.8 over the full vocabulary (and with top_p 0.9 alone, the
    kept prefix selected on the device), step by step: the oracle runs
    the same step on the GPU's committed sequence and draft tokens (teacher
    forcing).  Every draft draw and every accept decision is bit-exact with the
    oracle's rule on the step's logits; the oracle's own logits for the same
    tokens agree within LOGIT_TOL of their RMS.  (Free-running sequences are not
    compared token for token: an inverse-CDF draw over 32000 tokens moves when
    the logits move by 1e-4, so fp32 order differences change some draws.)"""
    tw, dw = weights
    k, n_new, seed = 4, 128 if top_p == 1.0 else 48, 2024
    s_gpu, s_ora = pkg.sampling(temperature=0.8, top_p=top_p), ora.sampling(temperature=0.8, top_p=top_p)
    gt, gd = _gpu_model(pkg, ctx, TARGET, tw), _gpu_model(pkg, ctx, DRAFT, dw)
    sp = pkg.Speculative(gt, gd, k, s_gpu, seed)
    sp.prefill(prompt)
    ot, od = _ora_model(ora, TARGET, tw), _ora_model(ora, DRAFT, dw)
    ot.forward(prompt[:-1], 0)
    od.forward(prompt[:-1], 0)
    seq = list(prompt)
    worst = 0.0
    steps = accepted = 0
    while len(seq) - len(prompt) < n_new:
        n = len(seq)
        sp.steps(1)
        r = sp.last_step()
        u = r["uniforms"]
        want_u = np.array([ora.uniforms(seed, steps * (2 * k + 1) + j, 1)[0] for j in range(2 * k + 1)], np.float32)
        assert np.array_equal(u.view(np.uint32), want_u.view(np.uint32))
        # draft draws
        for j in range(k):
            assert ora.sample(s_ora, r["draft_logits"][j:j + 1], u[j:j + 1])[0] == r["draft_tokens"][j], (steps, j)
        # accept rule on the step's logits
        out, nacc = ora.accept(s_ora, r["target_logits"][None], r["draft_logits"][None], r["draft_tokens"][None],
                               u[k:][None])
        assert int(nacc[0]) == r["n_accepted"] and np.array_equal(out[0], r["out_tokens"]), steps
        # the oracle's logits for the same tokens
        d = r["draft_tokens"]
        dl = [od.forward(np.array(seq[n - 2:n], np.int32), n - 2, n_logits=1)[0]]
        for j in range(1, k):
            dl.append(od.forward(d[j - 1:j], n - 1 + j, n_logits=1)[0])
        tl = ot.forward(np.concatenate([[seq[n - 1]], d]).astype(np.int32), n - 1, n_logits=k + 1)
        for a, b in ((r["draft_logits"], np.array(dl)), (r["target_logits"], tl)):
            worst = max(worst, np.abs(a.astype(np.float64) - b).max() / np.sqrt((b.astype(np.float64) ** 2).mean()))
        seq += list(r["out_tokens"][:r["n_accepted"] + 1])
        steps += 1
        accepted += r["n_accepted"]
    st = sp.state()
    assert np.array_equal(sp.tokens(), np.array(seq, np.int32))
    assert st["steps"] == steps and st["accepted"] == accepted and st["proposed"] == k * steps
    print(f"  t0.8 top_p {top_p}: {len(seq) - len(prompt)} tokens in {steps} steps, accepted {accepted}/{k * steps}, "
          f"logits max err / rms {worst:.2e}")
    assert worst <= LOGIT_TOL
    for m in (sp, gt, gd):
        m.close()


def test_graph_replay_equals_direct_launches(pkg, ctx, weights, prompt):
    tw, dw = weights
    outs = []
    for use_graph in (True, False, True):
        gt, gd = _gpu_model(pkg, ctx, TARGET, tw), _gpu_model(pkg, ctx, DRAFT, dw)
        sp = pkg.Speculative(gt, gd, 5, pkg.sampling(temperature=0.8), 7)
        sp.set_graph(use_graph)
        sp.prefill(prompt)
        for _ in range(4):  # several replays with host work and syncs between them
            sp.steps(3)
            sp.state()
        outs.append((sp.tokens(), sp.state()))
        sp.close()
        gt.close()
        gd.close()
    for t, s in outs[1:]:
        assert np.array_equal(t, outs[0][0]) and s == outs[0][1]


def test_draft_equal_to_target_accepts_everything(pkg, ctx, weights, prompt):
    _, dw = weights
    a, b = _gpu_model(pkg, ctx, DRAFT, dw), _gpu_model(pkg, ctx, DRAFT, dw)
    sp = pkg.Speculative(a, b, 4, pkg.sampling(temperature=0.8), 99)
    sp.prefill(prompt)
    sp.steps(10)
    st = sp.state()
    assert st["steps"] == 10 and st["accepted"] == st["proposed"] == 40 and st["n"] == 64 + 50
    sp.close()
    a.close()
    b.close()


def test_greedy_speculation_equals_autoregressive_argmax(pkg, ctx, weights, prompt):
    tw, dw = weights
    gt, gd = _gpu_model(pkg, ctx, TARGET, tw), _gpu_model(pkg, ctx, DRAFT, dw)
    sp = pkg.Speculative(gt, gd, 3, pkg.sampling(greedy=True), 1)
    sp.prefill(prompt[:20])
    sp.generate(24)
    got = sp.tokens()
    ref = _gpu_model(pkg, ctx, TARGET, tw)
    seq = list(prompt[:20])
    ref.forward(np.array(seq[:-1], np.int32), 0)
    while len(seq) < len(got):
        lg = ref.forward(np.array(seq[-1:], np.int32), len(seq) - 1, n_logits=1)[0]
        seq.append(int(np.argmax(lg)))
    assert list(got) == seq
    for m in (sp, gt, gd, ref):
        m.close()


def test_plain_decoding_bit_exact_with_oracle(pkg, ctx, ora, weights, prompt):
    """k = 0 (no draft): one target row and one draw per token.  Greedy:
    the oracle's own plain loop, free-running, token for token.  T = 0.8:
    every draw is the oracle's rule on the step's logits with u(seed, step)."""
    tw, _ = weights
    gt = _gpu_model(pkg, ctx, TARGET, tw)
    ot = _ora_model(ora, TARGET, tw)
    sp = pkg.Speculative(gt, None, 0, pkg.sampling(greedy=True), 5)
    sp.prefill(prompt[:30])
    sp.generate(20)
    osp = ora.Speculative(ot, None, 0, ora.sampling(greedy=True), 5)
    osp.prefill(prompt[:30])
    osp.generate(20)
    assert np.array_equal(sp.tokens(), osp.tokens())
    assert sp.state() == dict(osp.state(), proposed=0, accepted=0) and sp.state()["steps"] == 20
    sp.close()
    s, so, seed = pkg.sampling(temperature=0.8), ora.sampling(temperature=0.8), 11
    sp = pkg.Speculative(gt, None, 0, s, seed)
    sp.prefill(prompt[:30])
    for step in range(12):
        n = sp.state()["n"]
        sp.steps(1)
        r = sp.last_step()
        u = ora.uniforms(seed, step, 1)
        assert r["uniforms"][0].view(np.uint32) == u[0].view(np.uint32)
        assert sp.tokens(n, 1)[0] == ora.sample(so, r["target_logits"], u)[0], step
    sp.close()
    gt.close()
    ot.close()


def test_one_token_prompt_starts_with_a_plain_step(pkg, ctx, ora, weights, prompt):
    """A prompt of one token: the first step is plain (the draft's catch-up
    pair needs two tokens), then speculative steps; greedy, bit-exact with the
    oracle's loop, which does the same."""
    tw, dw = weights
    gt, gd = _gpu_model(pkg, ctx, TARGET, tw), _gpu_model(pkg, ctx, DRAFT, dw)
    ot, od = _ora_model(ora, TARGET, tw), _ora_model(ora, DRAFT, dw)
    sp = pkg.Speculative(gt, gd, 4, pkg.sampling(greedy=True), 3)
    sp.prefill(prompt[:1])
    sp.generate(30)
    osp = ora.Speculative(ot, od, 4, ora.sampling(greedy=True), 3)
    osp.prefill(prompt[:1])
    osp.generate(30)
    assert np.array_equal(sp.tokens(), osp.tokens())
    assert sp.state() == osp.state()
    for m in (sp, gt, gd, ot, od):
        m.close()


def test_synth_matches_oracle_synthesizer(pkg, ctx, ora):
    for wtype, N, K in ((2, 64, 4096), (12, 48, 2048)):
        buf = ctx.alloc(N * pkg.row_bytes(wtype, K))
        ctx.synth_q4(wtype, 5, 3, N, K, 0.02, buf)
        got = ctx.download(buf, np.uint8, (N * pkg.row_bytes(wtype, K),))
        want = ora.synth_q4(wtype, 5, 3, N, K, float(np.float32(0.02)))
        bs = 18 if wtype == 2 else 144
        same = (got.reshape(-1, bs) == want.reshape(-1, bs)).all(axis=1).mean()
        # device double log / cos / sin may round a normal differently from libm
        assert same >= 0.999, same
        x = ora.dequantize(wtype, got, N * K)
        assert abs(x.std() - 0.02) < 0.002 and abs(x.mean()) < 0.002
        buf.free()


def test_model_and_spec_argument_errors(pkg, ctx, weights):
    tw, _ = weights
    m = pkg.Model(ctx, **DRAFT)
    with pytest.raises(pkg.UlspecError) as e:
        m.set_tensor("blk.0.nonsense.weight", 2, np.zeros(18, np.uint8), 32, 1)
    assert e.value.status == pkg.EINVAL
    with pytest.raises(pkg.UlspecError) as e:
        m.set_tensor("blk.9.attn_q.weight", *tw["blk.0.attn_q.weight"])
    assert e.value.status == pkg.EINVAL
    name = "blk.0.ffn_down.weight"
    wtype, data, ne0, ne1 = tw[name]
    with pytest.raises(pkg.UlspecError) as e:
        m.set_tensor(name, wtype, data, ne1, ne0)  # transposed shape
    assert e.value.status == pkg.EINVAL
    with pytest.raises(pkg.UlspecError) as e:  # tensors missing
        m.forward(np.array([1, 2], np.int32), 0)
    assert e.value.status == pkg.EINVAL
    with pytest.raises(pkg.UlspecError) as e:
        pkg.Model(ctx, **dict(DRAFT, dim=96 * 8))  # head dim 96
    assert e.value.status == pkg.EUNSUPPORTED
    m.close()


def test_spec_k_limit(pkg, ctx, weights):
    """k draft tokens need k + 1 verify rows of the 16 a forward takes: k = 15
    is the largest loop, k = 16 fails with EINVAL."""
    _, dw = weights
    t, d = _gpu_model(pkg, ctx, DRAFT, dw), _gpu_model(pkg, ctx, DRAFT, dw)
    sp = pkg.Speculative(t, d, 15, pkg.sampling(greedy=True), 1)
    sp.close()
    with pytest.raises(pkg.UlspecError) as e:
        pkg.Speculative(t, d, 16, pkg.sampling(greedy=True), 1)
    assert e.value.status == pkg.EINVAL and "k <= 15" in str(e.value)
    t.close()
    d.close()
