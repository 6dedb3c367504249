"""Speculative decoding at the 7B shape against the oracle, through the C ABI.

Workload: random-init Q4_K target (dim 4096, 32 layers, 32 heads, FFN 11008,
vocab 32000) and draft (dim 2048, 16 layers, 16 heads, FFN 5632), k = 5,
batch 1, a seeded prompt of 2048 tokens.  The GPU runs the prefill; the
oracle starts from the GPU's post-prefill K/V cache (a CPU prefill of 2047
tokens through both models would take minutes) and then computes every step
itself.

Bars:
  - greedy, free-running: the committed tokens and the acceptance counters
    of 8 steps are bit-exact with the oracle's own loop;
  - temperature 0.8 over the full vocabulary, teacher-forced on the GPU's
    committed tokens: every draft draw and accept decision is bit-exact with
    the oracle's rule on the step's logits, the oracle's own logits for the
    same tokens are within LOGIT_TOL of their RMS (max |error| / RMS over all
    rows of the step), and the oracle's own draws and decisions on its own
    logits equal the GPU's.  The activations are fp32 on both sides (split
    fp16 pairs into the GPU's MFMAs); only Q and the K/V cache are fp16, so
    the two differ by fp32 summation order and the fp16 roundings that order
    moves.
  - the growth of that difference with depth: the same weights cut to 1, 2,
    4, 8, 16 and 32 layers, one 64-token forward on each side.
"""
import importlib

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TARGET = dict(dim=4096, n_layers=32, n_heads=32, n_kv_heads=32, ffn=11008, vocab=32000, rms_eps=1e-5,
              rope_base=10000.0)
DRAFT = dict(dim=2048, n_layers=16, n_heads=16, n_kv_heads=16, ffn=5632, vocab=32000, rms_eps=1e-5,
             rope_base=10000.0)
CONTEXT, K_SPEC, STEPS = 2048, 5, 8
CAP = CONTEXT + 2 * STEPS * (K_SPEC + 1) + 32
LOGIT_TOL = 1e-2
Q4_K = 12


@pytest.fixture(scope="module")
def host_target(pkg, ctx):
    """GGUF bytes of every target tensor (the synthetic weights of seed 1)."""
    synthetic_llama = importlib.import_module("universal_loader_amd.synthetic").synthetic_llama
    gt, th = synthetic_llama(pkg, ctx, dict(TARGET, max_ctx=CAP), Q4_K, seed=1, keep_host=True)
    yield gt, th
    gt.close()


@pytest.fixture(scope="module")
def models(pkg, ctx, ora, host_target):
    synthetic_llama = importlib.import_module("universal_loader_amd.synthetic").synthetic_llama
    gt, th = host_target
    gd, dh = synthetic_llama(pkg, ctx, dict(DRAFT, max_ctx=CAP), Q4_K, seed=2, keep_host=True)
    oms = []
    for cfg, host in ((TARGET, th), (DRAFT, dh)):
        m = ora.Llama(**cfg, max_ctx=CAP, nthreads=ora.nthreads_default())
        for name, (wtype, data, ne0, ne1) in host.items():
            m.set_tensor(name, wtype, data, ne0, ne1)
        oms.append(m)
    del dh
    yield gt, gd, oms[0], oms[1]
    for m in (gd, *oms):
        m.close()


@pytest.fixture(scope="module")
def prompt():
    return np.random.default_rng(1234).integers(0, TARGET["vocab"], CONTEXT).astype(np.int32)


def _prefill(pkg, models, prompt, s, seed):
    """GPU prefill, then the oracle models take the GPU's K/V rows 0 .. n-2."""
    gt, gd, ot, od = models
    sp = pkg.Speculative(gt, gd, K_SPEC, s, seed)
    sp.prefill(prompt)
    for g, o, cfg in ((gt, ot, TARGET), (gd, od, DRAFT)):
        for l in range(cfg["n_layers"]):
            k, v = g.kv_io(l, 0, 0, CONTEXT - 1)
            o.kv_io(l, 1, 0, CONTEXT - 1, k, v)
    return sp


def test_7b_greedy_tokens_bit_exact(pkg, ora, models, prompt):
    gt, gd, ot, od = models
    seed = 31
    sp = _prefill(pkg, models, prompt, pkg.sampling(greedy=True), seed)
    osp = ora.Speculative(ot, od, K_SPEC, ora.sampling(greedy=True), seed, cap=CAP)
    osp.seq[:CONTEXT] = prompt
    osp.st.n = CONTEXT
    for step in range(STEPS):
        sp.steps(1)
        osp.step()
        print(f"  step {step}: gpu n={sp.state()['n']} oracle n={osp.state()['n']}", flush=True)
    got, st = sp.tokens(), sp.state()
    print(f"  greedy 7B: {st['n'] - CONTEXT} tokens in {st['steps']} steps, accepted {st['accepted']}/{st['proposed']}")
    assert np.array_equal(got, osp.tokens())
    assert st == osp.state()
    sp.close()


def test_7b_sampling_steps_bit_exact(pkg, ora, models, prompt):
    gt, gd, ot, od = models
    seed, k = 2024, K_SPEC
    s_ora = ora.sampling(temperature=0.8)
    sp = _prefill(pkg, models, prompt, pkg.sampling(temperature=0.8), seed)
    seq = list(prompt)
    worst = 0.0
    accepted = 0
    for step in range(STEPS):
        n = len(seq)
        sp.steps(1)
        r = sp.last_step()
        u, d = r["uniforms"], r["draft_tokens"]
        for j in range(k):
            assert ora.sample(s_ora, r["draft_logits"][j:j + 1], u[j:j + 1])[0] == d[j], (step, j)
        out, nacc = ora.accept(s_ora, r["target_logits"][None], r["draft_logits"][None], d[None], u[k:][None])
        assert int(nacc[0]) == r["n_accepted"] and np.array_equal(out[0], r["out_tokens"]), step
        dl = [od.forward(np.array(seq[n - 2:n], np.int32), n - 2, n_logits=1)[0]]
        for j in range(1, k):
            dl.append(od.forward(d[j - 1:j], n - 1 + j, n_logits=1)[0])
        dl = np.array(dl)
        tl = ot.forward(np.concatenate([[seq[n - 1]], d]).astype(np.int32), n - 1, n_logits=k + 1)
        errs = []
        for a, b in ((r["draft_logits"], dl), (r["target_logits"], tl)):
            b64 = b.astype(np.float64)
            errs.append(np.abs(a.astype(np.float64) - b64).max() / np.sqrt((b64 ** 2).mean()))
        worst = max(worst, *errs)
        # the CPU path's own step: its draws on its own draft logits, its decisions on its own logits
        own_d = [int(ora.sample(s_ora, dl[j][None], u[j:j + 1])[0]) for j in range(k)]
        out_c, nacc_c = ora.accept(s_ora, tl[None], dl[None], d[None], u[k:][None])
        print(f"  step {step}: accepted {r['n_accepted']} (oracle's own {int(nacc_c[0])}), logits max err / rms "
              f"draft {errs[0]:.2e} target {errs[1]:.2e}", flush=True)
        assert own_d == [int(x) for x in d], step
        assert int(nacc_c[0]) == r["n_accepted"] and np.array_equal(out_c[0], r["out_tokens"]), step
        seq += list(r["out_tokens"][:r["n_accepted"] + 1])
        accepted += r["n_accepted"]
    assert np.array_equal(sp.tokens(), np.array(seq, np.int32))
    assert sp.state()["accepted"] == accepted
    print(f"  T=0.8 7B: {len(seq) - CONTEXT} tokens, accepted {accepted}/{k * STEPS}, worst logits err {worst:.2e}")
    assert worst <= LOGIT_TOL
    sp.close()


@pytest.mark.parametrize("mode", ["greedy", "sampling"])
def test_7b_tree_steps_bit_exact(pkg, ora, models, prompt, mode):
    """16-node tree steps (branching <= 3, depth 5) on the 7B pair: draws,
    ulspec_accept_tree decisions, K/V compaction of both caches and commits
    against the oracle, teacher-forced (tree_step_util.check_tree_steps); the
    node logits against the oracle's path forwards within LOGIT_TOL."""
    from tree_step_util import TREE16, check_tree_steps
    gt, gd, ot, od = models
    seed = 4242
    args = dict(greedy=True) if mode == "greedy" else dict(temperature=0.8)
    sp = pkg.Speculative(gt, gd, 0, pkg.sampling(**args), seed, parent=TREE16)
    sp.prefill(prompt)
    for g, o, cfg in ((gt, ot, TARGET), (gd, od, DRAFT)):
        for l in range(cfg["n_layers"]):
            k, v = g.kv_io(l, 0, 0, CONTEXT - 1)
            o.kv_io(l, 1, 0, CONTEXT - 1, k, v)
    seq, worst = check_tree_steps(ora, sp, ot, od, ora.sampling(**args), list(prompt), TREE16, seed, 3,
                                  mode == "greedy", LOGIT_TOL)
    print(f"  7B tree {mode}: {len(seq) - CONTEXT} tokens in 3 steps, worst logits err {worst:.2e}")
    sp.close()


def test_7b_logit_error_by_depth(pkg, ctx, ora, host_target):
    """The GPU / oracle logit difference as the target grows from 1 to 32
    layers (the same weights, a fresh 64-token prompt, the last 6 rows): the
    measured growth behind LOGIT_TOL.  Each depth must stay within it."""
    _, th = host_target
    prompt = np.random.default_rng(99).integers(0, TARGET["vocab"], 64).astype(np.int32)
    rows = []
    for L in (1, 2, 4, 8, 16, 32):
        cfg = dict(TARGET, n_layers=L)
        keep = {name: t for name, t in th.items()
                if not name.startswith("blk.") or int(name.split(".")[1]) < L}
        g = pkg.Model(ctx, **cfg, max_ctx=128)
        o = ora.Llama(**cfg, max_ctx=128, nthreads=ora.nthreads_default())
        for name, (wtype, data, ne0, ne1) in keep.items():
            g.set_tensor(name, wtype, data, ne0, ne1)
            o.set_tensor(name, wtype, data, ne0, ne1)
        lg = g.forward(prompt, 0, n_logits=K_SPEC + 1).astype(np.float64)
        lo = o.forward(prompt, 0, n_logits=K_SPEC + 1).astype(np.float64)
        rms = float(np.sqrt((lo ** 2).mean()))
        err = float(np.abs(lg - lo).max() / rms)
        mean = float(np.abs(lg - lo).mean() / rms)
        same = int((np.argmax(lg, axis=1) == np.argmax(lo, axis=1)).sum())
        rows.append((L, err, mean, rms, same))
        print(f"  {L:2d} layers: max err / rms {err:.2e}, mean {mean:.2e} (logit rms {rms:.3f}), "
              f"argmax equal in {same}/{K_SPEC + 1} rows", flush=True)
        g.close()
        o.close()
    assert all(err <= LOGIT_TOL for _, err, _, _, _ in rows)
