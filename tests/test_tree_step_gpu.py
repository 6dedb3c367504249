"""Tree steps of the device loop (a 16-node draft tree, branching <= 3,
depth 5) on the GPU against the oracle, through the C ABI.

Bar, for every step (teacher-forced on the GPU's committed tokens): the
uniforms follow u(seed, s(2n-1) + j); every child token is the oracle's draw
from its parent's draft logits (sampling: i.i.d. with the child's uniform;
greedy: the parent's best tokens in order); the accepted path, tokens and
count equal ulspec_accept_tree's oracle on the step's logits; the committed
sequence is the path plus the final token; and every node's target and draft
logits agree with the oracle's causal forward of the node's root-to-node
path within LOGIT_TOL of their RMS (fp32 activations on both sides; fp16
K/V) -- which also checks the K/V compaction of both caches across steps.
A chain-shaped tree reproduces the chain loop token for token.
"""
import numpy as np
import pytest

from llama_util import load, make_tensors
from tree_step_util import TREE16, check_tree_steps

pytestmark = pytest.mark.gpu

TARGET = dict(dim=512, n_layers=8, n_heads=8, n_kv_heads=8, ffn=1376, vocab=32000, max_ctx=256, rms_eps=1e-5,
              rope_base=10000.0)
DRAFT = dict(TARGET, n_layers=2)
LOGIT_TOL = 2e-3


@pytest.fixture(scope="module")
def weights(ora):
    return make_tensors(ora, TARGET, 2, seed=101), make_tensors(ora, DRAFT, 2, seed=202)


@pytest.fixture(scope="module")
def prompt():
    return np.random.default_rng(77).integers(0, 32000, 40).astype(np.int32)


def _models(pkg, ctx, ora, weights):
    tw, dw = weights
    out = []
    for cfg, w in ((TARGET, tw), (DRAFT, dw)):
        m = pkg.Model(ctx, **cfg)
        load(m, w)
        out.append(m)
    for cfg, w in ((TARGET, tw), (DRAFT, dw)):
        m = ora.Llama(**cfg, nthreads=ora.nthreads_default())
        load(m, w)
        out.append(m)
    return out


@pytest.mark.parametrize("mode", ["greedy", "full", "topk_topp"])
def test_tree_steps_bit_exact_with_oracle(pkg, ctx, ora, weights, prompt, mode):
    args = {"greedy": dict(greedy=True), "full": dict(temperature=0.8),
            "topk_topp": dict(temperature=0.8, top_k=40, top_p=0.9)}[mode]
    gt, gd, ot, od = _models(pkg, ctx, ora, weights)
    seed = 99
    sp = pkg.Speculative(gt, gd, 0, pkg.sampling(**args), seed, parent=TREE16)
    sp.prefill(prompt)
    ot.forward(prompt[:-1], 0)
    od.forward(prompt[:-1], 0)
    seq, worst = check_tree_steps(ora, sp, ot, od, ora.sampling(**args), list(prompt), TREE16, seed, 5,
                                  mode == "greedy", LOGIT_TOL)
    st = sp.state()
    print(f"  {mode}: {len(seq) - len(prompt)} tokens in {st['steps']} steps, accepted {st['accepted']}, "
          f"worst logits err {worst:.2e}")
    assert st["steps"] == 5 and st["proposed"] == 5 * 5 and st["n"] == len(seq)
    for m in (sp, gt, gd, ot, od):
        m.close()


def test_chain_tree_equals_chain_loop(pkg, ctx, ora, weights, prompt):
    """A chain of k + 1 nodes drafts, accepts and commits as the chain loop
    (greedy: the draft rows of a tree forward take other GEMM row counts than
    the chain's single-token forwards, so sampled draws could move on fp32
    order)."""
    gt, gd, ot, od = _models(pkg, ctx, ora, weights)
    k, seed = 4, 5
    s = pkg.sampling(greedy=True)
    a = pkg.Speculative(gt, gd, 0, s, seed, parent=np.arange(-1, k, dtype=np.int32))
    a.prefill(prompt)
    a.generate(30)
    ta = a.tokens()
    a.close()
    b = pkg.Speculative(gt, gd, k, s, seed)
    b.prefill(prompt)
    b.generate(30)
    tb = b.tokens()
    b.close()
    m = min(len(ta), len(tb))
    assert m >= len(prompt) + 30 and np.array_equal(ta[:m], tb[:m])
    for x in (gt, gd, ot, od):
        x.close()


def test_tree_loop_rejects_bad_shapes(pkg, ctx, ora, weights):
    gt, gd, ot, od = _models(pkg, ctx, ora, weights)
    s = pkg.sampling(greedy=True)
    for parent in ([0, 0], [-1, 0, 1, 0], [-1, 0, 0, 2, 1], list(range(-1, 16))):  # root, depth order, BFS, 17 nodes
        with pytest.raises(pkg.UlspecError) as e:
            pkg.Speculative(gt, gd, 0, s, 1, parent=np.array(parent, np.int32))
        assert e.value.status == pkg.EINVAL, parent
    for x in (gt, gd, ot, od):
        x.close()
