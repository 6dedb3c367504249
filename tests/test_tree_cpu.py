"""Pins of the oracle's tree acceptance (ora_accept_tree), CPU only: on a
chain it must be ora_accept's rule token for token (that rule is pinned in
test_oracle_cpu.py); greedy walks satisfy the argmax invariants; and with
sibling drafts drawn from the draft distribution, the emitted tokens follow
the target distribution (multi-draft speculative sampling is unbiased), which
fails for a plausible slip such as testing later siblings against p instead
of the running residual."""
import numpy as np
import pytest

from tree_util import random_tree


@pytest.mark.parametrize("mode", ["greedy", "full", "topk"])
def test_chain_tree_is_the_linear_rule(ora, rng, mode):
    B, k, V = 24, 5, 300
    s = {"greedy": ora.sampling(greedy=True), "full": ora.sampling(0.8),
         "topk": ora.sampling(0.8, top_k=20, top_p=0.9)}[mode]
    tl = (rng.standard_normal((B, k + 1, V)) * 3).astype(np.float32)
    dl = (rng.standard_normal((B, k + 1, V)) * 3).astype(np.float32)
    dl[:, :k] = np.where(rng.random((B, k, 1)) < 0.5, tl[:, :k], dl[:, :k])  # some rows agree: long accepts
    drafts = np.argmax(dl[:, :k] + rng.gumbel(size=(B, k, V)).astype(np.float32), axis=2).astype(np.int32)
    u = rng.random((B, k + 1)).astype(np.float32)
    out_l, nacc_l = ora.accept(s, tl, dl[:, :k], drafts, u)
    tokens = np.concatenate([np.full((B, 1), 9, np.int32), drafts], 1)
    parent = np.arange(-1, k, dtype=np.int32)
    out_t, path, nacc_t = ora.accept_tree(s, parent, tl, dl, tokens, u)
    assert np.array_equal(nacc_t, nacc_l) and np.array_equal(out_t, out_l)
    for b in range(B):
        assert list(path[b, :nacc_t[b] + 1]) == list(range(nacc_t[b] + 1)) and all(path[b, nacc_t[b] + 1:] == -1)
    assert 0 < nacc_l.sum() < B * k


def test_greedy_tree_walk_invariants(ora, rng):
    B, n, V = 40, 16, 50
    parent = random_tree(rng, n)
    tl = rng.standard_normal((B, n, V)).astype(np.float32)
    tokens = rng.integers(0, V, (B, n)).astype(np.int32)
    # make about half of the children carry their parent's argmax
    am = np.argmax(tl, axis=2)
    for b in range(B):
        for c in range(1, n):
            if rng.random() < 0.5:
                tokens[b, c] = am[b, parent[c]]
    out, path, nacc = ora.accept_tree(ora.sampling(greedy=True), parent, tl, None, tokens, None)
    for b in range(B):
        L = nacc[b]
        assert path[b, 0] == 0 and all(path[b, L + 1:] == -1) and all(out[b, L + 1:] == -1)
        for d in range(1, L + 1):
            c, v = path[b, d], path[b, d - 1]
            assert parent[c] == v and out[b, d - 1] == tokens[b, c] == am[b, v]
            # the first child of v with that token
            assert not any(parent[c2] == v and tokens[b, c2] == am[b, v] for c2 in range(1, c))
        last = path[b, L]
        assert out[b, L] == am[b, last]
        assert not any(parent[c] == last and tokens[b, c] == am[b, last] for c in range(1, n))
    assert nacc.max() >= 2


def _probs(ora, s, logits):
    E, Z, _ = ora.warp_row(s, logits)
    return E.astype(np.float64) / Z


def _chi2(obs, p):
    exp = p * obs.sum()
    m = exp > 0
    assert np.all(obs[~m] == 0)
    return float(((obs[m] - exp[m]) ** 2 / exp[m]).sum())


@pytest.mark.parametrize("temp,top_k", [(1.0, 0), (0.7, 3)])
def test_siblings_drawn_from_q_give_p(ora, rng, temp, top_k):
    # root with three children drawn i.i.d. from q: the first emitted token
    # follows p, and the token after an accepted child follows that child's row
    V, B = 5, 120000
    s = ora.sampling(temp, top_k=top_k)
    parent = np.array([-1, 0, 0, 0], np.int32)
    p0 = (rng.standard_normal(V) * 1.5).astype(np.float32)
    q0 = (rng.standard_normal(V) * 1.5).astype(np.float32)
    rows = (rng.standard_normal((V, V)) * 1.5).astype(np.float32)  # target row of a child with token x
    pp, qq = _probs(ora, s, p0), _probs(ora, s, q0)
    kids = rng.choice(V, size=(B, 3), p=qq).astype(np.int32)
    tokens = np.concatenate([np.zeros((B, 1), np.int32), kids], 1)
    tl = np.empty((B, 4, V), np.float32)
    tl[:, 0] = p0
    tl[:, 1:] = rows[kids]
    dl = np.zeros((B, 4, V), np.float32)
    dl[:, 0] = q0
    u = rng.random((B, 4)).astype(np.float32)
    out, path, nacc = ora.accept_tree(s, parent, tl, dl, tokens, u)
    assert _chi2(np.bincount(out[:, 0], minlength=V).astype(np.float64), pp) < 30.0
    acc = nacc == 1
    assert 0.01 < acc.mean() < 1.0
    for x in range(V):
        sel = acc & (out[:, 0] == x)
        if sel.sum() > 2000:
            assert _chi2(np.bincount(out[sel, 1], minlength=V).astype(np.float64), _probs(ora, s, rows[x])) < 30.0


def test_residual_chain_matters(ora, rng):
    # the same trials with the running residual replaced by p for every
    # sibling (a plausible slip, planted here on the CPU) are biased:
    # the rule above is what makes the first token follow p
    V, B = 5, 60000
    s = ora.sampling(1.0)
    p0 = np.array([2.0, 0.0, -1.0, 0.5, -0.5], np.float32)
    q0 = np.array([-1.0, 2.0, 0.0, -0.5, 1.0], np.float32)
    pp, qq = _probs(ora, s, p0), _probs(ora, s, q0)
    kids = rng.choice(V, size=(B, 3), p=qq)
    u = rng.random((B, 4))
    emitted = np.empty(B, np.int64)
    for b in range(B):
        for j in range(3):
            x = kids[b, j]
            if u[b, j] * qq[x] < pp[x]:  # every sibling against p: the slip
                emitted[b] = x
                break
        else:
            r = np.maximum(pp - qq, 0)
            emitted[b] = np.searchsorted(np.cumsum(r / r.sum()), u[b, 3], side="right")
    assert _chi2(np.bincount(emitted, minlength=V).astype(np.float64), pp) > 100.0


def test_tree_rejects_bad_parents(ora, rng):
    V = 10
    tl = rng.standard_normal((1, 3, V)).astype(np.float32)
    s = ora.sampling(greedy=True)
    for parent in ([0, 0, 1], [-1, 1, 0], [-1, 0, 3], [-1, -1, 0]):
        with pytest.raises(ValueError):
            ora.accept_tree(s, np.array(parent, np.int32), tl, None, np.zeros((1, 3), np.int32), None)
