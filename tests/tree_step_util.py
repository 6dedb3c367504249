"""Shared checks of the device loop's tree steps against the oracle
(test_tree_step_gpu.py at dim 512, test_spec7b_gpu.py at the 7B shape)."""
import numpy as np

# 16 nodes in breadth-first order, branching <= 3, depth 5: the root's three
# children, then 4, 4, 3 and 1 nodes on the next levels
TREE16 = np.array([-1, 0, 0, 0, 1, 1, 2, 3, 4, 4, 5, 6, 8, 8, 9, 12], np.int32)


def ancestors(parent, i):
    path = [i]
    while parent[path[-1]] >= 0:
        path.append(int(parent[path[-1]]))
    return path[::-1]


def check_tree_steps(ora, sp, ot, od, s_ora, seq, parent, seed, steps, greedy, logit_tol, log=print):
    """Step the GPU tree loop `steps` times from the committed sequence `seq`
    (the oracle models ot / od hold its K/V up to position len(seq) - 2) and
    check every step: uniforms, every draft draw, the acceptance, the
    committed tokens, and the logits of every node against the oracle's
    forward of the node's root-to-node path (max |error| / RMS <= logit_tol).
    Returns the committed sequence and the worst logits error."""
    n = len(parent)
    kids = {p: [c for c in range(1, n) if parent[c] == p] for p in range(n)}
    worst = 0.0
    for step in range(steps):
        n0 = len(seq)
        sp.steps(1)
        r = sp.last_step()
        u, tok, tl, dl = r["uniforms"], r["tokens"], r["target_logits"], r["draft_logits"]
        want_u = ora.uniforms(seed, step * (2 * n - 1), 2 * n - 1)
        assert np.array_equal(u.view(np.uint32), want_u.view(np.uint32)), step
        assert tok[0] == seq[-1]
        for p, cs in kids.items():
            if not cs:
                continue
            if greedy:  # the parent's best tokens in (logit desc, index asc) order
                order = np.lexsort((np.arange(dl.shape[1]), -dl[p].astype(np.float64)))
                assert [int(tok[c]) for c in cs] == [int(x) for x in order[:len(cs)]], (step, p)
            else:
                for c in cs:
                    assert ora.sample(s_ora, dl[p][None], u[c - 1:c])[0] == tok[c], (step, c)
        dfull = np.zeros((1, n, dl.shape[1]), np.float32)
        dfull[0, :n - 1] = dl
        out, path, nacc = ora.accept_tree(s_ora, parent, tl[None], dfull, tok[None], None if greedy else u[n - 1:][None])
        assert int(nacc[0]) == r["n_accepted"], step
        assert np.array_equal(out[0], r["out_tokens"]) and np.array_equal(path[0], r["path"]), step
        # every node's logits against the oracle's forward of its path
        errs = [0.0, 0.0]
        for i in range(n):
            anc = ancestors(parent, i)
            toks = np.array([tok[j] for j in anc], np.int32)
            want_t = ot.forward(toks, n0 - 1, n_logits=1)[0]
            rms = np.sqrt((want_t.astype(np.float64) ** 2).mean())
            errs[0] = max(errs[0], float(np.abs(tl[i] - want_t).max() / rms))
            if kids[i]:
                want_d = od.forward(np.concatenate([[seq[n0 - 2]], toks]).astype(np.int32), n0 - 2, n_logits=1)[0]
                rms = np.sqrt((want_d.astype(np.float64) ** 2).mean())
                errs[1] = max(errs[1], float(np.abs(dl[i] - want_d).max() / rms))
        a = r["n_accepted"]
        seq = seq + [int(t) for t in r["out_tokens"][:a + 1]]
        # the oracle caches take the committed tokens (all but the last, which is pending)
        ot.forward(np.array(seq[n0 - 1:len(seq) - 1], np.int32), n0 - 1)
        od.forward(np.array(seq[n0 - 2:len(seq) - 1], np.int32), n0 - 2)
        worst = max(worst, *errs)
        log(f"  tree step {step}: accepted {a} (path {list(r['path'][:a + 1])}), logits max err / rms "
            f"target {errs[0]:.2e} draft {errs[1]:.2e}")
    assert np.array_equal(sp.tokens(), np.array(seq, np.int32))
    assert worst <= logit_tol
    return seq, worst
