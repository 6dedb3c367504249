"""Tree verification on the GPU, through the C ABI: tree acceptance against
the oracle (bit-exact, as the chain rule), the forward of a draft tree
against causal oracle forwards of each root-to-node path, and the KV-cache
compaction that commits an accepted path.

Bars: acceptance tokens, paths and counts bit-exact; compaction moves rows
bit for bit; logits within 1e-2 of their RMS of the oracle's (the bar of the
model forward, see test_spec_gpu.py) with the same greedy argmax."""
import numpy as np
import pytest

from llama_util import load, make_tensors
from tree_util import path_to, random_tree

pytestmark = pytest.mark.gpu


def _logits(rng, shape, boost=8.0):
    x = (rng.standard_normal(shape) * 3.0).astype(np.float32)
    flat = x.reshape(-1, shape[-1])
    flat[np.arange(flat.shape[0]), rng.integers(0, shape[-1], flat.shape[0])] += boost
    return x


def _tree_inputs(ora, rng, s_ora, B, n, V, parent):
    tl = _logits(rng, (B, n, V))
    dl = (tl * 0.7 + _logits(rng, (B, n, V)) * 0.5).astype(np.float32)  # correlated draft
    tokens = np.zeros((B, n), np.int32)
    u_draw = ora.uniforms(99, 0, B * n).reshape(B, n)
    for b in range(B):
        for c in range(1, n):
            v = parent[c]
            if s_ora.greedy:  # half the children carry their parent's argmax
                tokens[b, c] = int(np.argmax(tl[b, v])) if rng.random() < 0.5 else int(rng.integers(0, V))
            else:  # siblings drawn from the parent's draft row
                tokens[b, c] = ora.sample(s_ora, dl[b, v][None], u_draw[b, c:c + 1])[0]
    u = rng.random((B, n)).astype(np.float32)
    return tl, dl, tokens, u


def _gpu_accept_tree(ctx, s, parent, tl, dl, tokens, u):
    B, n, V = tl.shape
    bufs = [ctx.upload(tl), ctx.upload(dl) if dl is not None else None, ctx.upload(tokens),
            ctx.upload(u) if u is not None else None, ctx.alloc(B * n * 4), ctx.alloc(B * n * 4), ctx.alloc(B * 4)]
    ctx.accept_tree(s, B, n, V, parent, *bufs)
    out = ctx.download(bufs[4], np.int32, (B, n))
    path = ctx.download(bufs[5], np.int32, (B, n))
    nacc = ctx.download(bufs[6], np.int32, (B,))
    for b in bufs:
        if b is not None:
            b.free()
    return out, path, nacc


@pytest.mark.parametrize("mode", ["topk", "full", "greedy", "large_topk"])
@pytest.mark.parametrize("V", [32000, 128256])
def test_accept_tree_bit_exact_with_oracle(ctx, ora, pkg, rng, mode, V):
    B, n = 4, 16
    args = {"topk": (0.8, 40, 0.9, False), "full": (0.8, 0, 1.0, False), "greedy": (1.0, 0, 1.0, True),
            "large_topk": (0.8, 2000, 0.9, False)}[mode]
    s = pkg.sampling(args[0], top_k=args[1], top_p=args[2], greedy=args[3])
    so = ora.sampling(args[0], top_k=args[1], top_p=args[2], greedy=args[3])
    for trial in range(2):
        parent = random_tree(rng, n)
        tl, dl, tokens, u = _tree_inputs(ora, rng, so, B, n, V, parent)
        if mode == "greedy":
            dl, u = None, None
        out, path, nacc = _gpu_accept_tree(ctx, s, parent, tl, dl, tokens, u)
        r_out, r_path, r_nacc = ora.accept_tree(so, parent, tl, dl, tokens, u)
        print(f"  {mode} V={V} tree {parent.tolist()} accepted {nacc.tolist()}")
        assert np.array_equal(nacc, r_nacc) and np.array_equal(out, r_out) and np.array_equal(path, r_path)


def test_accept_tree_on_a_chain_is_accept(ctx, ora, pkg, rng):
    B, k, V = 8, 6, 32000
    s = pkg.sampling(0.8, top_k=40, top_p=0.9)
    so = ora.sampling(0.8, top_k=40, top_p=0.9)
    parent = np.arange(-1, k, dtype=np.int32)
    tl, dl, tokens, u = _tree_inputs(ora, rng, so, B, k + 1, V, parent)
    out, path, nacc = _gpu_accept_tree(ctx, s, parent, tl, dl, tokens, u)
    bt, bd, bx, bu = ctx.upload(tl), ctx.upload(np.ascontiguousarray(dl[:, :k])), ctx.upload(tokens[:, 1:].copy()), \
        ctx.upload(u)
    bo, bn = ctx.alloc(B * (k + 1) * 4), ctx.alloc(B * 4)
    ctx.accept(s, B, k, V, bt, bd, bx, bu, bo, bn)
    assert np.array_equal(ctx.download(bo, np.int32, (B, k + 1)), out)
    assert np.array_equal(ctx.download(bn, np.int32, (B,)), nacc)
    for b in (bt, bd, bx, bu, bo, bn):
        b.free()


def test_accept_tree_rejects_bad_shapes(ctx, pkg):
    s = pkg.sampling(greedy=True)
    buf = ctx.alloc(4 * 32 * 8)
    for parent in ([0, 0, 1], [-1, 2, 0], [-1, -1, 0]):
        with pytest.raises(pkg.UlspecError):
            ctx.accept_tree(s, 1, 3, 8, parent, buf, None, buf, None, buf, buf, buf)
    with pytest.raises(pkg.UlspecError):
        ctx.accept_tree(s, 1, 17, 8, [-1] + list(range(16)), buf, None, buf, None, buf, buf, buf)
    buf.free()


# ---- tree forward and KV compaction on a tiny Llama --------------------------

CFG = dict(dim=512, n_layers=4, n_heads=8, n_kv_heads=4, ffn=1376, vocab=32000, max_ctx=128, rms_eps=1e-5,
           rope_base=10000.0)


@pytest.fixture(scope="module")
def models(pkg, ctx, ora):
    w = make_tensors(ora, CFG, 2, seed=303)
    g = pkg.Model(ctx, **CFG)
    load(g, w)
    o = ora.Llama(**CFG, nthreads=ora.nthreads_default())
    load(o, w)
    yield g, o
    g.close()
    o.close()


def _close(a, b):
    scale = np.sqrt((b.astype(np.float64) ** 2).mean())
    return np.abs(a.astype(np.float64) - b).max() / scale


def test_tree_forward_equals_path_forwards_then_compact(pkg, ctx, ora, rng, models):
    g, o = models
    P, n = 40, 12
    prompt = rng.integers(0, CFG["vocab"], P).astype(np.int32)
    g.forward(prompt, 0)
    o.forward(prompt, 0)
    parent = random_tree(rng, n)
    tokens = rng.integers(0, CFG["vocab"], n).astype(np.int32)
    lg = g.forward_tree(tokens, parent, P)
    worst = 0.0
    for i in range(n):
        p = path_to(parent, i)
        lo = o.forward(tokens[p], P, n_logits=1)[0]
        worst = max(worst, _close(lg[i], lo))
        assert int(np.argmax(lg[i])) == int(np.argmax(lo)), i
    print(f"  tree {parent.tolist()}: node logits max err / rms {worst:.2e}")
    assert worst <= 1e-2

    # commit the path to the deepest node: greedy tree acceptance on the
    # GPU's own logits with the children set to follow that path
    leaf = max(range(n), key=lambda i: (len(path_to(parent, i)), -i))
    keep = path_to(parent, leaf)
    L = CFG["n_layers"]
    before = [g.kv_io(l, 0, P, n) for l in range(L)]
    path = np.full(n, -1, np.int32)
    path[:len(keep)] = keep
    bp, bn = ctx.upload(path), ctx.upload(np.array([len(keep) - 1], np.int32))
    g.kv_compact(P, bp, bn, n)
    for l in range(L):
        k_after, v_after = g.kv_io(l, 0, P, n)
        kb, vb = before[l]
        assert np.array_equal(k_after[:len(keep)], kb[keep]) and np.array_equal(v_after[:len(keep)], vb[keep])
        assert np.array_equal(k_after[len(keep):], kb[len(keep):]) and np.array_equal(v_after[len(keep):], vb[len(keep):])
    bp.free()
    bn.free()
    # the compacted cache serves the next token like a causal forward of the path
    nxt = rng.integers(0, CFG["vocab"], 1).astype(np.int32)
    lg1 = g.forward(nxt, P + len(keep), n_logits=1)[0]
    o.forward(tokens[keep], P)
    lo1 = o.forward(nxt, P + len(keep), n_logits=1)[0]
    err = _close(lg1, lo1)
    print(f"  after compaction of path {keep}: next-token logits err / rms {err:.2e}")
    assert err <= 1e-2 and int(np.argmax(lg1)) == int(np.argmax(lo1))


def test_tree_step_greedy_accept_and_commit(pkg, ctx, ora, rng, models):
    """Forward a tree, accept it greedily on the device from the device
    logits, compact the cache from the device-written path, and compare the
    committed tokens with the oracle's tree rule on the same logits."""
    g, o = models
    P, n, V = 30, 10, CFG["vocab"]
    prompt = rng.integers(0, V, P).astype(np.int32)
    g.forward(prompt, 0)
    parent = random_tree(rng, n, branch=2)
    tokens = rng.integers(0, V, n).astype(np.int32)
    lg = g.forward_tree(tokens, parent, P)
    # children of the root take their parent's argmax where they can: a long accept
    for c in range(1, n):
        tokens[c] = int(np.argmax(lg[parent[c]])) if c % 3 else tokens[c]
    lg = g.forward_tree(tokens, parent, P)
    s = pkg.sampling(greedy=True)
    bt, bx = ctx.upload(lg[None]), ctx.upload(tokens[None])
    bo, bpth, bn = ctx.alloc(n * 4), ctx.alloc(n * 4), ctx.alloc(4)
    ctx.accept_tree(s, 1, n, V, parent, bt, None, bx, None, bo, bpth, bn)
    out = ctx.download(bo, np.int32, (n,))
    path = ctx.download(bpth, np.int32, (n,))
    nacc = int(ctx.download(bn, np.int32, (1,))[0])
    r_out, r_path, r_nacc = ora.accept_tree(ora.sampling(greedy=True), parent, lg[None], None, tokens[None], None)
    assert nacc == r_nacc[0] and np.array_equal(out, r_out[0]) and np.array_equal(path, r_path[0])
    before = g.kv_io(0, 0, P, n)
    g.kv_compact(P, bpth, bn, n)
    after = g.kv_io(0, 0, P, n)
    keep = list(path[:nacc + 1])
    assert np.array_equal(after[0][:nacc + 1], before[0][keep])
    print(f"  tree {parent.tolist()}: accepted {nacc}, path {[int(x) for x in keep]}, emitted {out[:nacc + 1].tolist()}")
    for b in (bt, bx, bo, bpth, bn):
        b.free()


def test_forward_tree_rejects_bad_input(pkg, models):
    g, _ = models
    with pytest.raises(pkg.UlspecError):
        g.forward_tree([1, 2, 3], [-1, 1, 0], 10)
    with pytest.raises(pkg.UlspecError):
        g.forward_tree([1, 2], [-1, 0], CFG["max_ctx"] - 1)
