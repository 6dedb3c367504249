"""K2 verify attention on the GPU against the oracle (through the C ABI).

Bar: fp16 inputs, fp32 softmax: |O - O_f64| <= 1e-3 |O_f64| + 1e-4, plus
bitwise properties at the full shape (causal masking ignores future keys,
a chain tree equals the causal mask, repeated calls are identical).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def random_tree(rng, n, branching=3, depth=5):
    """Parent array (parent[i] < i, -1 = child of the prefix), each node has at
    most `branching` children and the tree at most `depth` levels."""
    parent = [-1]
    lvl = [1]
    kids = [0]
    roots = 1
    for i in range(1, n):
        cand = [j for j in range(i) if kids[j] < branching and lvl[j] < depth]
        if roots < branching:
            cand.append(-1)
        p = cand[rng.integers(0, len(cand))]
        parent.append(p)
        if p < 0:
            roots += 1
            lvl.append(1)
        else:
            kids[p] += 1
            lvl.append(lvl[p] + 1)
        kids.append(0)
    return np.array(parent, np.int32)


def _inputs(rng, ora, n_prefix, nq, H, Hkv, D):
    L = n_prefix + nq
    q = ora.f2h_fast(rng.standard_normal((nq, H, D)).astype(np.float32))
    k = ora.f2h_fast(rng.standard_normal((L, Hkv, D)).astype(np.float32))
    v = ora.f2h_fast(rng.standard_normal((L, Hkv, D)).astype(np.float32))
    return q, k, v


def _gpu(ctx, q, k, v, n_prefix, parent, H, Hkv, D, scale):
    nq = q.shape[0]
    bq, bk, bv, bo = ctx.upload(q), ctx.upload(k), ctx.upload(v), ctx.alloc(nq * H * D * 4)
    ctx.verify_attention(bq, bk, bv, n_prefix, nq, parent, H, Hkv, D, scale, bo)
    out = ctx.download(bo, np.float32, (nq, H, D))
    for b in (bq, bk, bv, bo):
        b.free()
    return out


def _close(out, ref):
    err = np.abs(out.astype(np.float64) - ref)
    worst = float((err / (np.abs(ref) + 0.1)).max())
    print(f"  max rel err {worst:.2e}")
    assert np.all(err <= 1e-3 * np.abs(ref) + 1e-4), worst


@pytest.mark.parametrize("mode", ["causal5", "tree16"])
def test_attention_config_shape(ctx, ora, rng, mode):
    H, D, P = 32, 128, 4096
    nq = 5 if mode == "causal5" else 16
    parent = None if mode == "causal5" else random_tree(rng, 16)
    q, k, v = _inputs(rng, ora, P, nq, H, H, D)
    scale = 1.0 / np.sqrt(D)
    out = _gpu(ctx, q, k, v, P, parent, H, H, D, scale)
    ref = ora.attention_f64(q, k, v, P, parent, H, H, D, scale)
    _close(out, ref)
    again = _gpu(ctx, q, k, v, P, parent, H, H, D, scale)
    assert np.array_equal(out.view(np.uint32), again.view(np.uint32))


@pytest.mark.parametrize("P,nq,H,Hkv,D", [
    (0, 1, 4, 4, 64), (0, 16, 2, 1, 128), (7, 3, 8, 2, 64), (63, 5, 8, 8, 128),
    (64, 6, 8, 8, 128), (250, 16, 6, 3, 64), (1000, 9, 4, 1, 128), (2047, 1, 16, 16, 64),
    (4096, 5, 8, 8, 64),  # 33 splits: the merge's 64-split instantiation
])
def test_attention_shapes(ctx, ora, rng, P, nq, H, Hkv, D):
    for parent in (None, random_tree(rng, nq)):
        q, k, v = _inputs(rng, ora, P, nq, H, Hkv, D)
        scale = 1.0 / np.sqrt(D)
        _close(_gpu(ctx, q, k, v, P, parent, H, Hkv, D, scale), ora.attention_f64(q, k, v, P, parent, H, Hkv, D, scale))


def test_attention_causal_ignores_future_and_chain_equals_causal(ctx, ora, rng):
    H, D, P, nq = 32, 128, 4096, 5
    q, k, v = _inputs(rng, ora, P, nq, H, H, D)
    base = _gpu(ctx, q, k, v, P, None, H, H, D, 0.088)
    k2, v2 = k.copy(), v.copy()
    k2[P + 3:] = ora.f2h_fast(rng.standard_normal(k2[P + 3:].shape).astype(np.float32))
    v2[P + 3:] = ora.f2h_fast(rng.standard_normal(v2[P + 3:].shape).astype(np.float32))
    pert = _gpu(ctx, q, k2, v2, P, None, H, H, D, 0.088)
    assert np.array_equal(base[:3].view(np.uint32), pert[:3].view(np.uint32))
    chain = _gpu(ctx, q, k, v, P, np.arange(-1, nq - 1, dtype=np.int32), H, H, D, 0.088)
    assert np.array_equal(base.view(np.uint32), chain.view(np.uint32))


def test_attention_one_visible_key_and_equal_scores(ctx, ora, rng):
    H, D = 4, 64
    q, k, v = _inputs(rng, ora, 0, 3, H, H, D)
    out = _gpu(ctx, q, k, v, 0, np.array([-1, -1, -1], np.int32), H, H, D, 0.125)
    assert np.array_equal(out, ora.h2f_fast(v).astype(np.float32))  # softmax over one key is exactly 1
    q0 = np.zeros_like(q)
    out = _gpu(ctx, q0, k, v, 0, None, H, H, D, 0.125)
    vf = ora.h2f_fast(v).astype(np.float64)
    for i in range(3):
        assert np.allclose(out[i], vf[:i + 1].mean(axis=0), rtol=1e-5, atol=1e-6)


def test_attention_argument_errors(ctx, pkg):
    b = ctx.alloc(1 << 16)
    for args, st in [((0, 17, None, 4, 4, 64), pkg.EINVAL), ((0, 2, None, 4, 3, 64), pkg.EINVAL),
                     ((0, 2, None, 4, 4, 96), pkg.EUNSUPPORTED), ((0, 2, np.array([0, 0], np.int32), 4, 4, 64), pkg.EINVAL)]:
        P, nq, parent, H, Hkv, D = args
        with pytest.raises(pkg.UlspecError) as e:
            ctx.verify_attention(b, b, b, P, nq, parent, H, Hkv, D, 0.1, b)
        assert e.value.status == st
    b.free()
