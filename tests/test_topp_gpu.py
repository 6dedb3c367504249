"""Top-p over the whole vocabulary (top_p < 1, no top_k) on the GPU against the
oracle, through the C ABI: acceptance, sampling, tree acceptance and the
device loop.

Bar: bit-exact.  The kept prefix (logit desc, index asc; the shortest with
(double)mass >= (double)top_p * Z) is selected on the device by a radix
select on mass; the tokens, accepted counts and paths must equal the
oracle's, which walks a sorted copy of the row.  Cases: ties at the
boundary (logits rounded to halves), a row of equal logits (the boundary
falls inside one logit and is resolved by index), +0 / -0 rows, top_p of 0
(the first token alone), 1e-6, 0.5, 0.9, 0.999.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _logits(rng, shape, boost=8.0):
    x = (rng.standard_normal(shape) * 3.0).astype(np.float32)
    flat = x.reshape(-1, shape[-1])
    flat[np.arange(flat.shape[0]), rng.integers(0, shape[-1], flat.shape[0])] += boost
    return x


def _shape_rows(x, rng):
    """Plant the edge cases in the first rows of a [..., V] array."""
    flat = x.reshape(-1, x.shape[-1])
    if flat.shape[0] >= 4:
        flat[0] = np.round(flat[0] * 2) / 2          # many ties, also at the boundary
        flat[1] = 0.75                               # every logit equal
        flat[2, ::2], flat[2, 1::2] = 0.0, -0.0      # signed zeros
        flat[2, rng.integers(0, x.shape[-1])] = 0.5
        flat[3] = np.round(flat[3])                  # integer logits
    return x


def _accept(ctx, s, tl, dl, dt, u):
    B, k1, V = tl.shape
    k = k1 - 1
    bt, bd, bx, bu = ctx.upload(tl), ctx.upload(dl), ctx.upload(dt.astype(np.int32)), ctx.upload(u)
    bo, bn = ctx.alloc(B * (k + 1) * 4), ctx.alloc(B * 4)
    ctx.accept(s, B, k, V, bt, bd, bx, bu, bo, bn)
    out, nacc = ctx.download(bo, np.int32, (B, k + 1)), ctx.download(bn, np.int32, (B,))
    for b in (bt, bd, bx, bu, bo, bn):
        b.free()
    return out, nacc


@pytest.mark.parametrize("top_p", [0.5, 0.9, 0.999])
@pytest.mark.parametrize("k,V", [(4, 32000), (8, 128256), (3, 1001)])
def test_accept_top_p_only(ctx, ora, pkg, rng, top_p, k, V):
    B = 8
    s, so = pkg.sampling(0.8, top_p=top_p), ora.sampling(0.8, top_p=top_p)
    tl = _shape_rows(_logits(rng, (B, k + 1, V)), rng)
    dl = _shape_rows((tl[:, :k] * 0.7 + _logits(rng, (B, k, V)) * 0.5).astype(np.float32), rng)
    dt = ora.sample(so, dl.reshape(B * k, V), ora.uniforms(3, 0, B * k)).reshape(B, k)
    dt[B - 1, 0] = V + 2
    u = rng.random((B, k + 1)).astype(np.float32)
    out, nacc = _accept(ctx, s, tl, dl, dt, u)
    ref_out, ref_nacc = ora.accept(so, tl, dl, dt, u)
    print(f"  top_p={top_p} k={k} V={V}: accepted {nacc.tolist()}")
    assert np.array_equal(nacc, ref_nacc), (nacc, ref_nacc)
    assert np.array_equal(out, ref_out)


@pytest.mark.parametrize("V", [7, 1001, 32000, 128256])
def test_sample_top_p_only(ctx, ora, pkg, rng, V):
    R = 12
    logits = _shape_rows(_logits(rng, (R, V), boost=3.0), rng)
    for tp in (0.0, 1e-6, 0.5, 0.9, 0.999):
        s, so = pkg.sampling(0.8, top_p=tp), ora.sampling(0.8, top_p=tp)
        u = ora.uniforms(17, 0, R)
        u[5] = 0.0
        u[6] = np.float32(1.0 - 2 ** -24)
        bl, bu, bo = ctx.upload(logits), ctx.upload(u), ctx.alloc(R * 4)
        ctx.sample(s, R, V, bl, bu, bo)
        got = ctx.download(bo, np.int32, (R,))
        for b in (bl, bu, bo):
            b.free()
        assert np.array_equal(got, ora.sample(so, logits, u)), (V, tp)


def test_accept_tree_top_p_only(ctx, ora, pkg, rng):
    parent = np.array([-1, 0, 0, 1, 1, 2, 3, 3, 4, 5, 9, 6], np.int32)
    n, B, V = len(parent), 4, 32000
    for tp in (0.9, 0.5):
        s, so = pkg.sampling(0.8, top_p=tp), ora.sampling(0.8, top_p=tp)
        tl = _shape_rows(_logits(rng, (B, n, V)), rng)
        dl = _shape_rows((tl * 0.6 + _logits(rng, (B, n, V)) * 0.6).astype(np.float32), rng)
        tok = np.zeros((B, n), np.int32)
        for b in range(B):
            for i in range(1, n):
                tok[b, i] = ora.sample(so, dl[b, parent[i]][None], ora.uniforms(9, b * n + i, 1))[0]
        u = rng.random((B, n)).astype(np.float32)
        bt, bd, bx, bu = ctx.upload(tl), ctx.upload(dl), ctx.upload(tok), ctx.upload(u)
        bo, bp, bn = ctx.alloc(B * n * 4), ctx.alloc(B * n * 4), ctx.alloc(B * 4)
        ctx.accept_tree(s, B, n, V, parent, bt, bd, bx, bu, bo, bp, bn)
        out, path, nacc = (ctx.download(bo, np.int32, (B, n)), ctx.download(bp, np.int32, (B, n)),
                           ctx.download(bn, np.int32, (B,)))
        for b in (bt, bd, bx, bu, bo, bp, bn):
            b.free()
        ref_out, ref_path, ref_nacc = ora.accept_tree(so, parent, tl, dl, tok, u)
        assert np.array_equal(nacc, ref_nacc), (tp, nacc, ref_nacc)
        assert np.array_equal(path, ref_path) and np.array_equal(out, ref_out)
