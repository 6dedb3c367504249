"""ulspec_accept_noalloc against ulspec_accept, through the C ABI.

Bar: bit-exact.  The no-allocation entry point runs the same kernels as
ulspec_accept on the library's static per-GPU scratch, so for the same logits,
draft tokens and uniforms it must emit exactly ulspec_accept's tokens and
accepted counts (and the oracle's).  Each case makes two calls in a row on the
shared scratch, the second with a smaller input, so state left in the scratch
by the first call cannot leak into the second.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _logits(rng, shape, boost=8.0):
    x = (rng.standard_normal(shape) * 3.0).astype(np.float32)
    flat = x.reshape(-1, shape[-1])
    flat[np.arange(flat.shape[0]), rng.integers(0, shape[-1], flat.shape[0])] += boost
    return x


def _inputs(ora, so, rng, B, k, V):
    tl = _logits(rng, (B, k + 1, V))
    dl = (tl[:, :k] * 0.7 + _logits(rng, (B, k, V)) * 0.5).astype(np.float32)
    if so.greedy:
        dt = dl.reshape(B * k, V).argmax(axis=1).astype(np.int32).reshape(B, k)
        dt[0, k - 1] = (dt[0, k - 1] + 1) % V
        return tl, None, dt, None
    dt = ora.sample(so, dl.reshape(B * k, V), ora.uniforms(11, 0, B * k)).reshape(B, k)
    dt[B - 1, 0] = V + 3  # out of range: never accepted
    return tl, dl, dt, rng.random((B, k + 1)).astype(np.float32)


def _run(ctx, fn, s, tl, dl, dt, u):
    B, k1, V = tl.shape
    k = k1 - 1
    bufs = [ctx.upload(tl), ctx.upload(dl) if dl is not None else None, ctx.upload(dt.astype(np.int32)),
            ctx.upload(u) if u is not None else None, ctx.alloc(B * (k + 1) * 4), ctx.alloc(B * 4)]
    # poison the outputs: every entry must be written by the call
    ctx.copy_in(bufs[4], np.full((B, k + 1), -7, np.int32))
    ctx.copy_in(bufs[5], np.full((B,), -7, np.int32))
    fn(s, B, k, V, *bufs)
    out = ctx.download(bufs[4], np.int32, (B, k + 1))
    nacc = ctx.download(bufs[5], np.int32, (B,))
    for b in bufs:
        if b is not None:
            b.free()
    return out, nacc


MODES = {
    "topk40_topp09": ((0.8, 40, 0.9, False), 32000),
    # rows past the one-workgroup kernels' registers: the sampled chunk pipeline
    "topk40_topp09_v128256": ((0.8, 40, 0.9, False), 128256),
    "full_vocab": ((0.8, 0, 1.0, False), 32000),
    "greedy": ((1.0, 0, 1.0, True), 128256),
}


@pytest.mark.parametrize("mode", sorted(MODES))
def test_noalloc_matches_accept(ctx, ora, pkg, rng, mode):
    (T, tk, tp, greedy), V = MODES[mode]
    s = pkg.sampling(T, top_k=tk, top_p=tp, greedy=greedy)
    so = ora.sampling(T, top_k=tk, top_p=tp, greedy=greedy)
    for B, k, VV in ((16, 8, V), (4, 4, V // 3)):
        print(f"  {mode}: B={B} k={k} V={VV}", flush=True)
        tl, dl, dt, u = _inputs(ora, so, rng, B, k, VV)
        got = _run(ctx, ctx.accept_noalloc, s, tl, dl, dt, u)
        want = _run(ctx, ctx.accept, s, tl, dl, dt, u)
        assert np.array_equal(got[1], want[1]), (got[1], want[1])
        assert np.array_equal(got[0], want[0])
        ref_out, ref_nacc = ora.accept(so, tl, dl, dt, u)
        assert np.array_equal(got[1], ref_nacc) and np.array_equal(got[0], ref_out)
        assert got[1][B - 1] == 0 or greedy


def test_noalloc_rejects_oversize(ctx, pkg, rng):
    """B (2k+1) logit rows of top-k scratch beyond the static array: rejected
    before any launch, and the next call in range still works."""
    B, k, V = 16, 16, 1000
    s = pkg.sampling(0.8, top_k=40)
    tl = _logits(rng, (B, k + 1, V))
    dl = _logits(rng, (B, k, V))
    dt = np.zeros((B, k), np.int32)
    u = rng.random((B, k + 1)).astype(np.float32)
    bufs = [ctx.upload(tl), ctx.upload(dl), ctx.upload(dt), ctx.upload(u), ctx.alloc(B * (k + 1) * 4),
            ctx.alloc(B * 4)]
    with pytest.raises(pkg.UlspecError) as e:
        ctx.accept_noalloc(s, B, k, V, *bufs)
    assert e.value.status == pkg.EUNSUPPORTED
    assert "scratch" in str(e.value)
    ctx.accept_noalloc(s, 2, 4, V, *bufs)  # rows of the first two sequences, k = 4: in range
    for b in bufs:
        b.free()
