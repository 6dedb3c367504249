"""K3 acceptance sampling on the GPU against the oracle (through the C ABI).

Bar: bit-exact.  Given the same logits, draft tokens and uniforms, the GPU
must emit exactly the oracle's tokens and accepted counts (the decision
arithmetic is exact fixed point, so no tolerance applies).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _logits(rng, shape, boost=8.0):
    """N(0, 3^2) with one random +boost token per row."""
    x = (rng.standard_normal(shape) * 3.0).astype(np.float32)
    flat = x.reshape(-1, shape[-1])
    flat[np.arange(flat.shape[0]), rng.integers(0, shape[-1], flat.shape[0])] += boost
    return x


def _draft_tokens(ora, s, dl, seed):
    B, k, V = dl.shape
    if s.greedy:
        return dl.reshape(B * k, V).argmax(axis=1).astype(np.int32).reshape(B, k)
    u = ora.uniforms(seed, 0, B * k)
    return ora.sample(s, dl.reshape(B * k, V), u).reshape(B, k)


def _run_gpu(ctx, s, tl, dl, dt, u):
    B, k1, V = tl.shape
    k = k1 - 1
    bt = ctx.upload(tl)
    bd = ctx.upload(dl) if dl is not None else None
    bx = ctx.upload(dt.astype(np.int32))
    bu = ctx.upload(u.astype(np.float32)) if u is not None else None
    bo = ctx.alloc(B * (k + 1) * 4)
    bn = ctx.alloc(B * 4)
    ctx.accept(s, B, k, V, bt, bd, bx, bu, bo, bn)
    out = ctx.download(bo, np.int32, (B, k + 1))
    nacc = ctx.download(bn, np.int32, (B,))
    for b in (bt, bd, bx, bu, bo, bn):
        if b is not None:
            b.free()
    return out, nacc


def _check(ctx, ora, pkg, s, tl, dl, dt, u):
    out, nacc = _run_gpu(ctx, s, tl, dl, dt, u)
    ref_out, ref_nacc = ora.accept(s, tl, dl, dt, u)
    assert np.array_equal(nacc, ref_nacc), (nacc, ref_nacc)
    assert np.array_equal(out, ref_out)
    return nacc


@pytest.mark.parametrize("k", [4, 8])
@pytest.mark.parametrize("V", [32000, 128256])
def test_accept_config_sampling_topk_topp(ctx, ora, pkg, rng, k, V):
    B = 16
    s = pkg.sampling(0.8, top_k=40, top_p=0.9)
    so = ora.sampling(0.8, top_k=40, top_p=0.9)
    tl = _logits(rng, (B, k + 1, V))
    dl = tl[:, :k] * 0.7 + _logits(rng, (B, k, V)) * 0.5  # correlated draft
    dl = dl.astype(np.float32)
    dt = _draft_tokens(ora, so, dl, 5)
    u = rng.random((B, k + 1)).astype(np.float32)
    nacc = _check(ctx, ora, pkg, s, tl, dl, dt, u)
    print(f"k={k} V={V} mean accepted {nacc.mean():.2f}")


@pytest.mark.parametrize("k", [4, 8])
@pytest.mark.parametrize("V", [32000, 128256])
def test_accept_config_greedy(ctx, ora, pkg, rng, k, V):
    B = 16
    s, so = pkg.sampling(greedy=True), ora.sampling(greedy=True)
    tl = _logits(rng, (B, k + 1, V))
    dt = tl[:, :k].argmax(axis=2).astype(np.int32)
    # break the chain at random positions
    cut = rng.integers(0, k + 1, B)
    for b in range(B):
        if cut[b] < k:
            dt[b, cut[b]] = (dt[b, cut[b]] + 1) % V
    nacc = _check(ctx, ora, pkg, s, tl, None, dt, None)
    assert np.array_equal(nacc, np.minimum(cut, k))


def test_accept_full_vocabulary(ctx, ora, pkg, rng):
    B, k, V = 6, 4, 32000
    s, so = pkg.sampling(0.8), ora.sampling(0.8)
    tl = _logits(rng, (B, k + 1, V), boost=2.0)
    dl = (tl[:, :k] + rng.standard_normal((B, k, V)).astype(np.float32)).astype(np.float32)
    dt = _draft_tokens(ora, so, dl, 9)
    for trial in range(4):
        u = rng.random((B, k + 1)).astype(np.float32)
        _check(ctx, ora, pkg, s, tl, dl, dt, u)


@pytest.mark.parametrize("V,k", [(32000, 16), (1001, 5), (128256, 3), (7, 2)])
def test_accept_full_vocabulary_edges(ctx, ora, pkg, rng, V, k):
    """Full vocabulary and greedy, rows split over many workgroups: an
    all-zero residual (draft row = target row, out-of-range draft token, so the
    draw falls back to the target row), zero draft mass at the drafted token,
    a row of equal logits, every draft accepted (bonus draw), u at 0 and just
    below 1."""
    B = 5
    tl = _logits(rng, (B, k + 1, V), boost=2.0)
    dl = (tl[:, :k] + 0.5 * rng.standard_normal((B, k, V))).astype(np.float32)
    dl[0] = tl[0, :k]
    tl[2, 0, :] = 0.75
    for T, greedy in ((0.8, False), (1.0, True)):
        s = pkg.sampling(T, greedy=greedy)
        so = ora.sampling(T, greedy=greedy)
        dt = _draft_tokens(ora, so, dl, 4)
        dt[0, 0] = V + 7
        dl_z = dl.copy()
        dl_z[1, 0, :] = -60.0
        dl_z[1, 0, int(dt[1, 0]) % V] = -1000.0
        dt_all = dt.copy()
        dt_all[4] = tl[4, :k].argmax(axis=1) if greedy else dt[4]
        for trial in range(3):
            u = rng.random((B, k + 1)).astype(np.float32)
            u[3, :] = 0.0 if trial == 0 else np.float32(1.0 - 2 ** -24)
            if trial == 2:
                u[4, :k] = 0.0  # every draft of sequence 4 accepted when its draft mass is positive
            _check(ctx, ora, pkg, s, tl, dl_z, dt_all, None if greedy else u)


def test_accept_edge_cases(ctx, ora, pkg, rng):
    # ties (every logit equal -> exact fallback of the top-k selection),
    # top_k >= V (full), top_k = 1, tiny top_p, k = 1 and k = 16, small V,
    # out-of-range draft tokens, draft token with zero draft mass
    cases = [
        dict(V=3000, k=3, s=(1.0, 40, 0.9), tie=True),
        dict(V=40, k=2, s=(0.8, 40, 1.0)),
        dict(V=5, k=1, s=(1.3, 0, 1.0)),
        dict(V=1000, k=16, s=(0.5, 1, 1.0)),
        dict(V=1000, k=5, s=(2.0, 200, 0.01)),
        dict(V=50000, k=6, s=(0.8, 256, 0.95)),
    ]
    for c in cases:
        V, k = c["V"], c["k"]
        B = 4
        T, tk, tp = c["s"]
        s, so = pkg.sampling(T, top_k=tk, top_p=tp), ora.sampling(T, top_k=tk, top_p=tp)
        tl = _logits(rng, (B, k + 1, V), boost=1.0)
        dl = _logits(rng, (B, k, V), boost=1.0)
        if c.get("tie"):
            tl[0] = 1.5
            dl[0] = 1.5
            tl[1, :, ::2] = 0.0
            tl[1, :, 1::2] = -0.0
        dt = _draft_tokens(ora, so, dl, 3)
        dt[2, 0] = V + 7          # out of range: never accepted
        dl[3, 0, :] = -60.0
        dl[3, 0, int(dt[3, 0])] = -1000.0  # zero draft mass at the drafted token
        u = rng.random((B, k + 1)).astype(np.float32)
        u[0, 0] = 0.0
        u[1, -1] = np.float32(1.0 - 2 ** -24)
        nacc = _check(ctx, ora, pkg, s, tl, dl, dt, u)
        assert nacc[2] == 0


TOPK_ROUTES = {1: "one 1024-thread workgroup per row", 2: "one 512-thread workgroup per row",
               3: "scanned chunk pipeline", 4: "sampled chunk pipeline"}


@pytest.fixture
def topk_route(ctx):
    """Force a top-k statistics route (ULSPEC_OPT_TOPK_ROUTE); automatic after."""
    def force(route):
        ctx.set_option(ctx.OPT_TOPK_ROUTE, route)
    yield force
    ctx.set_option(ctx.OPT_TOPK_ROUTE, 0)


@pytest.mark.parametrize("route", sorted(TOPK_ROUTES))
@pytest.mark.parametrize("B,k", [(2, 4), (16, 8)])
def test_accept_topk_ties_at_the_threshold(ctx, ora, pkg, rng, topk_route, route, B, k):
    # integer-valued logits, 300 tokens at each of the three largest values:
    # the one-workgroup-per-row kernels' candidate threshold lands on a value
    # ~900 tokens share (16 waves: the sorted, not the counted, candidate
    # list); with 8 waves they keep fewer maxima per row and the threshold
    # admits ~9800 tokens (the exact tie fallback); the scanned chunk
    # pipeline's threshold comes from its per-chunk wave maxima, the sampled
    # one's from an eighth of each row (~300 or ~600 tied candidates: the
    # sorted list).  Every route is forced
    # in turn, whatever the device's CU count.  Ties are broken by lowest
    # index, as in the oracle.
    V = 32000
    s, so = pkg.sampling(0.8, top_k=40, top_p=0.9), ora.sampling(0.8, top_k=40, top_p=0.9)

    def tied(shape):
        x = rng.integers(0, 7, size=shape).astype(np.float32)
        flat = x.reshape(-1, shape[-1])
        for row in flat:
            idx = rng.permutation(V)[:900]
            row[idx[:300]], row[idx[300:600]], row[idx[600:]] = 9.0, 8.0, 7.0
        return x

    topk_route(route)
    tl, dl = tied((B, k + 1, V)), tied((B, k, V))
    dt = _draft_tokens(ora, so, dl, 5)
    u = rng.random((B, k + 1)).astype(np.float32)
    _check(ctx, ora, pkg, s, tl, dl, dt, u)


@pytest.mark.parametrize("route", sorted(TOPK_ROUTES))
@pytest.mark.parametrize("V", [32000, 128256])
def test_accept_topk_routes_random_logits(ctx, ora, pkg, rng, topk_route, route, V):
    """N(0, 3^2) logits through each top-k route, forced: B = 32, k = 8 (544
    rows, more than twice the CUs of an MI355X: the automatic choice at V =
    32000 would be a chunk pipeline) and B = 16, k = 4; at V = 128256 (rows
    past the one-workgroup kernels' registers: routes 1 and 2 fall back to
    the sampled pipeline) B = 16, k = 8, and top_k 100 (a quarter of each row
    sampled) with k = 4."""
    s, so = pkg.sampling(0.8, top_k=40, top_p=0.9), ora.sampling(0.8, top_k=40, top_p=0.9)
    topk_route(route)
    if V == 128256:
        for B, k, tk in ((16, 8, 40), (16, 4, 100)):
            s, so = pkg.sampling(0.8, top_k=tk, top_p=0.9), ora.sampling(0.8, top_k=tk, top_p=0.9)
            tl = _logits(rng, (B, k + 1, V))
            dl = (tl[:, :k] * 0.7 + _logits(rng, (B, k, V)) * 0.5).astype(np.float32)
            dt = _draft_tokens(ora, so, dl, 5)
            u = rng.random((B, k + 1)).astype(np.float32)
            _check(ctx, ora, pkg, s, tl, dl, dt, u)
        return
    for B, k in ((32, 8), (16, 4)):
        tl = _logits(rng, (B, k + 1, V))
        dl = (tl[:, :k] * 0.7 + _logits(rng, (B, k, V)) * 0.5).astype(np.float32)
        dt = _draft_tokens(ora, so, dl, 5)
        u = rng.random((B, k + 1)).astype(np.float32)
        _check(ctx, ora, pkg, s, tl, dl, dt, u)


@pytest.mark.parametrize("V", [32000, 128256])
@pytest.mark.parametrize("top_k,top_p", [(257, 1.0), (1000, 0.9), (20000, 0.95), (5000, 1.0)])
def test_accept_large_top_k(ctx, ora, pkg, rng, V, top_k, top_p):
    """top_k past the kept-list size (256): the full-vocabulary kernels with a
    per-row bound (the order key of the k-th token, then the top-p prefix
    inside the top k), bit-exact with the oracle's sorted warp at the
    acceptance shapes (B = 16, k = 4)."""
    B, k = 16, 4
    s, so = pkg.sampling(0.8, top_k=top_k, top_p=top_p), ora.sampling(0.8, top_k=top_k, top_p=top_p)
    tl = _logits(rng, (B, k + 1, V), boost=2.0)
    dl = (tl[:, :k] * 0.7 + _logits(rng, (B, k, V), boost=2.0) * 0.5).astype(np.float32)
    dt = _draft_tokens(ora, so, dl, 5)
    dt[3, 0] = V + 7  # out of range: never accepted
    u = rng.random((B, k + 1)).astype(np.float32)
    nacc = _check(ctx, ora, pkg, s, tl, dl, dt, u)
    assert nacc[3] == 0
    R = 24
    logits = _logits(rng, (R, V), boost=3.0)
    uu = ora.uniforms(78, 0, R)
    bl, bu, bo = ctx.upload(logits), ctx.upload(uu), ctx.alloc(R * 4)
    ctx.sample(s, R, V, bl, bu, bo)
    assert np.array_equal(ctx.download(bo, np.int32, (R,)), ora.sample(so, logits, uu))
    for b in (bl, bu, bo):
        b.free()


@pytest.mark.parametrize("top_p", [1.0, 0.5])
def test_accept_large_top_k_ties_at_the_cut(ctx, ora, pkg, rng, top_p):
    """Integer-valued logits (every value shared by thousands of tokens): the
    k-th token falls inside a run of ties, which the bound cuts by lowest
    index; a row of equal logits; top_k = V - 1."""
    V, B, k = 32000, 4, 3
    for top_k in (1000, 4321, V - 1):
        s, so = pkg.sampling(1.0, top_k=top_k, top_p=top_p), ora.sampling(1.0, top_k=top_k, top_p=top_p)
        tl = rng.integers(-3, 4, size=(B, k + 1, V)).astype(np.float32)
        dl = rng.integers(-3, 4, size=(B, k, V)).astype(np.float32)
        tl[1] = 0.5
        dt = _draft_tokens(ora, so, dl, 6)
        u = rng.random((B, k + 1)).astype(np.float32)
        _check(ctx, ora, pkg, s, tl, dl, dt, u)


def test_sample_matches_oracle(ctx, ora, pkg, rng):
    for (T, tk, tp, greedy), V in [((0.8, 40, 0.9, False), 32000), ((1.0, 0, 1.0, False), 32000),
                                   ((1.0, 0, 1.0, True), 128256), ((0.7, 5, 1.0, False), 7),
                                   ((0.8, 0, 1.0, False), 128256), ((0.8, 0, 1.0, False), 1001),
                                   ((1.0, 0, 1.0, False), 7), ((1.0, 0, 1.0, True), 5), ((1.3, 0, 1.0, False), 16385)]:
        R = 24
        s, so = pkg.sampling(T, top_k=tk, top_p=tp, greedy=greedy), ora.sampling(T, top_k=tk, top_p=tp, greedy=greedy)
        logits = _logits(rng, (R, V), boost=3.0)
        u = ora.uniforms(77, 0, R)
        bl, bu, bo = ctx.upload(logits), ctx.upload(u), ctx.alloc(R * 4)
        ctx.sample(s, R, V, bl, bu, bo)
        got = ctx.download(bo, np.int32, (R,))
        assert np.array_equal(got, ora.sample(so, logits, u))
        for b in (bl, bu, bo):
            b.free()


def test_sample_full_vocabulary_edges(ctx, ora, pkg, rng):
    """Rows split over many workgroups: u at 0 and just below 1, rows with one
    dominant logit (all weight in one token, the rest underflow to 0), a row of
    equal logits and rows whose mass sits at either end of the vocabulary."""
    V = 32000
    s, so = pkg.sampling(0.8), ora.sampling(0.8)
    logits = _logits(rng, (8, V), boost=3.0)
    logits[2, :] = -1e4
    logits[2, 31999] = 50.0
    logits[3, :] = 0.25
    logits[4, :] = -1e4
    logits[4, 0] = 10.0
    logits[5, :] = -1e4
    logits[5, 17] = 10.0
    logits[5, 31990] = 10.0
    u = ora.uniforms(5, 0, 8)
    u[0] = 0.0
    u[1] = np.float32(1.0 - 2 ** -24)
    u[5] = np.float32(0.5)
    bl, bu, bo = ctx.upload(logits), ctx.upload(u), ctx.alloc(8 * 4)
    ctx.sample(s, 8, V, bl, bu, bo)
    got = ctx.download(bo, np.int32, (8,))
    assert np.array_equal(got, ora.sample(so, logits, u))
    assert got[2] == 31999 and got[4] == 0 and got[5] in (17, 31990)
    for b in (bl, bu, bo):
        b.free()


def test_uniforms_match_oracle(ctx, ora):
    n = 100003
    b = ctx.alloc(n * 4)
    ctx.uniforms(0xC0FFEE, 123456789, n, b)
    got = ctx.download(b, np.float32, (n,))
    assert np.array_equal(got.view(np.uint32), ora.uniforms(0xC0FFEE, 123456789, n).view(np.uint32))
    b.free()


def test_accept_argument_errors(ctx, pkg):
    b = ctx.alloc(1024)
    with pytest.raises(pkg.UlspecError) as e:
        ctx.accept(pkg.sampling(0.0), 1, 1, 10, b, b, b, b, b, b)
    assert e.value.status == pkg.EINVAL
    with pytest.raises(pkg.UlspecError) as e:
        ctx.accept(pkg.sampling(1.0), 1, 17, 10, b, b, b, b, b, b)
    assert e.value.status == pkg.EINVAL
    with pytest.raises(pkg.UlspecError) as e:
        ctx.accept(pkg.sampling(1.0, top_p=float("nan")), 1, 1, 1000, b, b, b, b, b, b)
    assert e.value.status == pkg.EINVAL
    # rows of one call: B (2k+1) and R at most 65535 (checked before any launch)
    with pytest.raises(pkg.UlspecError) as e:
        ctx.accept(pkg.sampling(1.0), 5000, 8, 1000, b, b, b, b, b, b)
    assert e.value.status == pkg.EUNSUPPORTED
    with pytest.raises(pkg.UlspecError) as e:
        ctx.sample(pkg.sampling(1.0), 70000, 1000, b, b, b)
    assert e.value.status == pkg.EUNSUPPORTED
    with pytest.raises(pkg.UlspecError) as e:
        ctx.set_option(ctx.OPT_TOPK_ROUTE, 5)
    assert e.value.status == pkg.EINVAL
    b.free()
