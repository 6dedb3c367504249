"""Pins of the CPU oracle (no GPU).  Each test checks the oracle against
something it does not itself compute: numpy's IEEE conversions, float64
math, closed forms on hand-built GGUF blocks, brute force on small inputs,
or exact-probability theorems of the sampling rule."""
import math
from fractions import Fraction

import numpy as np
import pytest


# ---- fp16 ------------------------------------------------------------------

def test_h2f_matches_numpy_for_every_half(ora):
    h = np.arange(65536, dtype=np.uint16)
    f = ora.h2f(h)
    ref = h.view(np.float16).astype(np.float32)
    same = (f.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(f) & np.isnan(ref))
    assert same.all()


def test_f2h_round_to_nearest_even_matches_numpy(ora, rng):
    x = rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 20000)
    edge = np.array([65504, 65519.99, 65520, 1e-8, 2 ** -25, 2 ** -24, 3 * 2 ** -26, 2 ** -14,
                     2 ** -14 * (1 - 2 ** -11), -0.0, np.inf, -np.inf], np.float32)
    x = np.concatenate([x, edge])
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(ora.f2h(x), ref)
    assert np.array_equal(ora.f2h_fast(x), ref)


# ---- deterministic exp -------------------------------------------------------

def test_expf_within_one_ulp_of_float64(ora):
    x = np.linspace(-87.0, 88.0, 400001, dtype=np.float32)
    e = ora.expf(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    assert (np.abs(e - ref) / ulp).max() <= 1.0


def test_expf_special_values(ora):
    assert ora.expf(np.float32([0.0]))[0] == 1.0
    assert ora.expf(np.float32([-87.5]))[0] == 0.0
    assert np.isinf(ora.expf(np.float32([89.0]))[0])
    tiny = ora.expf(np.float32([-86.99]))[0]
    assert tiny > 0 and tiny >= np.finfo(np.float32).tiny  # never subnormal


# ---- counter-based uniforms / normals --------------------------------------

def test_uniforms_deterministic_and_uniform(ora):
    u = ora.uniforms(7, 0, 200000)
    assert np.array_equal(u, ora.uniforms(7, 0, 200000))
    assert np.array_equal(u[1000:1010], ora.uniforms(7, 1000, 10))
    assert u.min() >= 0.0 and u.max() < 1.0
    assert np.all((u * 2 ** 24) == np.floor(u * 2 ** 24))  # 24-bit grid
    hist = np.histogram(u, bins=20, range=(0, 1))[0]
    assert abs(hist - 10000).max() < 5 * math.sqrt(10000)


def test_normals_moments(ora):
    z = ora.normals(3, 4, 400000, 0.0, 2.0).astype(np.float64)
    assert abs(z.mean()) < 0.02 and abs(z.std() - 2.0) < 0.02


# ---- GGUF blocks ---------------------------------------------------------------

def _q40_block(d, qs):
    b = np.zeros(18, np.uint8)
    b[0:2] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
    b[2:] = qs
    return b


def test_type_table(ora):
    L = ora.lib()
    assert (L.ora_blck_size(2), L.ora_type_size(2)) == (32, 18)
    assert (L.ora_blck_size(12), L.ora_type_size(12)) == (256, 144)
    assert ora.row_bytes(2, 4096) == 4096 // 32 * 18
    assert ora.row_bytes(12, 11008) == 43 * 144


def test_q4_0_closed_form_decode(ora):
    # element j = low nibble of qs[j], element j+16 = high nibble, value (q-8)*d
    qs = np.array([(j & 15) | ((15 - j) << 4) for j in range(16)], np.uint8)
    d = 0.375
    y = ora.dequantize(2, _q40_block(d, qs), 32)
    expect = [(j - 8) * d for j in range(16)] + [(15 - j - 8) * d for j in range(16)]
    assert np.array_equal(y, np.array(expect, np.float32))


def test_q4_0_scale_edge_cases(ora):
    qs = np.full(16, 0x0F, np.uint8)  # low nibble 15 -> 7, high nibble 0 -> -8
    for d in (2.0 ** -24, 65504.0, -0.0, 0.0, 6.1e-5):
        y = ora.dequantize(2, _q40_block(d, qs), 32)
        dq = float(np.float16(d))
        assert np.array_equal(y[:16], np.full(16, np.float32(7 * dq)))
        assert np.array_equal(y[16:], np.full(16, np.float32(-8 * dq)))


def _pack_q4k_scales(sc, m):
    s = np.zeros(12, np.uint8)
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (m[j] & 63) | ((m[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((m[j + 4] & 15) << 4)
    return s


def test_q4_k_closed_form_decode(ora, rng):
    # hand-built block: known 6-bit scales/mins (incl. values >= 16 that use the
    # packed high bits) and known nibbles
    sc = np.array([1, 17, 33, 63, 5, 48, 0, 62])
    mm = np.array([63, 2, 40, 9, 31, 16, 57, 0])
    q = rng.integers(0, 16, 256)
    d, dmin = 0.0625, 0.5
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
    blk[2:4] = np.frombuffer(np.float16(dmin).tobytes(), np.uint8)
    blk[4:16] = _pack_q4k_scales(sc, mm)
    for c in range(4):
        blk[16 + 32 * c: 16 + 32 * c + 32] = q[64 * c: 64 * c + 32] | (q[64 * c + 32: 64 * c + 64] << 4)
    y = ora.dequantize(12, blk, 256)
    expect = np.array([d * sc[e // 32] * q[e] - dmin * mm[e // 32] for e in range(256)])
    assert np.array_equal(y.astype(np.float64), expect)


@pytest.mark.parametrize("wtype", [2, 12])
def test_quantize_round_trip_error_bound(ora, rng, wtype):
    x = rng.standard_normal(256 * 64).astype(np.float32) * 0.02
    y = ora.dequantize(wtype, ora.quantize(wtype, x), x.size)
    bs = 32
    for b in range(x.size // bs):
        xb, yb = x[b * bs:(b + 1) * bs].astype(np.float64), y[b * bs:(b + 1) * bs].astype(np.float64)
        err = np.abs(xb - yb)
        if wtype == 2:
            # grid step |d| = |max| / 8 (largest-magnitude element keeps its sign,
            # maps to q = 0); values round to the nearest step (<= d/2) except those
            # beyond +7d on the other side, which clamp to q = 15 (<= d); fp16
            # storage of d adds at most 8 * |d| * 2^-11
            d = np.abs(xb).max() / 8.0
            vmax = xb[np.argmax(np.abs(xb))]
            t = -xb / vmax * 8.0  # position on the grid in steps
            slack = 8 * d * 2.0 ** -11 + 1e-12
            assert np.all(err[t <= 7.5] <= 0.5 * d * (1 + 1e-6) + slack)
            assert np.all(err <= d * (1 + 1e-6) + slack)
        else:
            # affine sub-block step (max - min) / 15, widened by the 6-bit
            # rounding of the sub-scale and sub-min
            step = (xb.max() - min(0.0, xb.min())) / 15.0
            assert err.max() <= step * 1.6 + 1e-6


def test_grid_values_round_trip_exactly(ora):
    # values on the Q4_0 grid of an exactly representable d come back unchanged
    d = 0.25
    q = np.array([(j % 16) - 8 for j in range(32)] * 8, np.float32)
    q[::32] = -8  # make -8*d the largest magnitude so d = max / -8 = d
    x = q * d
    y = ora.dequantize(2, ora.quantize(2, x), x.size)
    assert np.array_equal(x, y)


def test_synth_matches_normals_then_quantize(ora):
    N, K = 8, 512
    for wtype in (2, 12):
        W = ora.synth_q4(wtype, 9, 5, N, K, std=0.02)
        x = ora.normals(9, 5, N * K, 0.0, 0.02)
        assert np.array_equal(W, ora.quantize(wtype, x))


# ---- dequant-GEMM ------------------------------------------------------------

@pytest.mark.parametrize("wtype", [2, 12])
def test_gemm_f64_equals_numpy_dequant_matmul(ora, rng, wtype):
    N, K, M = 40, 1024, 5
    W = ora.synth_q4(wtype, 1, 2, N, K)
    X = ora.f2h_fast(rng.standard_normal((M, K)).astype(np.float32))
    deq = ora.dequantize(wtype, W, N * K).reshape(N, K).astype(np.float64)
    ref = ora.h2f_fast(X).astype(np.float64) @ deq.T
    assert np.allclose(ora.q4_gemm_f64(wtype, W, N, K, X), ref, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("wtype", [2, 12])
def test_gemm_f32_baseline_within_fp32_tolerance(ora, rng, wtype):
    N, K, M = 96, 2048, 9
    W = ora.synth_q4(wtype, 3, 4, N, K)
    X = ora.f2h_fast(rng.standard_normal((M, K)).astype(np.float32))
    y64 = ora.q4_gemm_f64(wtype, W, N, K, X)
    y32 = ora.q4_gemm_f32(wtype, W, N, K, X, nthreads=4)
    rms = np.sqrt(np.mean(y64 ** 2))
    assert np.all(np.abs(y32 - y64) <= 1e-3 * np.abs(y64) + 1e-4 * rms)


# ---- attention -------------------------------------------------------------------

def _attn_inputs(rng, ora, n_prefix, nq, H, Hkv, D):
    L = n_prefix + nq
    q = ora.f2h_fast(rng.standard_normal((nq, H, D)).astype(np.float32))
    k = ora.f2h_fast(rng.standard_normal((L, Hkv, D)).astype(np.float32))
    v = ora.f2h_fast(rng.standard_normal((L, Hkv, D)).astype(np.float32))
    return q, k, v


def test_attention_single_visible_key_returns_v(ora, rng):
    # tree node with parent -1 and an empty prefix sees only itself
    q, k, v = _attn_inputs(rng, ora, 0, 3, 2, 2, 8)
    out = ora.attention_f64(q, k, v, 0, np.array([-1, -1, -1]), 2, 2, 8, 0.5)
    assert np.allclose(out, ora.h2f_fast(v).astype(np.float64), atol=0, rtol=0)


def test_attention_equal_scores_average_visible_values(ora, rng):
    _, k, v = _attn_inputs(rng, ora, 6, 2, 1, 1, 4)
    q = np.zeros((2, 1, 4), np.uint16)  # zero query: all scores 0
    out = ora.attention_f64(q, k, v, 6, None, 1, 1, 4, 1.0)
    vf = ora.h2f_fast(v).astype(np.float64)
    assert np.allclose(out[0, 0], vf[:7, 0].mean(axis=0), rtol=1e-12)
    assert np.allclose(out[1, 0], vf[:8, 0].mean(axis=0), rtol=1e-12)


def test_attention_causal_ignores_future_keys(ora, rng):
    q, k, v = _attn_inputs(rng, ora, 10, 4, 2, 1, 16)
    base = ora.attention_f64(q, k, v, 10, None, 2, 1, 16, 0.25)
    k2, v2 = k.copy(), v.copy()
    k2[12:] = ora.f2h_fast(rng.standard_normal(k2[12:].shape).astype(np.float32))
    v2[12:] = ora.f2h_fast(rng.standard_normal(v2[12:].shape).astype(np.float32))
    pert = ora.attention_f64(q, k2, v2, 10, None, 2, 1, 16, 0.25)
    assert np.array_equal(base[:2], pert[:2])
    assert not np.allclose(base[3], pert[3])


def test_attention_tree_ignores_non_ancestors_and_chain_equals_causal(ora, rng):
    q, k, v = _attn_inputs(rng, ora, 5, 6, 2, 2, 8)
    parent = np.array([-1, 0, 0, 1, 2, -1])
    base = ora.attention_f64(q, k, v, 5, parent, 2, 2, 8, 0.3)
    # node 3 sees 5 prefix keys + {0, 1, 3}; perturb node 2 and 4 and 5 keys
    k2, v2 = k.copy(), v.copy()
    for a in (2, 4, 5):
        k2[5 + a] ^= 0x0400
        v2[5 + a] ^= 0x0400
    pert = ora.attention_f64(q, k2, v2, 5, parent, 2, 2, 8, 0.3)
    assert np.array_equal(base[3], pert[3]) and np.array_equal(base[1], pert[1])
    chain = ora.attention_f64(q, k, v, 5, np.arange(-1, 5), 2, 2, 8, 0.3)
    causal = ora.attention_f64(q, k, v, 5, None, 2, 2, 8, 0.3)
    assert np.array_equal(chain, causal)


def test_attention_f64_brute_force_and_f32(ora, rng):
    H, Hkv, D, P, nq = 4, 2, 16, 20, 5
    q, k, v = _attn_inputs(rng, ora, P, nq, H, Hkv, D)
    out = ora.attention_f64(q, k, v, P, None, H, Hkv, D, 0.25)
    qf, kf, vf = (ora.h2f_fast(a).astype(np.float64) for a in (q, k, v))
    for i in range(nq):
        for h in range(H):
            s = 0.25 * (kf[:P + i + 1, h // 2] @ qf[i, h])
            p = np.exp(s - s.max())
            p /= p.sum()
            assert np.allclose(out[i, h], p @ vf[:P + i + 1, h // 2], rtol=1e-12, atol=1e-14)
    out32 = ora.attention_f32(q, k, v, P, None, H, Hkv, D, 0.25, nthreads=2)
    assert np.allclose(out32, out, rtol=1e-4, atol=1e-5)


# ---- acceptance sampling -----------------------------------------------------------

def test_warp_full_softmax_matches_float64(ora, rng):
    logits = (rng.standard_normal(1000) * 3).astype(np.float32)
    s = ora.sampling(0.8)
    E, Z, nk = ora.warp_row(s, logits)
    assert nk == 1000 and Z == int(E.sum())
    z = (logits.astype(np.float64) - logits.max()) / np.float64(np.float32(0.8))
    p = np.exp(z) / np.exp(z).sum()
    # fp32 exp (1 ulp) of an fp32-rounded argument: relative error ~ |z| * 2^-24
    assert np.allclose(E / Z, p, rtol=4e-6, atol=1e-14)
    assert ora.lib().ora_warp_shift(32000) == 48 and ora.lib().ora_warp_shift(128256) == 46


def test_warp_top_k_top_p_against_sort(ora, rng):
    logits = (rng.standard_normal(5000) * 3).astype(np.float32)
    logits[123] = logits[456] = logits.max() + 1  # a tie at the top
    s = ora.sampling(0.8, top_k=40, top_p=0.9)
    E, Z, nk = ora.warp_row(s, logits)
    order = sorted(range(5000), key=lambda i: (-float(logits[i]), i))[:40]
    z = (logits[order].astype(np.float64) - logits.max()) / np.float64(np.float32(0.8))
    w = np.exp(z)
    cum = np.cumsum(w) / w.sum()
    keep = int(np.searchsorted(cum, 0.9) + 1)  # smallest prefix with mass >= 0.9
    assert nk == keep
    assert set(np.nonzero(E)[0]) == set(order[:keep])
    assert E[123] == E[456] and Z == int(E.sum())


@pytest.mark.parametrize("top_k,top_p", [(300, 1.0), (2999, 1.0), (1500, 0.9), (1000, 0.3)])
def test_warp_large_top_k_against_sort(ora, rng, top_k, top_p):
    """top_k past the GPU's kept-list size (256): the kept set is the first
    top_k of (logit desc, index asc) order, ties at the cut included by
    lowest index, then the top-p prefix inside it, against a sorted walk."""
    V = 3000
    logits = (np.round(rng.standard_normal(V) * 6) / 2).astype(np.float32)  # many ties
    full, _, _ = ora.warp_row(ora.sampling(0.8), logits)
    E, Z, nk = ora.warp_row(ora.sampling(0.8, top_k=top_k, top_p=top_p), logits)
    order = sorted(range(V), key=lambda i: (-float(logits[i]), i))[:top_k]
    keep = len(order)
    if top_p < 1.0:
        thr = float(np.float32(top_p)) * float(sum(int(full[i]) for i in order))
        c = 0
        for t, i in enumerate(order):
            c += int(full[i])
            if float(c) >= thr:
                keep = t + 1
                break
    kept = order[:keep]
    assert nk == keep and Z == sum(int(full[i]) for i in kept)
    assert all(E[i] == full[i] for i in kept) and int(np.count_nonzero(E)) == int(np.count_nonzero(full[kept]))
    if top_k <= 1500:  # these cuts fall inside a run of equal logits (lower indices of that value kept first)
        assert logits[order[-1]] == logits[sorted(range(V), key=lambda i: (-float(logits[i]), i))[top_k]]


@pytest.mark.parametrize("kind", ["normal", "ties", "flat", "signed_zeros"])
def test_warp_top_p_without_top_k_is_the_shortest_prefix(ora, rng, kind):
    """Full-vocabulary top-p: the kept tokens are a prefix of (logit desc,
    index asc) order, their mass reaches top_p * Z (as doubles) and the prefix
    one shorter does not; kept tokens keep their full-warp weight."""
    V = 3000
    logits = (rng.standard_normal(V) * 3).astype(np.float32)
    if kind == "ties":
        logits = (np.round(logits * 2) / 2).astype(np.float32)
    elif kind == "flat":
        logits[:] = 0.75
    elif kind == "signed_zeros":
        logits[::2], logits[1::2] = 0.0, -0.0
        logits[17] = 0.5
    full, Zf, _ = ora.warp_row(ora.sampling(0.8), logits)
    order = sorted(range(V), key=lambda i: (-float(logits[i]), i))
    for tp in (0.0, 1e-6, 0.3, 0.9, 0.97):
        E, Z, nk = ora.warp_row(ora.sampling(0.8, top_p=tp), logits)
        kept = order[:nk]
        assert all(E[i] == full[i] for i in kept) and all(E[i] == 0 for i in order[nk:])
        mass = sum(int(full[i]) for i in kept)
        thr = float(np.float32(tp)) * float(Zf)
        assert Z == mass and float(mass) >= thr
        assert nk == 1 or float(mass - int(full[kept[-1]])) < thr


def test_cdf_pick_convention(ora):
    W = np.array([0, 3, 0, 5, 2], np.uint64)  # Z = 10
    # T = floor(u * 10); first i with T < cumsum -> [1,1,1,3,3,3,3,3,4,4]
    picks = [ora.cdf_pick(W, 10, u) for u in np.arange(10) / 10.0]
    assert picks == [1, 1, 1, 3, 3, 3, 3, 3, 4, 4]


def _tiny_dist(logits, s, ora):
    E, Z, _ = ora.warp_row(s, np.asarray(logits, np.float32))
    return [Fraction(int(e), Z) for e in E]


def test_accept_first_token_distribution_is_exactly_p(ora, rng):
    # Enumerate a fine uniform grid for (u_0, u_k): the emitted first token's
    # frequency equals p(x) exactly up to grid quantisation (k = 1, V = 5)
    V = 5
    tl = (rng.standard_normal((1, 2, V)) * 1.5).astype(np.float32)
    dl = (rng.standard_normal((1, 1, V)) * 1.5).astype(np.float32)
    s = ora.sampling(1.0)
    p = _tiny_dist(tl[0, 0], s, ora)
    q = _tiny_dist(dl[0, 0], s, ora)
    n = 64
    grid = (np.arange(n) + 0.5) / n
    counts = np.zeros(V)
    accepted = 0.0
    for x in range(V):  # draft token drawn from q: weight each x by q(x)
        for u0 in grid:
            us = np.stack([np.full(n, u0), grid], 1).astype(np.float32)
            T = np.repeat(tl, n, 0)
            D = np.repeat(dl, n, 0)
            out, nacc = ora.accept(s, T, D, np.full((n, 1), x, np.int32), us)
            for t in out[:, 0]:
                counts[t] += float(q[x]) / (n * n)
            accepted += float(q[x]) * float((nacc == 1).sum()) / (n * n)
    assert np.allclose(counts, [float(v) for v in p], atol=3.0 / n)
    # the accepted fraction for x ~ q is sum_x q(x) min(1, p(x)/q(x)) = sum min(p, q);
    # the u_0 grid quantises each x's acceptance to 1/n
    acc = sum(min(a, b) for a, b in zip(p, q))
    assert 0.05 < float(acc) < 0.95  # a case where both outcomes occur
    assert abs(accepted - float(acc)) <= 1.0 / n


def test_accept_equal_distributions_always_accept(ora, rng):
    V, k = 50, 4
    tl = (rng.standard_normal((3, k + 1, V)) * 3).astype(np.float32)
    dl = tl[:, :k].copy()
    s = ora.sampling(0.8, top_k=10, top_p=0.9)
    u = rng.random((3, k + 1)).astype(np.float32)
    dt = np.array([[int(np.argmax(tl[b, i])) for i in range(k)] for b in range(3)], np.int32)
    out, nacc = ora.accept(s, tl, dl, dt, u)
    assert np.all(nacc == k)
    assert np.array_equal(out[:, :k], dt)


def test_accept_zero_target_mass_rejects_and_resamples_from_p(ora, rng):
    V = 30
    tl = (rng.standard_normal((1, 2, V))).astype(np.float32)
    dl = np.full((1, 1, V), -50.0, np.float32)
    dl[0, 0, 7] = 50.0                       # q one-hot on 7
    tl[0, 0, 7] = -1000.0                    # p(7) = 0
    s = ora.sampling(1.0)
    for u0 in (0.0, 0.3, 0.999):
        out, nacc = ora.accept(s, tl, dl, np.array([[7]], np.int32), np.array([[u0, 0.42]], np.float32))
        assert nacc[0] == 0
        E, Z, _ = ora.warp_row(s, tl[0, 0])
        # residual max(0, p - q) is proportional to p here (q is one-hot on 7, p(7) = 0)
        assert out[0, 0] != 7 and E[out[0, 0]] > 0
        assert out[0, 0] == ora.cdf_pick(E, Z, 0.42)
        assert out[0, 1] == -1


def test_greedy_matches_brute_force_argmax_chain(ora, rng):
    V, k, B = 40, 5, 6
    tl = rng.standard_normal((B, k + 1, V)).astype(np.float32)
    tl[0, :, 3] = 10.0  # sequence 0: argmax 3 everywhere
    dt = rng.integers(0, V, (B, k)).astype(np.int32)
    dt[0] = 3
    s = ora.sampling(greedy=True)
    out, nacc = ora.accept(s, tl, None, dt, None)
    for b in range(B):
        n = 0
        while n < k and int(np.argmax(tl[b, n])) == dt[b, n]:
            n += 1
        assert nacc[b] == n
        emitted = list(dt[b, :n]) + [int(np.argmax(tl[b, n]))]
        assert list(out[b, :n + 1]) == emitted and all(out[b, n + 1:] == -1)
    assert nacc[0] == k and list(out[0]) == [3] * (k + 1)


def test_sample_statistics_chi_square(ora, rng):
    V = 16
    logits = (rng.standard_normal(V) * 2).astype(np.float32)
    s = ora.sampling(1.0)
    E, Z, _ = ora.warp_row(s, logits)
    n = 100000
    u = ora.uniforms(11, 0, n)
    toks = ora.sample(s, np.repeat(logits[None], n, 0), u)
    obs = np.bincount(toks, minlength=V)
    exp = E.astype(np.float64) / Z * n
    chi2 = float(((obs - exp) ** 2 / np.maximum(exp, 1e-9)).sum())
    assert chi2 < 50.0  # 15 dof: p ~ 1e-5 tail
