"""K1 verify dequant-GEMM on the GPU against the oracle (through the C ABI).

Bar: fp32 accumulation, so |Y - Y_f64| <= 1e-3 * |Y_f64| + 1e-3 * rms(Y_f64)
elementwise (the 1e-3 relative of the fp32 tolerance), plus size-independent
properties at the full shapes: bitwise row independence across M, bitwise
run-to-run determinism, linearity in X.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _x(rng, ora, M, K):
    return ora.f2h_fast(rng.standard_normal((M, K)).astype(np.float32))


def _run(ctx, wid, X, N):
    M = X.shape[0]
    xb = ctx.upload(X)
    yb = ctx.alloc(M * N * 4)
    ctx.verify_gemm(wid, xb, M, yb)
    y = ctx.download(yb, np.float32, (M, N))
    xb.free()
    yb.free()
    return y


def _assert_close(y, ref):
    rms = float(np.sqrt(np.mean(ref ** 2)))
    err = np.abs(y.astype(np.float64) - ref)
    bound = 1e-3 * np.abs(ref) + 1e-3 * rms
    worst = float((err / (np.abs(ref) + rms)).max())
    print(f"  max rel err {worst:.3e}")
    assert np.all(err <= bound), f"max rel err {worst:.3e}"


CASES = [
    # (type, N, K, Ms) -- the dequant-GEMM shapes, plus tails
    (2, 4096, 4096, (1, 5, 9, 17)),
    (2, 11008, 4096, (1, 5, 9, 17)),
    (2, 4096, 11008, (1, 5, 9, 17)),
    (12, 4096, 4096, (1, 6, 17)),
    (12, 11008, 4096, (5, 48)),
    (12, 4096, 11008, (1, 6, 9, 16)),  # M >= 9: X past LDS, the split-K kernel
    (2, 100, 1376, (1, 3, 16, 33)),   # N % 16 != 0, K = 43 blocks (partial quad)
    (12, 40, 512, (2, 64, 65)),       # M > 64 splits into launches
    (2, 32000, 512, (5,)),            # LM-head shape of the small model
    (12, 11264, 2048, (1, 2, 6)),     # 704 tiles of <= 8 chunks: one-tile kernel (4 waves of 2 chunks), 2.75 tiles per CU
    (2, 16384, 1024, (1, 5)),         # 1024 tiles of 8 chunks: one-tile kernel, 4 tiles per CU
    (12, 11264, 2048, (8,)),          # 8 staged rows: the ring instead, 2 tiles per iteration
    (2, 8192, 1536, (1, 5)),          # 12 chunks: ring parts of 2 chunks, 2 tiles per iteration
    (12, 16384, 1536, (8,)),          # 6 chunks at 8 rows: ring parts of 2 chunks, 4 tiles per iteration
    (12, 22016, 4096, (1, 6)),        # the 7B gate/up: 5-6 ring iterations per CU in groups of 3, the
                                      # first iteration's weights issued ahead of X
    (12, 2048, 2048, (1, 2, 6)),      # 128 tiles of 8 chunks, fewer than CUs: the one-tile kernel too
]


@pytest.mark.parametrize("wtype,N,K,Ms", CASES)
def test_gemm_matches_oracle(ctx, ora, rng, wtype, N, K, Ms):
    W = ora.synth_q4(wtype, 11, N * 7 + K, N, K)
    wid = ctx.weight_upload(wtype, W, N, K)
    for M in Ms:
        X = _x(rng, ora, M, K)
        y = _run(ctx, wid, X, N)
        ref = ora.q4_gemm_f64(wtype, W, N, K, X)
        print(f"type {wtype} N {N} K {K} M {M}")
        _assert_close(y, ref)


@pytest.mark.parametrize("wtype", [2, 12])
def test_gemm_row_independence_and_determinism(ctx, ora, rng, wtype):
    # Rows are computed independently: within one kernel path (whole X in LDS
    # for small M, split-K for large M) row m is bitwise the same for every M;
    # across the two paths it agrees to fp32 rounding.  Repeated calls are
    # bitwise identical (fixed reduction order, no atomics).
    N, K = 4096, 11008 if wtype == 2 else 4096 * 2
    W = ora.synth_q4(wtype, 5, 99, N, K)
    wid = ctx.weight_upload(wtype, W, N, K)
    X = _x(rng, ora, 48, K)
    # largest M whose X fits in LDS: M * pitch <= 160 KiB - 16.5 KiB, pitch =
    # 2K rounded up to 1 KiB, + 16
    pitch = (2 * K + 1023) // 1024 * 1024 + 16
    m_small = min(16, (160 * 1024 - 16896) // pitch)
    small = _run(ctx, wid, X[:m_small], N)
    assert np.array_equal(small.view(np.uint32), _run(ctx, wid, X[:m_small], N).view(np.uint32))
    for M in (1, 2, 5):
        part = _run(ctx, wid, X[:M], N)
        assert np.array_equal(part.view(np.uint32), small[:M].view(np.uint32))
    big = _run(ctx, wid, X, N)
    assert np.array_equal(big.view(np.uint32), _run(ctx, wid, X, N).view(np.uint32))
    for M in (17, 33):
        part = _run(ctx, wid, X[:M], N)
        assert np.array_equal(part.view(np.uint32), big[:M].view(np.uint32))
    _assert_close(small, big[:m_small].astype(np.float64))


def test_gemm_linearity_full_shape(ctx, ora, rng):
    N, K = 4096, 11008
    W = ora.synth_q4(2, 8, 1, N, K)
    wid = ctx.weight_upload(2, W, N, K)
    # x2 = 2 * x1 exactly in fp16 -> y2 = 2 * y1 bitwise (power-of-two scaling)
    X1 = _x(rng, ora, 5, K)
    X2 = ora.f2h_fast(2.0 * ora.h2f_fast(X1))
    y1 = _run(ctx, wid, X1, N)
    y2 = _run(ctx, wid, X2, N)
    assert np.array_equal((2.0 * y1).view(np.uint32), y2.view(np.uint32))
    # additivity within fp32 rounding
    Xa = _x(rng, ora, 5, K)
    Xs = ora.f2h_fast(ora.h2f_fast(X1) + ora.h2f_fast(Xa))
    exact = ora.h2f_fast(Xs) == ora.h2f_fast(X1) + ora.h2f_fast(Xa)
    if exact.all():
        ya = _run(ctx, wid, Xa, N)
        ys = _run(ctx, wid, Xs, N)
        _assert_close(ys, (y1 + ya).astype(np.float64))


def test_gemm_closed_form_all_equal_nibbles(ctx, ora, rng):
    # every nibble q, every scale d  ->  Y[m][n] = (q - 8) * d * sum_k X[m][k]
    N, K = 64, 1024
    for q, d in ((3, 0.5), (15, 0.0078125), (0, 2.0)):
        blk = np.zeros(18, np.uint8)
        blk[0:2] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
        blk[2:] = q | (q << 4)
        W = np.tile(blk, N * K // 32)
        wid = ctx.weight_upload(2, W, N, K)
        X = _x(rng, ora, 5, K)
        y = _run(ctx, wid, X, N)
        rs = ora.h2f_fast(X).astype(np.float64).sum(axis=1)
        ref = np.repeat(((q - 8) * d * rs)[:, None], N, axis=1)
        _assert_close(y, ref)


def test_gemm_unit_rows_extract_columns(ctx, ora):
    # X = e_j picks weight column j: checks nibble order and scale placement
    for wtype in (2, 12):
        N, K = 48, 512
        W = ora.synth_q4(wtype, 3, 4, N, K)
        wid = ctx.weight_upload(wtype, W, N, K)
        ks = np.arange(0, K, 7)
        X = np.zeros((len(ks), K), np.uint16)
        X[np.arange(len(ks)), ks] = 0x3C00  # 1.0
        y = np.concatenate([_run(ctx, wid, X[i:i + 60], N) for i in range(0, len(ks), 60)])
        deq = ora.dequantize(wtype, W, N * K).reshape(N, K)
        assert np.array_equal(y, deq[:, ks].T)


def test_gemm_argument_errors(ctx, pkg, ora):
    W = ora.synth_q4(2, 1, 1, 16, 64)
    with pytest.raises(pkg.UlspecError) as e:
        ctx.weight_upload(2, W[:-1], 16, 64)
    assert e.value.status == pkg.EINVAL
    with pytest.raises(pkg.UlspecError) as e:
        ctx.weight_upload(2, W, 16, 48)
    assert e.value.status == pkg.EINVAL
    with pytest.raises(pkg.UlspecError) as e:
        ctx.weight_upload(3, W, 16, 64)
    assert e.value.status == pkg.EUNSUPPORTED
    with pytest.raises(pkg.UlspecError) as e:
        ctx.weight_upload(12, W, 16, 64)
    assert e.value.status == pkg.EINVAL
    wid = ctx.weight_upload(2, W, 16, 64)
    xb = ctx.alloc(64 * 2)
    yb = ctx.alloc(16 * 4)
    with pytest.raises(pkg.UlspecError) as e:
        ctx.verify_gemm(wid, xb, 0, yb)
    assert e.value.status == pkg.EINVAL
    with pytest.raises(pkg.UlspecError) as e:
        ctx.verify_gemm(wid + 1000, xb, 1, yb)
    assert e.value.status == pkg.EINVAL
