"""Pins of the oracle's F16 / Q8_0 / Q6_K decode (the GGUF types Q4_K_M files
mix in), CPU only.  Layouts restated from ggml's published block_q8_0 /
block_q6_K and dequantize_row_q6_K; neither ggml nor a GGUF fixture holding
these types is in this container, so the element order is pinned by closed
forms of that layout (which byte and bit feed which element), not by an
independent decoder."""
import numpy as np
import pytest

from llama_util import NumpyLlama, load, make_mixed_tensors


def _f16(x):
    return np.float32(np.float16(x))


def test_sizes(ora):
    assert (ora.row_bytes(ora.F16, 64), ora.row_bytes(ora.Q8_0, 64), ora.row_bytes(ora.Q6_K, 512)) == (128, 68, 420)
    assert ora.row_bytes(ora.Q8_0, 48) == 0 and ora.row_bytes(ora.Q6_K, 128) == 0


def test_f16_is_the_half(ora, rng):
    x = rng.standard_normal(64).astype(np.float16)
    assert np.array_equal(ora.dequantize(ora.F16, x.view(np.uint8), 64), x.astype(np.float32))


def test_q8_0_closed_form(ora):
    blk = np.zeros(34, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(0.25).tobytes(), np.uint8)
    q = np.array([-128, -127, -1, 0, 1, 2, 100, 127] * 4, np.int8)
    blk[2:] = q.view(np.uint8)
    assert np.array_equal(ora.dequantize(ora.Q8_0, blk, 32), 0.25 * q.astype(np.float32))


def _q6k_block(d, scales, ql, qh):
    b = np.zeros(210, np.uint8)
    b[0:128] = ql
    b[128:192] = qh
    b[192:208] = np.asarray(scales, np.int8).view(np.uint8)
    b[208:210] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
    return b


def test_q6_k_scale_groups_and_bias(ora):
    # all quants 0 -> q = -32 everywhere: element e = -32 d sc[e // 16]
    sc = np.array([1, -2, 3, -4, 5, 6, 7, 8, 9, 10, 11, 12, 127, -128, 0, 2], np.int8)
    y = ora.dequantize(ora.Q6_K, _q6k_block(0.5, sc, 0, 0), 256)
    want = np.repeat(-32.0 * 0.5 * sc.astype(np.float32), 16)
    assert np.array_equal(y, want)
    # all bits set -> q = 63 - 32 = 31
    y = ora.dequantize(ora.Q6_K, _q6k_block(0.5, sc, 255, 255), 256)
    assert np.array_equal(y, np.repeat(31.0 * 0.5 * sc.astype(np.float32), 16))


@pytest.mark.parametrize("half", [0, 1])
def test_q6_k_bit_to_element_map(ora, half):
    # flipping one bit moves exactly one element, the one the layout names:
    # ql[64h + l] low nibble -> 128h + l, high -> 128h + 64 + l;
    # ql[64h + 32 + l] low -> 128h + 32 + l, high -> 128h + 96 + l;
    # qh[32h + l] bits 2i, 2i+1 -> 128h + 32 i + l (weights 16, 32)
    sc = np.ones(16, np.int8)
    base = ora.dequantize(ora.Q6_K, _q6k_block(1.0, sc, 0, 0), 256)
    h = half
    for l in (0, 5, 17, 31):
        for byte, bit, elem, delta in [(64 * h + l, 0, 128 * h + l, 1), (64 * h + l, 4, 128 * h + 64 + l, 1),
                                       (64 * h + 32 + l, 1, 128 * h + 32 + l, 2),
                                       (64 * h + 32 + l, 7, 128 * h + 96 + l, 8)]:
            ql = np.zeros(128, np.uint8)
            ql[byte] = 1 << bit
            y = ora.dequantize(ora.Q6_K, _q6k_block(1.0, sc, ql, np.zeros(64, np.uint8)), 256)
            d = np.nonzero(y != base)[0]
            assert list(d) == [elem] and y[elem] - base[elem] == delta
        for i in range(4):
            for b in range(2):
                qh = np.zeros(64, np.uint8)
                qh[32 * h + l] = 1 << (2 * i + b)
                y = ora.dequantize(ora.Q6_K, _q6k_block(1.0, sc, np.zeros(128, np.uint8), qh), 256)
                d = np.nonzero(y != base)[0]
                assert list(d) == [128 * h + 32 * i + l] and y[d[0]] - base[d[0]] == 16 << b


# Q8_0: half a step of amax/127 plus 127 steps' worth of the fp16 rounding of
# d.  Q6_K: half a step of group-amax/31 plus 32 times the int8 rounding of the
# group scale (half of block-max/127 in units of d) plus the fp16 rounding of d.
@pytest.mark.parametrize("wtype,group,bound", [(8, 32, 0.5 / 127 + 2.0 ** -11),
                                               (14, 256, 0.5 / 31 + 32 * 0.5 / (31 * 127) + 2.0 ** -11)])
def test_quantize_round_trip(ora, rng, wtype, group, bound):
    x = (rng.standard_normal(256 * 8) * 0.02).astype(np.float32)
    y = ora.dequantize(wtype, ora.quantize(wtype, x), x.size)
    amax = np.repeat(np.abs(x.reshape(-1, group)).max(axis=1), group)
    assert np.all(np.abs(y - x) <= bound * amax + 1e-7)


def test_gemm_f64_matches_numpy_for_the_new_types(ora, rng):
    N, K, M = 8, 512, 3
    X = ora.f2h_fast((rng.standard_normal((M, K))).astype(np.float32))
    xf = ora.h2f_fast(X).astype(np.float64)
    for t in (ora.F16, ora.Q8_0, ora.Q6_K):
        w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
        W = ora.quantize(t, w.ravel())
        wd = ora.dequantize(t, W, N * K).reshape(N, K).astype(np.float64)
        Y = ora.q4_gemm_f64(t, W, N, K, X)
        assert np.allclose(Y, xf @ wd.T, rtol=1e-6, atol=1e-7)
        Y32 = ora.q4_gemm_f32(t, W, N, K, X)
        assert np.abs(Y32 - Y).max() <= 1e-5 * np.abs(Y).max() + 1e-6


def test_mixed_type_oracle_model_matches_numpy(ora):
    """The oracle model with Q6_K / Q8_0 / F16 / Q4_0 / Q4_K tensors side by
    side agrees with the independent float64 forward."""
    cfg = dict(dim=256, n_layers=2, n_heads=4, n_kv_heads=2, ffn=512, vocab=300, max_ctx=32, rms_eps=1e-5,
               rope_base=10000.0)
    t = make_mixed_tensors(ora, cfg, seed=7, std=0.05)
    m = ora.Llama(**cfg, nthreads=4)
    load(m, t)
    ref = NumpyLlama(ora, t, cfg)
    toks = [5, 17, 250, 3, 99]
    lo, lr = m.forward(toks, 0, n_logits=5), ref.forward(toks, 0)
    scale = np.sqrt((lr ** 2).mean())
    assert np.abs(lo - lr).max() <= 5e-3 * scale
