"""The GGUF types Q4_K_M files mix in (Q6_K, Q8_0, F16) on the GPU: the
dequant-GEMM against the oracle's float64 product (Q6_K natively, read back
bit for bit through unit rows), and a model whose
tensors mix all five types (one fused QKV weight mixing Q4_K and Q6_K) read
from a GGUF file against the oracle model.

Bar: the GEMM bound of test_gemm_gpu.py (1e-3 relative plus 1e-3 of the RMS;
the one fp16 rounding of a dequantized Q8_0 / Q6_K element is 2^-11 relative
and averages out over K), and the logits bound of test_gguf_gpu.py."""
import numpy as np
import pytest

import gguf_io as G
from llama_util import MIXED_TYPES, load, make_mixed_tensors, make_tensors

pytestmark = pytest.mark.gpu


def _gemm(ctx, wid, X, N):
    M = X.shape[0]
    xb, yb = ctx.upload(X), ctx.alloc(M * N * 4)
    ctx.verify_gemm(wid, xb, M, yb)
    y = ctx.download(yb, np.float32, (M, N))
    xb.free()
    yb.free()
    return y


def _close(y, ref):
    rms = float(np.sqrt(np.mean(ref ** 2)))
    err = np.abs(y.astype(np.float64) - ref)
    worst = float((err / (np.abs(ref) + rms)).max())
    print(f"  max rel err {worst:.3e}", flush=True)
    assert np.all(err <= 1e-3 * np.abs(ref) + 1e-3 * rms), worst


@pytest.mark.parametrize("wtype", [1, 8, 14], ids=["f16", "q8_0", "q6_k"])
@pytest.mark.parametrize("N,K,Ms", [(4096, 4096, (1, 6, 17)), (32000, 4096, (6,)), (100, 1536, (1, 3, 33)),
                                    (40, 512, (2, 65)), (2048, 11008, (9,))])
def test_gemm_matches_oracle(ctx, ora, rng, wtype, N, K, Ms):
    print(f"type {wtype} N {N} K {K}", flush=True)
    W = ora.synth_q4(wtype, 13, N + K, N, K)
    wid = ctx.weight_upload(wtype, W, N, K)
    assert ctx.weight_info(wid)[:3] == (wtype, N, K)
    for M in Ms:
        X = ora.f2h_fast(rng.standard_normal((M, K)).astype(np.float32))
        y = _gemm(ctx, wid, X, N)
        _close(y, ora.q4_gemm_f64(wtype, W, N, K, X))


@pytest.mark.parametrize("wtype", [1, 8], ids=["f16", "q8_0"])
def test_gemm_k_tail(ctx, ora, rng, wtype):
    """K = 1376 = 10.75 chunks of 128: the last chunk is a quarter full."""
    N, K = 72, 1376
    W = ora.synth_q4(wtype, 17, 3, N, K)
    wid = ctx.weight_upload(wtype, W, N, K)
    for M in (1, 5):
        X = ora.f2h_fast(rng.standard_normal((M, K)).astype(np.float32))
        _close(_gemm(ctx, wid, X, N), ora.q4_gemm_f64(wtype, W, N, K, X))


def test_f16_gemm_is_exact_in_the_weights(ctx, ora, rng):
    """F16 weights are taken as they are: with X = e_k rows the product reads
    back the weight columns bit for bit."""
    N, K = 48, 256
    W = (rng.standard_normal((N, K)) * 0.1).astype(np.float16)
    wid = ctx.weight_upload(1, W.view(np.uint8), N, K)
    ks = [0, 1, 7, 31, 32, 127, 128, 255]
    X = np.zeros((len(ks), K), np.float16)
    X[np.arange(len(ks)), ks] = 1
    y = _gemm(ctx, wid, X.view(np.uint16), N)
    assert np.array_equal(y, W[:, ks].T.astype(np.float32))


def _q6_k_fields(W, N, K):
    """q (0..63), int8 scale and fp16 d of every element of GGUF Q6_K rows
    (ggml's block_q6_K: ql[128] low nibbles, qh[64] 2-bit pairs, scales[16],
    d), as [N][K] arrays."""
    blk = W.reshape(N, K // 256, 210)
    i = np.arange(256)
    h, p = i // 128, i % 128
    quarter, l = p // 32, p % 32
    lo = blk[:, :, 64 * h + l + 32 * (quarter & 1)]
    lo = np.where(quarter < 2, lo & 15, lo >> 4).astype(np.int32)
    hb = ((blk[:, :, 128 + 32 * h + l] >> (2 * quarter)) & 3).astype(np.int32)
    sc = blk[:, :, 192 + i // 16].view(np.int8).astype(np.int32)
    d = np.ascontiguousarray(blk[:, :, 208:210]).view(np.float16)[..., 0]
    return (lo | (hb << 4)).reshape(N, K), sc.reshape(N, K), np.repeat(d, 256, axis=1).reshape(N, K)


def test_q6_k_gemm_reads_back_the_weights(ctx, ora, rng):
    """Native Q6_K: with X = e_k rows the product reads back each weight as
    f32(d) * f16((q - 32) sc), bit for bit -- exact wherever |(q - 32) sc|
    <= 2048, one fp16 rounding beyond -- on the whole-X path (M = 8) and the
    split-K path (M = 16).  The numpy decode is checked against the oracle's
    dequantization first."""
    N, K = 40, 512
    W = ora.synth_q4(14, 21, 3, N, K)
    W = W.reshape(N, K // 256, 210).copy()
    W[:5, :, 192:208] = rng.integers(-128, 128, (5, K // 256, 16)).astype(np.int8).view(np.uint8)  # large scales
    W = W.ravel()
    q, sc, d = _q6_k_fields(W, N, K)
    want_w = d.astype(np.float64) * sc * (q - 32)
    assert np.array_equal(ora.dequantize(14, W, N * K).reshape(N, K), want_w.astype(np.float32))
    wid = ctx.weight_upload(14, W, N, K)
    b16 = ((q - 32) * sc).astype(np.float16).astype(np.float32)
    want = d.astype(np.float32) * b16
    assert (np.abs((q - 32) * sc) > 2048).any()  # the rounded case is covered
    ks = np.array([0, 1, 7, 8, 15, 16, 31, 32, 63, 64, 100, 127, 128, 200, 255, 256,
                   257, 300, 383, 384, 400, 450, 500, 511])
    for M in (8, 16):
        for k0 in range(0, len(ks), M):
            kk = ks[k0:k0 + M]
            X = np.zeros((len(kk), K), np.float16)
            X[np.arange(len(kk)), kk] = 1
            y = _gemm(ctx, wid, X.view(np.uint16), N)
            assert np.array_equal(y, want[:, kk].T), (M, kk)


def test_f16_k_must_be_a_multiple_of_32(pkg, ctx):
    with pytest.raises(pkg.UlspecError) as e:
        ctx.weight_upload(1, np.zeros(4 * 48 * 2, np.uint8), 4, 48)
    assert e.value.status == pkg.EINVAL


CFG = dict(dim=256, n_layers=2, n_heads=4, n_kv_heads=2, ffn=512, vocab=1000, max_ctx=64, rms_eps=1e-5,
           rope_base=10000.0)


@pytest.fixture(scope="module")
def mixed_file(ora, tmp_path_factory):
    t = make_mixed_tensors(ora, CFG, seed=21)
    p = tmp_path_factory.mktemp("gguf") / "tiny_mixed.gguf"
    G.write(p, G.llama_kv(CFG), G.model_tensors(t))
    return p, t


def test_mixed_type_model_matches_oracle(pkg, ctx, ora, mixed_file):
    path, tensors = mixed_file
    assert {tensors[n][0] for n, _ in MIXED_TYPES} == {14, 8, 1, 2}
    print(f"  loading {path.name}", flush=True)
    fm = pkg.load_gguf_model(ctx, str(path))
    sm = pkg.Model(ctx, **CFG)
    load(sm, tensors)
    toks = np.random.default_rng(4).integers(0, CFG["vocab"], 12).astype(np.int32)
    lf, ls = fm.forward(toks, 0, n_logits=12), sm.forward(toks, 0, n_logits=12)
    assert np.array_equal(lf.view(np.uint32), ls.view(np.uint32))
    om = ora.Llama(**CFG, nthreads=ora.nthreads_default())
    load(om, tensors)
    lo = om.forward(toks, 0, n_logits=12)
    err = np.abs(lf.astype(np.float64) - lo).max() / np.sqrt((lo.astype(np.float64) ** 2).mean())
    print(f"  logits max err / rms vs oracle = {err:.2e}", flush=True)
    assert err <= 1e-2
    # decode continues on the cache the mixed weights wrote
    nxt = np.array([int(np.argmax(lo[-1]))], np.int32)
    lf2, lo2 = fm.forward(nxt, 12, n_logits=1), om.forward(nxt, 12, n_logits=1)
    err2 = np.abs(lf2.astype(np.float64) - lo2).max() / np.sqrt((lo2.astype(np.float64) ** 2).mean())
    assert err2 <= 1e-2
    fm.close()
    sm.close()


def test_mixed_type_speculative_loop(pkg, ctx, ora, mixed_file):
    """Mixed-type target with a Q4_K draft: the greedy loop commits what the
    target's own greedy decoding, one token at a time, produces."""
    path, tensors = mixed_file
    prompt = list(np.random.default_rng(8).integers(0, CFG["vocab"], 10))
    t = pkg.load_gguf_model(ctx, str(path))
    d = pkg.Model(ctx, **CFG)
    load(d, make_tensors(ora, CFG, 12, seed=22, norm_std=0.1))
    sp = pkg.Speculative(t, d, 3, pkg.sampling(greedy=True), 5)
    sp.prefill(np.array(prompt, np.int32))
    sp.generate(16)
    got = sp.tokens()
    ref = pkg.load_gguf_model(ctx, str(path))
    seq = list(prompt)
    ref.forward(np.array(seq[:-1], np.int32), 0)
    while len(seq) < len(got):
        lg = ref.forward(np.array(seq[-1:], np.int32), len(seq) - 1, n_logits=1)[0]
        seq.append(int(np.argmax(lg)))
    assert list(got) == seq
    for m in (sp, t, d, ref):
        m.close()


def test_mixed_type_batch_of_48_verify_rows(pkg, ctx, ora, mixed_file):
    """Mixed-type target (Q6_K LM head, Q8_0 O projection, fp16 fused and
    down weights, Q4_K elsewhere), 8 sequences x (k + 1) = 48 verify rows per
    step: every type's split-K GEMM at 6 column tiles of split X.  Every
    verify row's target logits within 2e-4 of their RMS (measured 1.8e-5) of a
    one-sequence
    GPU model's (whole-X kernels at 6 rows, the same fp16 copies of the mixed
    fused weights) and within 1e-2 of the oracle's forward (as for one
    sequence: those fp16 copies round); greedy tokens equal to the oracle's
    loop."""
    path, tensors = mixed_file
    B, k = 8, 5
    rng = np.random.default_rng(12)
    prompts = [rng.integers(0, CFG["vocab"], n).astype(np.int32) for n in (9, 14, 20, 11, 25, 7, 16, 30)]
    draft = make_tensors(ora, CFG, 12, seed=23, norm_std=0.1)
    t, d = pkg.Model(ctx, **CFG, n_seq=B), pkg.Model(ctx, **CFG, n_seq=B)
    load(t, tensors)
    load(d, draft)
    sp = pkg.Speculative(t, d, k, pkg.sampling(greedy=True), 5, n_seq=B)
    sp.prefill(prompts)
    ot, od = ora.Llama(**CFG, nthreads=ora.nthreads_default()), ora.Llama(**CFG, nthreads=ora.nthreads_default())
    load(ot, tensors)
    load(od, draft)
    ref = pkg.Model(ctx, **CFG)
    load(ref, tensors)
    seqs = [list(p) for p in prompts]
    worst, worst_gpu = 0.0, 0.0
    for _ in range(3):
        ns = [len(q) for q in seqs]
        sp.steps(1)
        r = sp.last_step()
        for b in range(B):
            n = ns[b]
            toks = np.concatenate([[seqs[b][n - 1]], r["draft_tokens"][b]]).astype(np.int32)
            got = r["target_logits"][b].astype(np.float64)
            ot.forward(np.array(seqs[b][:n - 1], np.int32), 0)
            want = ot.forward(toks, n - 1, n_logits=k + 1).astype(np.float64)
            worst = max(worst, float(np.abs(got - want).max() / np.sqrt((want ** 2).mean())))
            ref.forward(np.array(seqs[b][:n - 1], np.int32), 0)
            one = ref.forward(toks, n - 1, n_logits=k + 1).astype(np.float64)
            worst_gpu = max(worst_gpu, float(np.abs(got - one).max() / np.sqrt((one ** 2).mean())))
            seqs[b] += list(r["out_tokens"][b][:r["n_accepted"][b] + 1])
    print(f"  mixed types, 48 verify rows: target logits max err / rms vs one sequence {worst_gpu:.2e}, "
          f"vs the oracle {worst:.2e}")
    assert worst_gpu <= 2e-4 and worst <= 1e-2
    steps = sp.state()["steps"]
    for b in range(B):
        osp = ora.Speculative(ot, od, k, ora.sampling(greedy=True), 5)
        osp.prefill(prompts[b])
        for _ in range(steps):
            osp.step()
        assert np.array_equal(sp.tokens(seq=b), osp.tokens()), b
    for m in (sp, t, d, ot, od, ref):
        m.close()
