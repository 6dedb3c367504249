"""The HIP path against the committed golden fixtures (tests/golden/golden.npz):
the verify GEMM and attention within the tolerances of test_gemm_gpu.py and
test_attn_gpu.py, sampling and acceptance tokens bit-exact."""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def gold():
    with np.load(os.path.join(HERE, "golden", "golden.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_gemm_matches_golden(ctx, gold):
    for t, N, K in ((2, 40, 1376), (12, 48, 512)):
        W, X, Y = gold[f"gemm{t}_W"], gold[f"gemm{t}_X"], gold[f"gemm{t}_Y"]
        M = X.shape[0]
        wid = ctx.weight_upload(t, W, N, K)
        xb, yb = ctx.upload(X), ctx.alloc(M * N * 4)
        ctx.verify_gemm(wid, xb, M, yb)
        y = ctx.download(yb, np.float32, (M, N)).astype(np.float64)
        rms = np.sqrt(np.mean(Y ** 2))
        assert np.all(np.abs(y - Y) <= 1e-3 * np.abs(Y) + 1e-3 * rms), t
        xb.free()
        yb.free()


def test_attention_matches_golden(ctx, gold):
    q, k, v, par = gold["attn_q"], gold["attn_k"], gold["attn_v"], gold["attn_parent"]
    nq, H, D = q.shape
    P = k.shape[0] - nq
    bq, bk, bv, bo = ctx.upload(q), ctx.upload(k), ctx.upload(v), ctx.alloc(nq * H * D * 4)
    for name, p in (("causal", None), ("tree", par)):
        ctx.verify_attention(bq, bk, bv, P, nq, p, H, H, D, D ** -0.5, bo)
        o = ctx.download(bo, np.float32, (nq, H, D)).astype(np.float64)
        ref = gold[f"attn_{name}_out"]
        assert np.all(np.abs(o - ref) <= 1e-3 * np.abs(ref) + 1e-4), name
    for b in (bq, bk, bv, bo):
        b.free()


def test_sampling_and_acceptance_match_golden(pkg, ctx, gold):
    tl, dl, u = gold["acc_tl"], gold["acc_dl"], gold["acc_u"]
    B, k1, V = tl.shape
    k = k1 - 1
    bt, bd, bu = ctx.upload(tl), ctx.upload(dl), ctx.upload(u)
    bo, bn, bs = ctx.alloc(B * k1 * 4), ctx.alloc(B * 4), ctx.alloc(B * k1 * 4)
    for name, s in (("full", pkg.sampling(0.8)), ("topk", pkg.sampling(0.8, top_k=20, top_p=0.9)),
                    ("greedy", pkg.sampling(greedy=True))):
        bx = ctx.upload(gold[f"acc_{name}_dt"].astype(np.int32))
        ctx.accept(s, B, k, V, bt, bd, bx, bu, bo, bn)
        assert np.array_equal(ctx.download(bo, np.int32, (B, k1)), gold[f"acc_{name}_out"]), name
        assert np.array_equal(ctx.download(bn, np.int32, (B,)), gold[f"acc_{name}_nacc"]), name
        ctx.sample(s, B * k1, V, bt, bu, bs)
        assert np.array_equal(ctx.download(bs, np.int32, (B * k1,)), gold[f"smp_{name}_tok"]), name
        bx.free()
    for b in (bt, bd, bu, bo, bn, bs):
        b.free()
