"""The committed golden fixtures (tests/golden/golden.npz, written by
tests/golden/make_golden.py): the oracle reproduces them exactly, and they
agree with the independent numpy float64 computations of make_golden.py."""
import importlib.util
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
_spec = importlib.util.spec_from_file_location("make_golden", os.path.join(HERE, "golden", "make_golden.py"))
mg = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(mg)


@pytest.fixture(scope="module")
def gold():
    with np.load(os.path.join(HERE, "golden", "golden.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_decode(ora, gold):
    for t, dq in ((ora.Q4_0, mg.np_dequant_q4_0), (ora.Q4_K, mg.np_dequant_q4_k)):
        W, y = gold[f"dec{t}_blocks"], gold[f"dec{t}_values"]
        assert np.array_equal(ora.synth_q4(t, 7, t, 8, 512, std=0.05), W)
        assert np.array_equal(ora.dequantize(t, W, y.size), y)
        assert np.array_equal(dq(W, y.size), y.astype(np.float64))


def test_gemm(ora, gold):
    for t, N, K in ((ora.Q4_0, 40, 1376), (ora.Q4_K, 48, 512)):
        W, X, Y = gold[f"gemm{t}_W"], gold[f"gemm{t}_X"], gold[f"gemm{t}_Y"]
        assert np.array_equal(ora.q4_gemm_f64(t, W, N, K, X), Y)
        wd = (mg.np_dequant_q4_0 if t == ora.Q4_0 else mg.np_dequant_q4_k)(W, N * K).reshape(N, K)
        assert np.allclose(ora.h2f_fast(X).astype(np.float64) @ wd.T, Y, rtol=1e-12, atol=1e-12)


def test_attention(ora, gold):
    q, k, v, par = gold["attn_q"], gold["attn_k"], gold["attn_v"], gold["attn_parent"]
    nq, H, D = q.shape
    P = k.shape[0] - nq
    for name, p in (("causal", None), ("tree", par)):
        o = gold[f"attn_{name}_out"]
        assert np.array_equal(ora.attention_f64(q, k, v, P, p, H, H, D, D ** -0.5), o)
        assert np.allclose(mg.np_attention(q, k, v, P, p, D ** -0.5), o, rtol=1e-10, atol=1e-12)


def test_sampling_and_acceptance(ora, gold):
    tl, dl, u = gold["acc_tl"], gold["acc_dl"], gold["acc_u"]
    V = tl.shape[-1]
    for name, s in (("full", ora.sampling(0.8)), ("topk", ora.sampling(0.8, top_k=20, top_p=0.9)),
                    ("greedy", ora.sampling(greedy=True))):
        dt = gold[f"acc_{name}_dt"]
        out, nacc = ora.accept(s, tl, dl, dt, None if s.greedy else u)
        assert np.array_equal(out, gold[f"acc_{name}_out"]) and np.array_equal(nacc, gold[f"acc_{name}_nacc"])
        assert np.array_equal(ora.sample(s, tl.reshape(-1, V), u.reshape(-1)), gold[f"smp_{name}_tok"])
    # greedy against numpy argmax
    assert np.array_equal(gold["smp_greedy_tok"], tl.reshape(-1, V).argmax(axis=1))
