"""Writes tests/golden/golden.npz: small seeded cases of the path with the
oracle's outputs (oracle/, the C restatement), each cross-checked here
against an independent numpy float64 computation where one exists:
  - Q4_0 / Q4_K blocks and their decoded values (numpy decoder written from
    the GGUF block layouts),
  - the verify GEMM Y = X W^T in float64 (numpy product of the decoded
    weights and the fp16 activations),
  - causal and tree-masked attention in float64 (numpy softmax with the mask
    built from the parent array),
  - full-vocabulary, top-k / top-p and greedy draws and acceptance decisions
    (the oracle's exact integer rule; greedy cross-checked with numpy argmax).
Run from the repository root:  python tests/golden/make_golden.py
The fixtures are data (inputs and expected outputs); the GPU tests compare
the HIP path with them and the CPU tests re-derive them from the oracle."""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import oracle as ora  # noqa: E402

OUT = os.path.join(ROOT, "tests", "golden", "golden.npz")


def np_dequant_q4_0(b, n):
    blk = b.reshape(-1, 18)
    d = blk[:, :2].copy().view(np.float16).astype(np.float64)[:, 0]
    qs = blk[:, 2:]
    q = np.concatenate([qs & 15, qs >> 4], axis=1).astype(np.float64) - 8.0
    return (q * d[:, None]).reshape(-1)[:n]


def np_dequant_q4_k(b, n):
    blk = b.reshape(-1, 144)
    d = blk[:, 0:2].copy().view(np.float16).astype(np.float64)[:, 0]
    dmin = blk[:, 2:4].copy().view(np.float16).astype(np.float64)[:, 0]
    s = blk[:, 4:16].astype(np.int64)
    qs = blk[:, 16:].astype(np.int64)
    out = np.empty((blk.shape[0], 256))
    for j in range(8):
        if j < 4:
            sc, m = s[:, j] & 63, s[:, j + 4] & 63
        else:
            sc = (s[:, j + 4] & 15) | ((s[:, j - 4] >> 6) << 4)
            m = (s[:, j + 4] >> 4) | ((s[:, j] >> 6) << 4)
        c, hi = j // 2, j % 2
        q = (qs[:, 32 * c:32 * c + 32] >> (4 * hi)) & 15
        out[:, 32 * j:32 * j + 32] = d[:, None] * sc[:, None] * q - dmin[:, None] * m[:, None]
    return out.reshape(-1)[:n]


def np_attention(q, k, v, n_prefix, parent, scale):
    nq, H, D = q.shape
    L = n_prefix + nq
    qf, kf, vf = (ora.h2f_fast(a).astype(np.float64) for a in (q, k, v))
    vis = np.zeros((nq, L), bool)
    vis[:, :n_prefix] = True
    for i in range(nq):
        j = i
        while j >= 0:
            vis[i, n_prefix + j] = True
            j = parent[j] if parent is not None else j - 1
    out = np.empty((nq, H, D))
    for h in range(H):
        s = qf[:, h, :] @ kf[:L, h, :].T * scale
        s[~vis] = -np.inf
        p = np.exp(s - s.max(axis=1, keepdims=True))
        out[:, h, :] = (p / p.sum(axis=1, keepdims=True)) @ vf[:L, h, :]
    return out


def main():
    rng = np.random.default_rng(2024)
    g = {}
    # decode
    for t, dq in ((ora.Q4_0, np_dequant_q4_0), (ora.Q4_K, np_dequant_q4_k)):
        W = ora.synth_q4(t, 7, t, 8, 512, std=0.05)
        y = ora.dequantize(t, W, 8 * 512)
        assert np.array_equal(y.astype(np.float64), dq(W, 8 * 512)), t
        g[f"dec{t}_blocks"], g[f"dec{t}_values"] = W, y
    # verify GEMM
    for t, N, K, M in ((ora.Q4_0, 40, 1376, 5), (ora.Q4_K, 48, 512, 6)):
        W = ora.synth_q4(t, 11, 100 + t, N, K)
        X = ora.f2h_fast(rng.standard_normal((M, K)).astype(np.float32))
        Y = ora.q4_gemm_f64(t, W, N, K, X)
        wd = (np_dequant_q4_0 if t == ora.Q4_0 else np_dequant_q4_k)(W, N * K).reshape(N, K)
        ref = ora.h2f_fast(X).astype(np.float64) @ wd.T
        assert np.allclose(Y, ref, rtol=1e-12, atol=1e-12), t
        g[f"gemm{t}_W"], g[f"gemm{t}_X"], g[f"gemm{t}_Y"] = W, X, Y
    # attention: causal and tree
    H, D, P, nq = 4, 64, 40, 6
    q = ora.f2h_fast(rng.standard_normal((nq, H, D)).astype(np.float32))
    k = ora.f2h_fast(rng.standard_normal((P + nq, H, D)).astype(np.float32))
    v = ora.f2h_fast(rng.standard_normal((P + nq, H, D)).astype(np.float32))
    parent = np.array([-1, 0, 0, 1, 1, 2], np.int32)
    for name, par in (("causal", None), ("tree", parent)):
        o = ora.attention_f64(q, k, v, P, par, H, H, D, D ** -0.5)
        assert np.allclose(o, np_attention(q, k, v, P, par, D ** -0.5), rtol=1e-10, atol=1e-12), name
        g[f"attn_{name}_out"] = o
    g["attn_q"], g["attn_k"], g["attn_v"], g["attn_parent"] = q, k, v, parent
    # sampling and acceptance
    B, kk, V = 4, 3, 1001
    tl = (rng.standard_normal((B, kk + 1, V)) * 3).astype(np.float32)
    dl = (tl[:, :kk] + rng.standard_normal((B, kk, V))).astype(np.float32)
    u = ora.uniforms(99, 0, B * (kk + 1)).reshape(B, kk + 1)
    g["acc_tl"], g["acc_dl"], g["acc_u"] = tl, dl, u
    for name, s in (("full", ora.sampling(0.8)), ("topk", ora.sampling(0.8, top_k=20, top_p=0.9)),
                    ("greedy", ora.sampling(greedy=True))):
        flat = dl.reshape(B * kk, V)
        if s.greedy:
            dt = flat.argmax(axis=1).astype(np.int32).reshape(B, kk)
        else:
            dt = ora.sample(s, flat, ora.uniforms(5, 0, B * kk)).reshape(B, kk)
        out, nacc = ora.accept(s, tl, dl, dt, None if s.greedy else u)
        if s.greedy:  # accepted prefix = the drafts matching the target argmax, then the argmax
            am = tl.argmax(axis=2)
            for b in range(B):
                n = 0
                while n < kk and dt[b, n] == am[b, n]:
                    n += 1
                assert nacc[b] == n and np.array_equal(out[b, :n + 1], am[b, :n + 1]), b
        g[f"acc_{name}_dt"], g[f"acc_{name}_out"], g[f"acc_{name}_nacc"] = dt, out, nacc
        tok = ora.sample(s, tl.reshape(-1, V), u.reshape(-1))
        if s.greedy:
            assert np.array_equal(tok, tl.reshape(-1, V).argmax(axis=1))
        g[f"smp_{name}_tok"] = tok
    np.savez_compressed(OUT, **g)
    print(f"wrote {OUT}: {len(g)} arrays, {os.path.getsize(OUT)} bytes")


if __name__ == "__main__":
    main()
