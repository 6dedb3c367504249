"""Synthetic Llama-shaped models for the tests: GGUF tensors from the oracle's
seeded synthesizer, and an independent float64 numpy forward used to pin the
oracle's restatement."""
import numpy as np


def tensor_shapes(dim, n_layers, n_heads, n_kv_heads, ffn, vocab):
    """(name, ne0, ne1) of every quantized tensor, in synthesis-stream order."""
    D = dim // n_heads
    out = [("token_embd.weight", dim, vocab), ("output.weight", dim, vocab)]
    for l in range(n_layers):
        out += [(f"blk.{l}.attn_q.weight", dim, n_heads * D), (f"blk.{l}.attn_k.weight", dim, n_kv_heads * D),
                (f"blk.{l}.attn_v.weight", dim, n_kv_heads * D), (f"blk.{l}.attn_output.weight", n_heads * D, dim),
                (f"blk.{l}.ffn_gate.weight", dim, ffn), (f"blk.{l}.ffn_up.weight", dim, ffn),
                (f"blk.{l}.ffn_down.weight", ffn, dim)]
    return out


def make_tensors(ora, cfg, wtype, seed, std=0.02, norm_std=0.0):
    """name -> (ggml type, data, ne0, ne1).  Matrices: stream i of the seed;
    norm weights 1 (+ norm_std * N(0,1) from streams 1000+)."""
    dim, n_layers = cfg["dim"], cfg["n_layers"]
    t = {}
    for i, (name, ne0, ne1) in enumerate(tensor_shapes(**{k: cfg[k] for k in
                                                          ("dim", "n_layers", "n_heads", "n_kv_heads", "ffn",
                                                           "vocab")})):
        t[name] = (wtype, ora.synth_q4(wtype, seed, i, ne1, ne0, std), ne0, ne1)
    norm_names = ["output_norm.weight"] + [f"blk.{l}.{n}.weight" for l in range(n_layers)
                                           for n in ("attn_norm", "ffn_norm")]
    for j, name in enumerate(norm_names):
        w = np.ones(dim, np.float32)
        if norm_std:
            w = (w + norm_std * ora.normals(seed, 1000 + j, dim)).astype(np.float32)
        t[name] = (0, w, dim, 1)
    return t


def load(model, tensors):
    for name, (wtype, data, ne0, ne1) in tensors.items():
        model.set_tensor(name, wtype, data, ne0, ne1)


def _deq(ora, tensors, name):
    wtype, data, ne0, ne1 = tensors[name]
    if wtype == 0:
        return data.astype(np.float64)
    return ora.dequantize(wtype, data, ne0 * ne1).reshape(ne1, ne0).astype(np.float64)


def _f16(x):
    return np.asarray(x, np.float64).astype(np.float16).astype(np.float64)


class NumpyLlama:
    """Float64 forward with the same fp16 rounding points as the oracle -- the
    attention's inputs Q, K and V -- and unrounded activations everywhere else
    (independent code: matrix products, explicit softmax, closed-form RoPE)."""

    def __init__(self, ora, tensors, cfg):
        self.cfg = cfg
        self.W = {name: _deq(ora, tensors, name) for name in tensors}
        H, Hkv, dim = cfg["n_heads"], cfg["n_kv_heads"], cfg["dim"]
        self.D = dim // H
        self.kc = [np.zeros((cfg["max_ctx"], Hkv, self.D)) for _ in range(cfg["n_layers"])]
        self.vc = [np.zeros((cfg["max_ctx"], Hkv, self.D)) for _ in range(cfg["n_layers"])]

    def _norm(self, h, w):
        r = 1.0 / np.sqrt((h * h).sum(axis=1, keepdims=True) / h.shape[1] + self.cfg["rms_eps"])
        return h * r * w

    def _rope(self, x, pos):  # x [M][heads][D]
        D = self.D
        i = np.arange(D // 2)
        th = np.asarray(pos, np.float64)[:, None] * self.cfg["rope_base"] ** (-2.0 * i / D)[None, :]
        c = np.cos(th).astype(np.float32).astype(np.float64)[:, None, :]
        s = np.sin(th).astype(np.float32).astype(np.float64)[:, None, :]
        x0, x1 = x[..., 0::2], x[..., 1::2]
        y = np.empty_like(x)
        y[..., 0::2] = x0 * c - x1 * s
        y[..., 1::2] = x0 * s + x1 * c
        return y

    def forward(self, tokens, pos0):
        cfg, W, D = self.cfg, self.W, self.D
        H, Hkv = cfg["n_heads"], cfg["n_kv_heads"]
        M = len(tokens)
        pos = np.arange(pos0, pos0 + M)
        h = W["token_embd.weight"][np.asarray(tokens)]
        for l in range(cfg["n_layers"]):
            x = self._norm(h, W[f"blk.{l}.attn_norm.weight"])
            q = _f16(self._rope((x @ W[f"blk.{l}.attn_q.weight"].T).reshape(M, H, D), pos))
            k = _f16(self._rope((x @ W[f"blk.{l}.attn_k.weight"].T).reshape(M, Hkv, D), pos))
            v = _f16((x @ W[f"blk.{l}.attn_v.weight"].T).reshape(M, Hkv, D))
            self.kc[l][pos] = k
            self.vc[l][pos] = v
            att = np.zeros((M, H, D))
            for r in range(M):
                keys = self.kc[l][:pos[r] + 1]
                vals = self.vc[l][:pos[r] + 1]
                for hh in range(H):
                    g = hh // (H // Hkv)
                    s = keys[:, g, :] @ q[r, hh] / np.sqrt(D)
                    p = np.exp(s - s.max())
                    att[r, hh] = (p / p.sum()) @ vals[:, g, :]
            h = h + att.reshape(M, H * D) @ W[f"blk.{l}.attn_output.weight"].T
            x = self._norm(h, W[f"blk.{l}.ffn_norm.weight"])
            g = x @ W[f"blk.{l}.ffn_gate.weight"].T
            u = x @ W[f"blk.{l}.ffn_up.weight"].T
            a = g / (1.0 + np.exp(-g)) * u
            h = h + a @ W[f"blk.{l}.ffn_down.weight"].T
        x = self._norm(h, W["output_norm.weight"])
        return x @ W["output.weight"].T


# Tensors re-encoded as the other GGUF types a Q4_K_M file mixes in: Q6_K
# output and one V projection (so the fused QKV weight mixes types), Q8_0
# embedding, one up projection (mixed gate/up) and one output projection (a
# Q8_0 weight of its own), F16 down projection, Q4_0 query.
MIXED_TYPES = [("output.weight", 14), ("blk.0.attn_v.weight", 14), ("token_embd.weight", 8),
               ("blk.1.ffn_down.weight", 1), ("blk.0.ffn_up.weight", 8), ("blk.1.attn_q.weight", 2),
               ("blk.1.attn_output.weight", 8)]


def make_mixed_tensors(ora, cfg, seed, std=0.02, norm_std=0.1):
    t = make_tensors(ora, cfg, 12, seed, std=std, norm_std=norm_std)
    for name, nt in MIXED_TYPES:
        wt, d, ne0, ne1 = t[name]
        t[name] = (nt, ora.quantize(nt, ora.dequantize(wt, d, ne0 * ne1)), ne0, ne1)
    return t
