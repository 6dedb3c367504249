"""ctypes binding of the CPU oracle (oracle/_build/liboracle.so).

TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py.  The product never imports this module.
"""
import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# ORACLE_LIB selects another build of the same sources (the sanitizer build,
# oracle/_build/liboracle_san.so, under a preloaded ASan runtime).
LIB_PATH = os.environ.get("ORACLE_LIB") or os.path.join(_HERE, "_build", "liboracle.so")

F16, Q4_0, Q8_0, Q4_K, Q6_K = 1, 2, 8, 12, 14


def build():
    subprocess.run(["make", "-s", "-C", _HERE, "-B"], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            subprocess.run(["make", "-s", "-C", _HERE], check=True)
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


class Sampling(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_uint32), ("top_p", C.c_float), ("greedy", C.c_int32)]


class LlamaCfg(C.Structure):
    _fields_ = [("dim", C.c_int64), ("n_layers", C.c_int64), ("n_heads", C.c_int64), ("n_kv_heads", C.c_int64),
                ("ffn", C.c_int64), ("vocab", C.c_int64), ("max_ctx", C.c_int64),
                ("rms_eps", C.c_float), ("rope_base", C.c_float)]


class SpecState(C.Structure):
    _fields_ = [("n", C.c_int64), ("step", C.c_int64), ("accepted", C.c_int64), ("proposed", C.c_int64)]


P = C.c_void_p
I64 = C.c_int64


def _declare(L):
    def d(name, res, *args):
        f = getattr(L, name, None)
        if f is None:
            return
        f.restype = res
        f.argtypes = list(args)

    d("ora_h2f", C.c_float, C.c_uint16)
    d("ora_f2h", C.c_uint16, C.c_float)
    d("ora_mix64", C.c_uint64, C.c_uint64)
    d("ora_uniform", C.c_float, C.c_uint64, C.c_uint64)
    d("ora_uniforms", None, C.c_uint64, C.c_uint64, C.c_size_t, P)
    d("ora_normals", None, C.c_uint64, C.c_uint64, C.c_size_t, C.c_double, C.c_double, P, C.c_int)
    d("ora_expf", C.c_float, C.c_float)
    d("ora_blck_size", C.c_int, C.c_int)
    d("ora_type_size", C.c_int, C.c_int)
    d("ora_row_bytes", C.c_size_t, C.c_int, I64)
    d("ora_quantize", C.c_int, C.c_int, P, I64, P)
    d("ora_dequantize", C.c_int, C.c_int, P, I64, P)
    d("ora_synth_q4", C.c_int, C.c_int, C.c_uint64, C.c_uint64, I64, I64, C.c_double, P, C.c_int)
    d("ora_q4_gemm_f64", C.c_int, C.c_int, P, I64, I64, P, I64, P)
    d("ora_q4_gemm_f32", C.c_int, C.c_int, P, I64, I64, P, I64, P, C.c_int)
    d("ora_attention_f64", C.c_int, P, P, P, I64, I64, P, I64, I64, I64, C.c_float, P)
    d("ora_attention_f32", C.c_int, P, P, P, I64, I64, P, I64, I64, I64, C.c_float, P, C.c_int)
    d("ora_warp_row", I64, P, P, I64, P, P)
    d("ora_warp_shift", C.c_int, I64)
    d("ora_cdf_pick", I64, P, I64, C.c_uint64, C.c_float)
    d("ora_sample", C.c_int, P, I64, I64, P, P, P)
    d("ora_accept", C.c_int, P, I64, I64, I64, P, P, P, P, P, P, C.c_int)
    d("ora_accept_tree", C.c_int, P, I64, I64, I64, P, P, P, P, P, P, P, P, C.c_int)
    d("ora_llama_create", P, P, C.c_int)
    d("ora_llama_set_threads", None, P, C.c_int)
    d("ora_llama_free", None, P)
    d("ora_llama_set_tensor", C.c_int, P, C.c_char_p, C.c_int, P, C.c_size_t, I64, I64)
    d("ora_llama_forward", C.c_int, P, P, I64, I64, P, I64)
    d("ora_llama_kv_io", C.c_int, P, I64, C.c_int, I64, I64, P, P)
    d("ora_spec_prefill", C.c_int, P, P, P, I64, P, I64, P)
    d("ora_spec_step", C.c_int, P, P, P, I64, C.c_uint64, P, I64, P)
    d("ora_spec_generate", I64, P, P, P, I64, C.c_uint64, I64, P, I64, P)


def _p(a):
    return a.ctypes.data_as(C.c_void_p) if a is not None else None


# Worker threads are capped at 16: the host share of one GPU on the MI355X
# machines this runs on, whatever count the process is allowed to run on.
MAX_THREADS = 16


def host_cpus():
    """(nproc, the CPUs this process may run on, the threads the oracle uses)."""
    nproc = os.cpu_count() or 1
    try:
        allowed = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        allowed = nproc
    return nproc, allowed, max(1, min(MAX_THREADS, allowed))


def nthreads_default():
    return host_cpus()[2]


# ---- thin numpy wrappers -----------------------------------------------------

def f2h_fast(x):
    """fp32 -> fp16 bits, round to nearest even (numpy; equal to ora_f2h, tested)."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def h2f_fast(h):
    return np.asarray(h, dtype=np.uint16).view(np.float16).astype(np.float32)


def f2h(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    return np.array([lib().ora_f2h(float(v)) for v in x.ravel()], dtype=np.uint16).reshape(x.shape)


def h2f(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    return np.array([lib().ora_h2f(int(v)) for v in h.ravel()], dtype=np.float32).reshape(h.shape)


def expf(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    f = lib().ora_expf
    return np.array([f(float(v)) for v in x.ravel()], dtype=np.float32).reshape(x.shape)


def uniforms(seed, idx0, n):
    out = np.empty(n, dtype=np.float32)
    lib().ora_uniforms(seed, idx0, n, _p(out))
    return out


def normals(seed, stream, n, mean=0.0, std=1.0, nthreads=None):
    out = np.empty(n, dtype=np.float32)
    lib().ora_normals(seed, stream, n, mean, std, _p(out), nthreads or nthreads_default())
    return out


def row_bytes(wtype, k):
    return lib().ora_row_bytes(wtype, k)


def quantize(wtype, x):
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.empty(row_bytes(wtype, x.size), dtype=np.uint8)
    assert lib().ora_quantize(wtype, _p(x), x.size, _p(out)) == 0
    return out


def dequantize(wtype, b, n):
    b = np.ascontiguousarray(b, dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    assert lib().ora_dequantize(wtype, _p(b), n, _p(out)) == 0
    return out


def synth_q4(wtype, seed, stream, N, K, std=0.02, nthreads=None):
    out = np.empty(N * row_bytes(wtype, K), dtype=np.uint8)
    assert lib().ora_synth_q4(wtype, seed, stream, N, K, std, _p(out), nthreads or nthreads_default()) == 0
    return out


def q4_gemm_f64(wtype, W, N, K, X):
    X = np.ascontiguousarray(X, dtype=np.uint16)
    M = X.shape[0]
    Y = np.empty((M, N), dtype=np.float64)
    assert lib().ora_q4_gemm_f64(wtype, _p(np.ascontiguousarray(W)), N, K, _p(X), M, _p(Y)) == 0
    return Y


def q4_gemm_f32(wtype, W, N, K, X, nthreads=None):
    X = np.ascontiguousarray(X, dtype=np.uint16)
    M = X.shape[0]
    Y = np.empty((M, N), dtype=np.float32)
    assert lib().ora_q4_gemm_f32(wtype, _p(np.ascontiguousarray(W)), N, K, _p(X), M, _p(Y),
                                 nthreads or nthreads_default()) == 0
    return Y


def attention_f64(q, k, v, n_prefix, parent, H, Hkv, D, scale):
    q = np.ascontiguousarray(q, dtype=np.uint16)
    nq = q.size // (H * D)
    out = np.empty((nq, H, D), dtype=np.float64)
    par = None if parent is None else np.ascontiguousarray(parent, dtype=np.int32)
    rc = lib().ora_attention_f64(_p(q), _p(np.ascontiguousarray(k, dtype=np.uint16)),
                                 _p(np.ascontiguousarray(v, dtype=np.uint16)), n_prefix, nq, _p(par),
                                 H, Hkv, D, scale, _p(out))
    assert rc == 0
    return out


def attention_f32(q, k, v, n_prefix, parent, H, Hkv, D, scale, nthreads=None):
    q = np.ascontiguousarray(q, dtype=np.uint16)
    nq = q.size // (H * D)
    out = np.empty((nq, H, D), dtype=np.float32)
    par = None if parent is None else np.ascontiguousarray(parent, dtype=np.int32)
    rc = lib().ora_attention_f32(_p(q), _p(np.ascontiguousarray(k, dtype=np.uint16)),
                                 _p(np.ascontiguousarray(v, dtype=np.uint16)), n_prefix, nq, _p(par),
                                 H, Hkv, D, scale, _p(out), nthreads or nthreads_default())
    assert rc == 0
    return out


def sampling(temperature=1.0, top_k=0, top_p=1.0, greedy=False):
    return Sampling(temperature, top_k, top_p, 1 if greedy else 0)


def warp_row(s, logits):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    V = logits.size
    E = np.empty(V, dtype=np.uint64)
    Z = C.c_uint64(0)
    nk = lib().ora_warp_row(C.byref(s), _p(logits), V, _p(E), C.byref(Z))
    return E, int(Z.value), int(nk)


def cdf_pick(W, Z, u):
    W = np.ascontiguousarray(W, dtype=np.uint64)
    return int(lib().ora_cdf_pick(_p(W), W.size, Z, u))


def sample(s, logits, u):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    R, V = logits.shape
    out = np.empty(R, dtype=np.int32)
    uu = None if u is None else np.ascontiguousarray(u, dtype=np.float32)
    assert lib().ora_sample(C.byref(s), R, V, _p(logits), _p(uu), _p(out)) == 0
    return out


def accept(s, target, draft, draft_tokens, u, nthreads=None):
    target = np.ascontiguousarray(target, dtype=np.float32)
    B, k1, V = target.shape
    k = k1 - 1
    out = np.empty((B, k + 1), dtype=np.int32)
    nacc = np.empty(B, dtype=np.int32)
    dr = None if draft is None else np.ascontiguousarray(draft, dtype=np.float32)
    uu = None if u is None else np.ascontiguousarray(u, dtype=np.float32)
    rc = lib().ora_accept(C.byref(s), B, k, V, _p(target), _p(dr),
                          _p(np.ascontiguousarray(draft_tokens, dtype=np.int32)), _p(uu),
                          _p(out), _p(nacc), nthreads or nthreads_default())
    assert rc == 0
    return out, nacc


def accept_tree(s, parent, target, draft, tokens, u, nthreads=None):
    """Tree verification (ora_accept_tree): target / draft [B][n][V], tokens
    and uniforms [B][n] -> (tokens [B][n], path [B][n], n_accepted [B])."""
    target = np.ascontiguousarray(target, dtype=np.float32)
    B, n, V = target.shape
    out = np.empty((B, n), dtype=np.int32)
    path = np.empty((B, n), dtype=np.int32)
    nacc = np.empty(B, dtype=np.int32)
    dr = None if draft is None else np.ascontiguousarray(draft, dtype=np.float32)
    uu = None if u is None else np.ascontiguousarray(u, dtype=np.float32)
    rc = lib().ora_accept_tree(C.byref(s), B, n, V, _p(np.ascontiguousarray(parent, dtype=np.int32)), _p(target),
                               _p(dr), _p(np.ascontiguousarray(tokens, dtype=np.int32)), _p(uu), _p(out), _p(path),
                               _p(nacc), nthreads or nthreads_default())
    if rc != 0:
        raise ValueError("ora_accept_tree rejected its arguments")
    return out, path, nacc


class Llama:
    """CPU restatement of the Llama-shaped model (ora_llama)."""

    def __init__(self, dim, n_layers, n_heads, n_kv_heads, ffn, vocab, max_ctx, rms_eps=1e-5, rope_base=10000.0,
                 nthreads=8):
        self.cfg = LlamaCfg(dim, n_layers, n_heads, n_kv_heads, ffn, vocab, max_ctx, rms_eps, rope_base)
        self.handle = lib().ora_llama_create(C.byref(self.cfg), nthreads)
        if not self.handle:
            raise ValueError("ora_llama_create rejected the configuration")

    def set_threads(self, nthreads):
        lib().ora_llama_set_threads(self.handle, nthreads)

    def close(self):
        if self.handle:
            lib().ora_llama_free(self.handle)
            self.handle = None

    def __del__(self):
        self.close()

    def set_tensor(self, name, wtype, data, ne0, ne1):
        data = np.ascontiguousarray(data)
        if lib().ora_llama_set_tensor(self.handle, name.encode(), wtype, data.ctypes.data_as(P), data.nbytes,
                                      ne0, ne1):
            raise ValueError(f"ora_llama_set_tensor rejected {name}")

    def forward(self, tokens, pos, n_logits=0):
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.empty((n_logits, self.cfg.vocab), np.float32) if n_logits else None
        if lib().ora_llama_forward(self.handle, tokens.ctypes.data_as(P), len(tokens), pos,
                                   out.ctypes.data_as(P) if out is not None else None, n_logits):
            raise ValueError("ora_llama_forward failed")
        return out

    def kv_io(self, layer, dir, pos0, n, k=None, v=None):
        row = self.cfg.n_kv_heads * (self.cfg.dim // self.cfg.n_heads)
        if dir == 0:
            k = np.empty((n, row), np.uint16)
            v = np.empty((n, row), np.uint16)
        else:
            k = np.ascontiguousarray(k, dtype=np.uint16)
            v = np.ascontiguousarray(v, dtype=np.uint16)
        if lib().ora_llama_kv_io(self.handle, layer, dir, pos0, n, k.ctypes.data_as(P), v.ctypes.data_as(P)):
            raise ValueError("ora_llama_kv_io failed")
        return k, v


class Speculative:
    """CPU restatement of the speculative loop (ora_spec_*)."""

    def __init__(self, target, draft, k, s, seed, cap=None):
        self.target, self.draft, self.k, self.s, self.seed = target, draft, k, s, seed
        self.cap = cap or (min(target.cfg.max_ctx, draft.cfg.max_ctx) if draft is not None else target.cfg.max_ctx)
        self.seq = np.zeros(self.cap, np.int32)
        self.st = SpecState()

    def _dh(self):
        return self.draft.handle if self.draft is not None else None

    def prefill(self, prompt):
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        if lib().ora_spec_prefill(self.target.handle, self._dh(), prompt.ctypes.data_as(P), len(prompt),
                                  self.seq.ctypes.data_as(P), self.cap, C.byref(self.st)):
            raise ValueError("ora_spec_prefill failed")

    def step(self):
        if lib().ora_spec_step(self.target.handle, self._dh(), C.byref(self.s), self.k, self.seed,
                               self.seq.ctypes.data_as(P), self.cap, C.byref(self.st)):
            raise ValueError("ora_spec_step failed")

    def generate(self, n_new):
        n = lib().ora_spec_generate(self.target.handle, self._dh(), C.byref(self.s), self.k, self.seed, n_new,
                                    self.seq.ctypes.data_as(P), self.cap, C.byref(self.st))
        if n < 0:
            raise ValueError("ora_spec_generate failed")
        return n

    def state(self):
        return {"n": self.st.n, "steps": self.st.step, "accepted": self.st.accepted, "proposed": self.st.proposed}

    def tokens(self):
        return self.seq[:self.st.n].copy()
