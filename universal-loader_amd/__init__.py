"""Python binding (ctypes) of libulspec, the gfx950 speculative-decoding
verification path.

Every call goes through the C ABI declared in include/ulspec.h and runs the
HIP kernels built into lib/libulspec.so.  There is no CPU fallback: if the
library is missing or no gfx950 device is present, the calls raise.

Import this directory as a package with load_package() (its name contains a
hyphen), e.g. from a test:

    import importlib.util, sys
    spec = importlib.util.spec_from_file_location(
        "universal_loader_amd", "<repo>/universal-loader_amd/__init__.py",
        submodule_search_locations=["<repo>/universal-loader_amd"])
"""
import ctypes as C
import os
import subprocess

import numpy as np

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "lib", "libulspec.so")
CSRC_DIR = os.path.join(PKG_DIR, "csrc")

F16 = 1
Q4_0 = 2
Q8_0 = 8
Q4_K = 12
Q6_K = 14

OK, EINVAL, ENOMEM, EDEVICE, EUNSUPPORTED = 0, 1, 2, 3, 4


class UlspecError(RuntimeError):
    def __init__(self, status, msg):
        super().__init__(f"ulspec status {status}: {msg}")
        self.status = status


def build(jobs=8, force=True):
    """Compile libulspec.so for gfx950 (hipcc cross-compiles without a GPU)."""
    args = ["make", "-s", "-C", CSRC_DIR, f"-j{jobs}"]
    if force:
        args.append("-B")
    subprocess.run(args, check=True)


class Sampling(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_uint32), ("top_p", C.c_float), ("greedy", C.c_int32)]


def sampling(temperature=1.0, top_k=0, top_p=1.0, greedy=False):
    return Sampling(temperature, top_k, top_p, 1 if greedy else 0)


class ModelCfg(C.Structure):
    _fields_ = [("dim", C.c_uint32), ("n_layers", C.c_uint32), ("n_heads", C.c_uint32), ("n_kv_heads", C.c_uint32),
                ("ffn", C.c_uint32), ("vocab", C.c_uint32), ("max_ctx", C.c_uint32), ("rms_eps", C.c_float),
                ("rope_base", C.c_float)]


_lib = None
P = C.c_void_p
U32 = C.c_uint32


def lib():
    """Load libulspec.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise UlspecError(EDEVICE, f"{LIB_PATH} not built; run __graft_entry__.build()")
        L = C.CDLL(LIB_PATH)
        _declare(L)
        _lib = L
    return _lib


# (name, restype, argtypes): every symbol include/ulspec.h declares
ABI = [
    ("ulspec_version", C.c_char_p, []),
    ("ulspec_ggml_blck_size", C.c_int, [U32]),
    ("ulspec_ggml_type_size", C.c_int, [U32]),
    ("ulspec_create", C.c_int, [C.c_int, C.POINTER(P)]),
    ("ulspec_destroy", None, [P]),
    ("ulspec_last_error", C.c_char_p, [P]),
    ("ulspec_status_str", C.c_char_p, [C.c_int]),
    ("ulspec_alloc", C.c_int, [P, C.c_size_t, C.POINTER(P)]),
    ("ulspec_free", C.c_int, [P, P]),
    ("ulspec_memcpy", C.c_int, [P, P, P, C.c_size_t, C.c_int]),
    ("ulspec_sync", C.c_int, [P]),
    ("ulspec_capture_begin", C.c_int, [P]),
    ("ulspec_capture_end", C.c_int, [P, C.POINTER(U32)]),
    ("ulspec_graph_replay", C.c_int, [P, U32, U32]),
    ("ulspec_graph_destroy", C.c_int, [P, U32]),
    ("ulspec_timer_mark", C.c_int, [P, U32]),
    ("ulspec_timer_elapsed_ms", C.c_int, [P, U32, U32, C.POINTER(C.c_float)]),
    ("ulspec_stream_read", C.c_int, [P, P, C.c_size_t, U32, P]),
    ("ulspec_set_option", C.c_int, [P, U32, C.c_int64]),
    ("ulspec_device_info", C.c_int, [P, C.POINTER(C.c_int), C.POINTER(C.c_int)]),
    ("ulspec_sync_probe", C.c_int, [P, U32, U32, U32, U32, C.POINTER(C.c_float), C.POINTER(U32)]),
    ("ulspec_weight_upload", C.c_int, [P, U32, P, C.c_size_t, U32, U32, C.POINTER(U32)]),
    ("ulspec_weight_info", C.c_int, [P, U32, C.POINTER(U32), C.POINTER(U32), C.POINTER(U32),
                                     C.POINTER(C.c_size_t)]),
    ("ulspec_verify_gemm", C.c_int, [P, U32, P, U32, P]),
    ("ulspec_verify_attention", C.c_int, [P, P, P, P, U32, U32, P, U32, U32, U32, C.c_float, P]),
    ("ulspec_accept", C.c_int, [P, C.POINTER(Sampling), U32, U32, U32, P, P, P, P, P, P]),
    ("ulspec_accept_noalloc", C.c_int, [P, C.POINTER(Sampling), U32, U32, U32, P, P, P, P, P, P]),
    ("ulspec_accept_tree", C.c_int, [P, C.POINTER(Sampling), U32, U32, U32, P, P, P, P, P, P, P, P]),
    ("ulspec_sample", C.c_int, [P, C.POINTER(Sampling), U32, U32, P, P, P]),
    ("ulspec_uniforms", C.c_int, [P, C.c_uint64, C.c_uint64, U32, P]),
    ("ulspec_synth_q4", C.c_int, [P, U32, C.c_uint64, C.c_uint64, U32, U32, C.c_float, P]),
    ("ulspec_model_create", C.c_int, [P, C.POINTER(ModelCfg), C.POINTER(P)]),
    ("ulspec_model_create_batch", C.c_int, [P, C.POINTER(ModelCfg), U32, C.POINTER(P)]),
    ("ulspec_model_forward_seq", C.c_int, [P, U32, P, U32, U32, P, U32]),
    ("ulspec_model_kv_io_seq", C.c_int, [P, U32, U32, C.c_int, U32, U32, P, P]),
    ("ulspec_model_destroy", None, [P]),
    ("ulspec_model_set_tensor", C.c_int, [P, C.c_char_p, U32, P, C.c_size_t, C.c_uint64, C.c_uint64, C.c_int]),
    ("ulspec_model_forward", C.c_int, [P, P, U32, U32, P, U32]),
    ("ulspec_model_kv_io", C.c_int, [P, U32, C.c_int, U32, U32, P, P]),
    ("ulspec_model_forward_tree", C.c_int, [P, P, P, U32, U32, P]),
    ("ulspec_model_kv_compact", C.c_int, [P, U32, P, P, U32]),
    ("ulspec_model_linear", C.c_int, [P, U32, U32, U32, U32]),
    ("ulspec_spec_create", C.c_int, [P, P, U32, C.POINTER(Sampling), C.c_uint64, C.POINTER(P)]),
    ("ulspec_spec_destroy", None, [P]),
    ("ulspec_spec_prefill", C.c_int, [P, P, U32]),
    ("ulspec_spec_steps", C.c_int, [P, U32]),
    ("ulspec_spec_generate", C.c_int, [P, U32, C.POINTER(U32)]),
    ("ulspec_spec_state", C.c_int, [P, C.POINTER(U32), C.POINTER(C.c_uint64), C.POINTER(C.c_uint64),
                                    C.POINTER(C.c_uint64)]),
    ("ulspec_spec_tokens", C.c_int, [P, U32, U32, P]),
    ("ulspec_spec_last_step", C.c_int, [P, P, P, P, P, P, P]),
    ("ulspec_spec_create_batch", C.c_int, [P, P, U32, C.POINTER(Sampling), C.c_uint64, U32, C.POINTER(P)]),
    ("ulspec_spec_prefill_batch", C.c_int, [P, P, P]),
    ("ulspec_spec_seq_state", C.c_int, [P, U32, C.POINTER(U32), C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]),
    ("ulspec_spec_seq_tokens", C.c_int, [P, U32, U32, U32, P]),
    ("ulspec_spec_create_tree", C.c_int, [P, P, U32, P, C.POINTER(Sampling), C.c_uint64, C.POINTER(P)]),
    ("ulspec_spec_tree_last_step", C.c_int, [P, P, P, P, P, P, P, P]),
    ("ulspec_spec_set_graph", C.c_int, [P, C.c_int]),
    ("ulspec_gguf_open", C.c_int, [C.c_char_p, C.POINTER(P), C.c_char_p, C.c_size_t]),
    ("ulspec_gguf_close", None, [P]),
    ("ulspec_gguf_last_error", C.c_char_p, [P]),
    ("ulspec_gguf_header", C.c_int, [P, C.POINTER(U32), C.POINTER(C.c_uint64), C.POINTER(C.c_uint64),
                                     C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]),
    ("ulspec_gguf_tensor", C.c_int, [P, C.c_uint64, C.POINTER(C.c_char_p), C.POINTER(U32), C.POINTER(U32),
                                     C.POINTER(C.c_uint64), C.POINTER(C.c_uint64), C.POINTER(C.c_uint64),
                                     C.POINTER(P)]),
    ("ulspec_gguf_find_tensor", C.c_int, [P, C.c_char_p, C.POINTER(C.c_uint64)]),
    ("ulspec_gguf_kv", C.c_int, [P, C.c_uint64, C.POINTER(C.c_char_p), C.POINTER(U32), C.POINTER(U32),
                                 C.POINTER(C.c_uint64)]),
    ("ulspec_gguf_kv_bytes", C.c_int, [P, C.c_uint64, C.POINTER(P), C.POINTER(C.c_uint64)]),
    ("ulspec_gguf_get_int", C.c_int, [P, C.c_char_p, C.POINTER(C.c_int64)]),
    ("ulspec_gguf_get_float", C.c_int, [P, C.c_char_p, C.POINTER(C.c_double)]),
    ("ulspec_gguf_get_str", C.c_int, [P, C.c_char_p, C.POINTER(P), C.POINTER(C.c_uint64)]),
    ("ulspec_gguf_llama_cfg", C.c_int, [P, U32, C.POINTER(ModelCfg)]),
    ("ulspec_model_load_gguf", C.c_int, [P, P, U32, C.POINTER(P)]),
    ("ulspec_model_load_gguf_batch", C.c_int, [P, P, U32, U32, C.POINTER(P)]),
]


def _declare(L):
    for name, res, args in ABI:
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args


class DeviceBuffer:
    """A device allocation made through ulspec_alloc on one context."""

    def __init__(self, ctx, nbytes):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        p = P()
        ctx._check(lib().ulspec_alloc(ctx.handle, max(1, self.nbytes), C.byref(p)))
        self.ptr = p.value

    def free(self):
        if self.ptr:
            self.ctx._check(lib().ulspec_free(self.ctx.handle, self.ptr))
            self.ptr = None

    def __int__(self):
        return self.ptr


class Context:
    """ulspec_ctx: one device, one HIP stream."""

    def __init__(self, device=0):
        h = P()
        st = lib().ulspec_create(device, C.byref(h))
        if st != OK:
            raise UlspecError(st, f"ulspec_create(device={device}) failed: "
                                  f"{lib().ulspec_status_str(st).decode()}")
        self.handle = h.value
        self._bufs = []

    def close(self):
        if self.handle:
            for b in self._bufs:
                b.ptr = None
            lib().ulspec_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def _check(self, st):
        if st != OK:
            raise UlspecError(st, lib().ulspec_last_error(self.handle).decode())

    # -- memory --------------------------------------------------------------
    def alloc(self, nbytes):
        b = DeviceBuffer(self, nbytes)
        return b

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        b = DeviceBuffer(self, arr.nbytes)
        if arr.nbytes:
            self._check(lib().ulspec_memcpy(self.handle, b.ptr, arr.ctypes.data_as(P), arr.nbytes, 0))
        return b

    def download(self, buf, dtype, shape):
        out = np.empty(shape, dtype=dtype)
        if out.nbytes:
            self._check(lib().ulspec_memcpy(self.handle, out.ctypes.data_as(P), buf.ptr if hasattr(buf, "ptr")
                                            else int(buf), out.nbytes, 1))
        return out

    def copy_in(self, buf, arr, offset=0):
        arr = np.ascontiguousarray(arr)
        self._check(lib().ulspec_memcpy(self.handle, int(buf.ptr) + offset, arr.ctypes.data_as(P), arr.nbytes, 0))

    def sync(self):
        self._check(lib().ulspec_sync(self.handle))

    # -- capture / timing ------------------------------------------------------
    def capture_begin(self):
        self._check(lib().ulspec_capture_begin(self.handle))

    def capture_end(self):
        g = U32()
        self._check(lib().ulspec_capture_end(self.handle, C.byref(g)))
        return g.value

    def graph_replay(self, gid, times=1):
        self._check(lib().ulspec_graph_replay(self.handle, gid, times))

    def graph_destroy(self, gid):
        self._check(lib().ulspec_graph_destroy(self.handle, gid))

    def timer_mark(self, slot):
        self._check(lib().ulspec_timer_mark(self.handle, slot))

    def timer_elapsed_ms(self, a, b):
        ms = C.c_float()
        self._check(lib().ulspec_timer_elapsed_ms(self.handle, a, b, C.byref(ms)))
        return ms.value

    OPT_TOPK_ROUTE = 1

    @property
    def n_cu(self):
        dev, n = C.c_int(), C.c_int()
        self._check(lib().ulspec_device_info(self.handle, C.byref(dev), C.byref(n)))
        return n.value

    def sync_probe(self, mode, workgroups, threads, rounds):
        """(us per grid-barrier round, stale reads) of ulspec_sync_probe."""
        us, err = C.c_float(), U32()
        self._check(lib().ulspec_sync_probe(self.handle, mode, workgroups, threads, rounds, C.byref(us),
                                            C.byref(err)))
        return us.value, err.value

    def set_option(self, option, value):
        self._check(lib().ulspec_set_option(self.handle, option, value))

    def stream_read(self, buf, nbytes, variant, sink):
        """The streaming-read measurement kernel over nbytes of device buffer buf."""
        self._check(lib().ulspec_stream_read(self.handle, _ptr(buf), nbytes, variant, _ptr(sink)))

    # -- K1 ------------------------------------------------------------------
    def weight_upload(self, wtype, blocks, n_rows, k):
        blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
        wid = U32()
        self._check(lib().ulspec_weight_upload(self.handle, wtype, blocks.ctypes.data_as(P), blocks.nbytes,
                                               n_rows, k, C.byref(wid)))
        return wid.value

    def weight_info(self, wid):
        t, n, k, b = U32(), U32(), U32(), C.c_size_t()
        self._check(lib().ulspec_weight_info(self.handle, wid, C.byref(t), C.byref(n), C.byref(k), C.byref(b)))
        return t.value, n.value, k.value, b.value

    def verify_gemm(self, wid, x, M, y):
        self._check(lib().ulspec_verify_gemm(self.handle, wid, int(x.ptr if hasattr(x, "ptr") else x), M,
                                             int(y.ptr if hasattr(y, "ptr") else y)))

    # -- K2 ------------------------------------------------------------------
    def verify_attention(self, q, k_cache, v_cache, n_prefix, nq, parent, H, Hkv, D, scale, out):
        par = None
        if parent is not None:
            par = np.ascontiguousarray(parent, dtype=np.int32)
        self._check(lib().ulspec_verify_attention(
            self.handle, _ptr(q), _ptr(k_cache), _ptr(v_cache), n_prefix, nq,
            par.ctypes.data_as(P) if par is not None else None, H, Hkv, D, scale, _ptr(out)))

    # -- K3 ------------------------------------------------------------------
    def accept(self, s, B, k, V, target, draft, draft_tokens, uniforms, out_tokens, out_nacc):
        self._check(lib().ulspec_accept(self.handle, C.byref(s), B, k, V, _ptr(target), _ptr(draft),
                                        _ptr(draft_tokens), _ptr(uniforms), _ptr(out_tokens), _ptr(out_nacc)))

    def accept_noalloc(self, s, B, k, V, target, draft, draft_tokens, uniforms, out_tokens, out_nacc):
        """accept() on the library's static scratch: allocates nothing."""
        self._check(lib().ulspec_accept_noalloc(self.handle, C.byref(s), B, k, V, _ptr(target), _ptr(draft),
                                                _ptr(draft_tokens), _ptr(uniforms), _ptr(out_tokens),
                                                _ptr(out_nacc)))

    def accept_tree(self, s, B, n, V, parent, target, draft, tokens, uniforms, out_tokens, out_path, out_nacc):
        """Tree verification; parent is a host array [n], the rest device buffers."""
        par = np.ascontiguousarray(parent, dtype=np.int32)
        self._check(lib().ulspec_accept_tree(self.handle, C.byref(s), B, n, V, par.ctypes.data_as(P), _ptr(target),
                                             _ptr(draft), _ptr(tokens), _ptr(uniforms), _ptr(out_tokens),
                                             _ptr(out_path), _ptr(out_nacc)))

    def sample(self, s, R, V, logits, uniforms, out_tokens):
        self._check(lib().ulspec_sample(self.handle, C.byref(s), R, V, _ptr(logits), _ptr(uniforms),
                                        _ptr(out_tokens)))

    def uniforms(self, seed, idx0, n, out):
        self._check(lib().ulspec_uniforms(self.handle, seed, idx0, n, _ptr(out)))

    # -- synthetic weights -----------------------------------------------------
    def synth_q4(self, wtype, seed, stream, n_rows, k, std, out):
        self._check(lib().ulspec_synth_q4(self.handle, wtype, seed, stream, n_rows, k, std, _ptr(out)))


def row_bytes(wtype, k):
    return (k // lib().ulspec_ggml_blck_size(wtype)) * lib().ulspec_ggml_type_size(wtype)


class Model:
    """ulspec_model: a Llama-shaped target or draft model on one context."""

    def __init__(self, ctx, dim, n_layers, n_heads, n_kv_heads, ffn, vocab, max_ctx, rms_eps=1e-5,
                 rope_base=10000.0, n_seq=1):
        """n_seq > 1: that many sequence slots (K/V caches) for a batch loop."""
        self.ctx = ctx
        self.n_seq = n_seq
        self.cfg = ModelCfg(dim, n_layers, n_heads, n_kv_heads, ffn, vocab, max_ctx, rms_eps, rope_base)
        h = P()
        ctx._check(lib().ulspec_model_create_batch(ctx.handle, C.byref(self.cfg), n_seq, C.byref(h)))
        self.handle = h.value

    def close(self):
        if self.handle:
            lib().ulspec_model_destroy(self.handle)
            self.handle = None

    def set_tensor(self, name, wtype, data, ne0, ne1):
        """data: a numpy array (host) or a DeviceBuffer (device) of GGUF bytes."""
        if hasattr(data, "ptr"):
            ptr, nbytes, dev = data.ptr, data.nbytes, 1
        else:
            data = np.ascontiguousarray(data)
            ptr, nbytes, dev = data.ctypes.data, data.nbytes, 0
        self.ctx._check(lib().ulspec_model_set_tensor(self.handle, name.encode(), wtype, ptr, nbytes, ne0, ne1, dev))

    def forward(self, tokens, pos, n_logits=0, seq=0):
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.empty((n_logits, self.cfg.vocab), np.float32) if n_logits else None
        self.ctx._check(lib().ulspec_model_forward_seq(self.handle, seq, tokens.ctypes.data_as(P), len(tokens), pos,
                                                       out.ctypes.data_as(P) if out is not None else None, n_logits))
        return out

    def forward_tree(self, tokens, parent, pos):
        """Logits [M][vocab] of the M tree nodes (K/V to slots pos .. pos+M-1)."""
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        parent = np.ascontiguousarray(parent, dtype=np.int32)
        out = np.empty((len(tokens), self.cfg.vocab), np.float32)
        self.ctx._check(lib().ulspec_model_forward_tree(self.handle, tokens.ctypes.data_as(P),
                                                        parent.ctypes.data_as(P), len(tokens), pos,
                                                        out.ctypes.data_as(P)))
        return out

    LIN_QKV, LIN_O, LIN_GATE_UP, LIN_DOWN, LIN_HEAD = range(5)

    def linear(self, layer, which, M, pos):
        """One linear of a layer (LIN_*) alone, with its fused prologue and
        epilogue, over the M rows the activation buffers hold (asynchronous)."""
        self.ctx._check(lib().ulspec_model_linear(self.handle, layer, which, M, pos))

    def kv_compact(self, pos, path, n_accepted, n_max):
        """Keep the accepted path's K/V rows (path, n_accepted: device buffers)."""
        self.ctx._check(lib().ulspec_model_kv_compact(self.handle, pos, _ptr(path), _ptr(n_accepted), n_max))

    def kv_io(self, layer, dir, pos0, n, k=None, v=None, seq=0):
        row = self.cfg.n_kv_heads * (self.cfg.dim // self.cfg.n_heads)
        if dir == 0:
            k = np.empty((n, row), np.uint16)
            v = np.empty((n, row), np.uint16)
        else:
            k = np.ascontiguousarray(k, dtype=np.uint16)
            v = np.ascontiguousarray(v, dtype=np.uint16)
        self.ctx._check(lib().ulspec_model_kv_io_seq(self.handle, seq, layer, dir, pos0, n, k.ctypes.data_as(P),
                                                     v.ctypes.data_as(P)))
        return k, v


class GGUFTensor:
    """One entry of a GGUF tensor table; data is a read-only view into the mapping."""

    def __init__(self, name, ggml_type, shape, offset, nbytes, data):
        self.name, self.ggml_type, self.shape = name, ggml_type, shape
        self.offset, self.nbytes, self.data = offset, nbytes, data

    def __repr__(self):
        return f"GGUFTensor({self.name!r}, type={self.ggml_type}, ne={self.shape}, {self.nbytes} B)"


class GGUFFile:
    """ulspec_gguf: a memory-mapped GGUF v2/v3 file (host only, no GPU needed).

    The reference's GGUFParser (src/core/gguf_parser.h:37-90) with the GGUF
    block sizes corrected; tensors are views into the mapping, metadata is read
    by key."""

    def __init__(self, path):
        L = lib()
        h = P()
        err = C.create_string_buffer(512)
        st = L.ulspec_gguf_open(os.fsencode(path), C.byref(h), err, len(err))
        if st != OK:
            raise UlspecError(st, err.value.decode(errors="replace"))
        self.handle = h.value
        v, nt, nkv, al, off = U32(), C.c_uint64(), C.c_uint64(), C.c_uint64(), C.c_uint64()
        L.ulspec_gguf_header(self.handle, C.byref(v), C.byref(nt), C.byref(nkv), C.byref(al), C.byref(off))
        self.version, self.n_tensors, self.n_kv = v.value, nt.value, nkv.value
        self.alignment, self.data_offset = al.value, off.value

    def close(self):
        if self.handle:
            lib().ulspec_gguf_close(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def _check(self, st):
        if st != OK:
            raise UlspecError(st, lib().ulspec_gguf_last_error(self.handle).decode(errors="replace"))

    def tensor(self, i):
        name, t, nd, ne = C.c_char_p(), U32(), U32(), (C.c_uint64 * 4)()
        off, nb, data = C.c_uint64(), C.c_uint64(), P()
        self._check(lib().ulspec_gguf_tensor(self.handle, i, C.byref(name), C.byref(t), C.byref(nd), ne, C.byref(off),
                                             C.byref(nb), C.byref(data)))
        view = None
        if data.value:
            view = np.ctypeslib.as_array(C.cast(data.value, C.POINTER(C.c_uint8)), shape=(nb.value,))
            view.flags.writeable = False
        return GGUFTensor(name.value.decode(), t.value, tuple(ne[:nd.value]), off.value, nb.value, view)

    def tensors(self):
        return [self.tensor(i) for i in range(self.n_tensors)]

    def find(self, name):
        i = C.c_uint64()
        if lib().ulspec_gguf_find_tensor(self.handle, name.encode(), C.byref(i)) != OK:
            return None
        return self.tensor(i.value)

    def keys(self):
        out = []
        for i in range(self.n_kv):
            k, t, at, n = C.c_char_p(), U32(), U32(), C.c_uint64()
            self._check(lib().ulspec_gguf_kv(self.handle, i, C.byref(k), C.byref(t), C.byref(at), C.byref(n)))
            out.append((k.value.decode(), t.value, at.value, n.value))
        return out

    def get_str_array(self, key):
        """The strings of an array-of-strings entry (e.g. tokenizer.ggml.tokens)."""
        for i, (k, t, at, n) in enumerate(self.keys()):
            if k == key:
                if t != 9 or at != 8:
                    raise UlspecError(EINVAL, f"{key} is not an array of strings")
                p, nb = P(), C.c_uint64()
                self._check(lib().ulspec_gguf_kv_bytes(self.handle, i, C.byref(p), C.byref(nb)))
                raw = C.string_at(p.value, nb.value)
                out, pos = [], 0
                for _ in range(n):
                    ln = int.from_bytes(raw[pos:pos + 8], "little")
                    out.append(raw[pos + 8:pos + 8 + ln].decode(errors="replace"))
                    pos += 8 + ln
                return out
        raise UlspecError(EINVAL, f"no metadata key {key}")

    def get_int(self, key):
        v = C.c_int64()
        self._check(lib().ulspec_gguf_get_int(self.handle, key.encode(), C.byref(v)))
        return v.value

    def get_float(self, key):
        v = C.c_double()
        self._check(lib().ulspec_gguf_get_float(self.handle, key.encode(), C.byref(v)))
        return v.value

    def get_str(self, key):
        p, n = P(), C.c_uint64()
        self._check(lib().ulspec_gguf_get_str(self.handle, key.encode(), C.byref(p), C.byref(n)))
        return C.string_at(p.value, n.value).decode(errors="replace")

    def llama_cfg(self, max_ctx=0):
        cfg = ModelCfg()
        self._check(lib().ulspec_gguf_llama_cfg(self.handle, max_ctx, C.byref(cfg)))
        return cfg


def load_gguf_model(ctx, gguf, max_ctx=0, n_seq=1):
    """Model from a GGUFFile (or a path): ulspec_model_load_gguf; n_seq > 1: a
    batch model (ulspec_model_load_gguf_batch)."""
    own = not isinstance(gguf, GGUFFile)
    f = GGUFFile(gguf) if own else gguf
    try:
        h = P()
        if n_seq == 1:
            ctx._check(lib().ulspec_model_load_gguf(ctx.handle, f.handle, max_ctx, C.byref(h)))
        else:
            ctx._check(lib().ulspec_model_load_gguf_batch(ctx.handle, f.handle, max_ctx, n_seq, C.byref(h)))
        m = Model.__new__(Model)
        m.ctx, m.handle, m.n_seq = ctx, h.value, n_seq
        m.cfg = f.llama_cfg(max_ctx)
        return m
    finally:
        if own:
            f.close()


class Speculative:
    """ulspec_spec: the device speculative-decoding loop over a target and a
    draft model; k = 0 (draft None) decodes with the target alone."""

    def __init__(self, target, draft, k, s, seed, n_seq=1, parent=None):
        """n_seq > 1: a batch of that many sequences (models with as many slots).
        parent (a breadth-first tree of n nodes): tree steps; k is then n - 1."""
        self.ctx = target.ctx
        self.target, self.draft, self.n_seq = target, draft, n_seq
        h = P()
        if parent is not None:
            self.parent = np.ascontiguousarray(parent, dtype=np.int32)
            self.k = len(self.parent) - 1
            self.ctx._check(lib().ulspec_spec_create_tree(target.handle, draft.handle, len(self.parent),
                                                          self.parent.ctypes.data_as(P), C.byref(s), seed,
                                                          C.byref(h)))
        else:
            self.parent, self.k = None, k
            self.ctx._check(lib().ulspec_spec_create_batch(target.handle, draft.handle if draft is not None else None,
                                                           k, C.byref(s), seed, n_seq, C.byref(h)))
        self.handle = h.value

    def close(self):
        if self.handle:
            lib().ulspec_spec_destroy(self.handle)
            self.handle = None

    def prefill(self, prompt):
        """One prompt, or a list of n_seq prompts for a batch."""
        if self.n_seq == 1 and not isinstance(prompt, (list, tuple)):
            prompt = np.ascontiguousarray(prompt, dtype=np.int32)
            self.ctx._check(lib().ulspec_spec_prefill(self.handle, prompt.ctypes.data_as(P), len(prompt)))
            return
        lens = np.array([len(p) for p in prompt], np.uint32)
        flat = np.ascontiguousarray(np.concatenate([np.asarray(p, np.int32) for p in prompt]), dtype=np.int32)
        self.ctx._check(lib().ulspec_spec_prefill_batch(self.handle, flat.ctypes.data_as(P), lens.ctypes.data_as(P)))

    def steps(self, n):
        self.ctx._check(lib().ulspec_spec_steps(self.handle, n))

    def generate(self, n_new):
        n = U32()
        self.ctx._check(lib().ulspec_spec_generate(self.handle, n_new, C.byref(n)))
        return n.value

    def state(self):
        n, steps, acc, prop = U32(), C.c_uint64(), C.c_uint64(), C.c_uint64()
        self.ctx._check(lib().ulspec_spec_state(self.handle, C.byref(n), C.byref(steps), C.byref(acc),
                                                C.byref(prop)))
        return {"n": n.value, "steps": steps.value, "accepted": acc.value, "proposed": prop.value}

    def seq_state(self, seq):
        n, acc, prop = U32(), C.c_uint64(), C.c_uint64()
        self.ctx._check(lib().ulspec_spec_seq_state(self.handle, seq, C.byref(n), C.byref(acc), C.byref(prop)))
        return {"n": n.value, "accepted": acc.value, "proposed": prop.value}

    def tokens(self, start=0, n=None, seq=0):
        if n is None:
            n = self.seq_state(seq)["n"] - start
        out = np.empty(n, np.int32)
        self.ctx._check(lib().ulspec_spec_seq_tokens(self.handle, seq, start, n, out.ctypes.data_as(P)))
        return out

    def last_step(self):
        """Inputs and outputs of the last step (host copies); for a batch, every
        array has a leading sequence axis and n_accepted is an array."""
        k, V, B = self.k, self.target.cfg.vocab, self.n_seq
        if self.parent is not None:
            n = k + 1
            r = {"target_logits": np.empty((n, V), np.float32), "draft_logits": np.empty((n - 1, V), np.float32),
                 "tokens": np.empty(n, np.int32), "uniforms": np.empty(2 * n - 1, np.float32),
                 "out_tokens": np.empty(n, np.int32), "path": np.empty(n, np.int32),
                 "n_accepted": np.empty(1, np.int32)}
            self.ctx._check(lib().ulspec_spec_tree_last_step(self.handle, *[a.ctypes.data_as(P) for a in r.values()]))
            r["n_accepted"] = int(r["n_accepted"][0])
            return r
        r = {"target_logits": np.empty((B, k + 1, V), np.float32), "draft_logits": np.empty((B, k, V), np.float32),
             "draft_tokens": np.empty((B, k), np.int32), "uniforms": np.empty((B, 2 * k + 1), np.float32),
             "out_tokens": np.empty((B, k + 1), np.int32), "n_accepted": np.empty(B, np.int32)}
        self.ctx._check(lib().ulspec_spec_last_step(self.handle, *[a.ctypes.data_as(P) for a in r.values()]))
        if B == 1:
            r = {name: a[0] for name, a in r.items()}
            r["n_accepted"] = int(r["n_accepted"])
        return r

    def set_graph(self, use_graph):
        self.ctx._check(lib().ulspec_spec_set_graph(self.handle, 1 if use_graph else 0))


def _ptr(b):
    if b is None:
        return None
    return int(b.ptr) if hasattr(b, "ptr") else int(b)
