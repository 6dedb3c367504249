"""Pure-Python GGUF v3 writer and reader (test infrastructure, independent of
the C reader in the library): files for the ingestion tests, and a second
reading of every file the tests write.

Layout (GGUF spec, little endian): magic "GGUF", u32 version, u64 tensor
count, u64 metadata count; metadata (string key, u32 value type, value);
tensor infos (string name, u32 n_dims, u64 ne[n_dims], u32 ggml type, u64
offset from the data section); zero padding to general.alignment; tensor data,
each tensor padded to the alignment.  Strings are a u64 length + UTF-8 bytes.
"""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
           I64: "<q", F64: "<d"}

# ggml block layouts, written out from their fields: (elements, bytes)
BLOCK = {
    0: (1, 4), 1: (1, 2), 30: (1, 2),     # F32, F16, BF16
    2: (32, 2 + 16),                      # Q4_0: d, qs[16]
    3: (32, 2 + 2 + 16),                  # Q4_1: d, m, qs[16]
    6: (32, 2 + 4 + 16),                  # Q5_0: d, qh[4], qs[16]
    7: (32, 2 + 2 + 4 + 16),              # Q5_1
    8: (32, 2 + 32),                      # Q8_0: d, qs[32]
    12: (256, 2 + 2 + 12 + 128),          # Q4_K: d, dmin, scales[12], qs[128]
    14: (256, 128 + 64 + 16 + 2),         # Q6_K: ql[128], qh[64], scales[16], d
    10: (256, 16 + 64 + 2 + 2),           # Q2_K: scales[16], qs[64], d, dmin
    11: (256, 32 + 64 + 12 + 2),          # Q3_K: hmask[32], qs[64], scales[12], d
    13: (256, 2 + 2 + 12 + 32 + 128),     # Q5_K: d, dmin, scales[12], qh[32], qs[128]
    15: (256, 4 + 256 + 32),              # Q8_K: f32 d, qs[256], i16 bsums[16]
}


def tensor_nbytes(ggml_type, ne):
    blk, nb = BLOCK[ggml_type]
    assert ne[0] % blk == 0
    n = ne[0] // blk * nb
    for d in ne[1:]:
        n *= d
    return n


def _str(s):
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _value(t, v):
    if t in _SCALAR:
        return struct.pack(_SCALAR[t], v)
    if t == STRING:
        return _str(v)
    if t == ARRAY:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        for x in items:
            out += _value(et, x)
        return out
    raise ValueError(t)


def write(path, kv, tensors, alignment=32, version=3):
    """kv: list of (key, value type, value) -- arrays as (ARRAY, (elem type, items));
    tensors: list of (name, ggml type, ne tuple, bytes).  Returns the data offset."""
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kv))
    for key, t, v in kv:
        head += _str(key) + struct.pack("<I", t) + _value(t, v)
    offsets, off = [], 0
    for name, gt, ne, data in tensors:
        assert len(data) == tensor_nbytes(gt, ne), name
        offsets.append(off)
        off += (len(data) + alignment - 1) // alignment * alignment
    for (name, gt, ne, data), o in zip(tensors, offsets):
        head += _str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", d) for d in ne)
        head += struct.pack("<IQ", gt, o)
    data_off = (len(head) + alignment - 1) // alignment * alignment
    with open(path, "wb") as f:
        f.write(head + b"\0" * (data_off - len(head)))
        for name, gt, ne, data in tensors:
            f.write(bytes(data))
            pad = (-len(data)) % alignment
            f.write(b"\0" * pad)
    return data_off


def read(path):
    """-> (version, {key: (type, value)}, [(name, type, ne, offset, bytes)], data offset)."""
    b = open(path, "rb").read()
    pos = 0

    def take(fmt):
        nonlocal pos
        v = struct.unpack_from(fmt, b, pos)
        pos += struct.calcsize(fmt)
        return v[0] if len(v) == 1 else v

    def string():
        n = take("<Q")
        nonlocal pos
        s = b[pos:pos + n].decode()
        pos += n
        return s

    def value(t):
        if t in _SCALAR:
            return take(_SCALAR[t])
        if t == STRING:
            return string()
        if t == ARRAY:
            et, n = take("<I"), take("<Q")
            return (et, [value(et) for _ in range(n)])
        raise ValueError(t)

    assert b[:4] == b"GGUF"
    pos = 4
    version, nt, nkv = take("<I"), take("<Q"), take("<Q")
    kv = {}
    for _ in range(nkv):
        k = string()
        t = take("<I")
        kv[k] = (t, value(t))
    infos = []
    for _ in range(nt):
        name = string()
        nd = take("<I")
        ne = tuple(take("<Q") for _ in range(nd))
        gt, off = take("<I"), take("<Q")
        infos.append((name, gt, ne, off))
    align = kv.get("general.alignment", (U32, 32))[1]
    data_off = (pos + align - 1) // align * align
    out = [(n, gt, ne, off, b[data_off + off:data_off + off + tensor_nbytes(gt, ne)]) for n, gt, ne, off in infos]
    return version, kv, out, data_off


def llama_kv(cfg, name="test-llama", alignment=None):
    """The llama.* metadata of a model configuration dict."""
    kv = [("general.architecture", STRING, "llama"), ("general.name", STRING, name),
          ("llama.context_length", U32, cfg["max_ctx"]), ("llama.embedding_length", U32, cfg["dim"]),
          ("llama.block_count", U32, cfg["n_layers"]), ("llama.feed_forward_length", U32, cfg["ffn"]),
          ("llama.attention.head_count", U32, cfg["n_heads"]),
          ("llama.attention.head_count_kv", U32, cfg["n_kv_heads"]),
          ("llama.attention.layer_norm_rms_epsilon", F32, cfg["rms_eps"]),
          ("llama.rope.freq_base", F32, cfg["rope_base"]),
          ("tokenizer.ggml.model", STRING, "llama"),
          ("tokenizer.ggml.tokens", ARRAY, (STRING, [f"<t{i}>" for i in range(8)]))]
    if alignment is not None:
        kv.append(("general.alignment", U32, alignment))
    return kv


def model_tensors(tensors):
    """llama_util.make_tensors output -> writer tensor list (ne = (ne0, ne1), or (ne0,) for norms)."""
    out = []
    for name, (wtype, data, ne0, ne1) in tensors.items():
        raw = np.ascontiguousarray(data).view(np.uint8).tobytes()
        out.append((name, wtype, (ne0,) if ne1 == 1 and wtype == 0 else (ne0, ne1), raw))
    return out
