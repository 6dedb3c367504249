"""GGUF ingestion on the CPU: the library's reader (ulspec_gguf_*) against a
hand-assembled file, against the independent Python writer/reader of
tests/gguf_io.py, and on malformed input.  No GPU is touched."""
import struct

import numpy as np
import pytest

import gguf_io as G


def hand_file(path):
    """A two-tensor GGUF v3 file assembled field by field, with its expected parse."""
    b = b"GGUF" + struct.pack("<IQQ", 3, 2, 3)
    b += struct.pack("<Q", 20) + b"general.architecture" + struct.pack("<I", 8) + struct.pack("<Q", 5) + b"llama"
    b += struct.pack("<Q", 17) + b"general.alignment" + struct.pack("<I", 4) + struct.pack("<I", 64)
    b += struct.pack("<Q", 3) + b"arr" + struct.pack("<I", 9) + struct.pack("<IQ", 5, 3) + struct.pack("<3i", -1, 2, 7)
    # tensor 0: Q4_0 [64 x 2] = 2 rows x 2 blocks x 18 B = 72 B at offset 0
    b += struct.pack("<Q", 1) + b"a" + struct.pack("<I", 2) + struct.pack("<QQ", 64, 2) + struct.pack("<IQ", 2, 0)
    # tensor 1: F32 [3] = 12 B at offset 128 (72 rounded up to 64 is 128)
    b += struct.pack("<Q", 1) + b"b" + struct.pack("<I", 1) + struct.pack("<Q", 3) + struct.pack("<IQ", 0, 128)
    data_off = (len(b) + 63) // 64 * 64
    b += b"\0" * (data_off - len(b))
    t0 = bytes(range(72))
    t1 = struct.pack("<3f", 1.5, -2.0, 0.25)
    b += t0 + b"\0" * (128 - 72) + t1
    with open(path, "wb") as f:
        f.write(b)
    return data_off, t0, t1


def test_hand_assembled_file(pkg, tmp_path):
    p = tmp_path / "hand.gguf"
    data_off, t0, t1 = hand_file(p)
    with pkg.GGUFFile(str(p)) as g:
        assert (g.version, g.n_tensors, g.n_kv, g.alignment, g.data_offset) == (3, 2, 3, 64, data_off)
        a, b = g.tensor(0), g.tensor(1)
        assert (a.name, a.ggml_type, a.shape, a.offset, a.nbytes) == ("a", 2, (64, 2), 0, 72)
        assert (b.name, b.ggml_type, b.shape, b.offset, b.nbytes) == ("b", 0, (3,), 128, 12)
        assert a.data.tobytes() == t0 and b.data.tobytes() == t1
        assert g.get_str("general.architecture") == "llama"
        assert g.get_int("general.alignment") == 64
        assert g.keys()[2] == ("arr", G.ARRAY, G.I32, 3)
        assert g.find("b").name == "b" and g.find("c") is None
        with pytest.raises(pkg.UlspecError):
            g.get_int("arr")


def test_block_table_matches_block_fields(pkg):
    L = pkg.lib()
    for t, (blk, nb) in G.BLOCK.items():
        assert (L.ulspec_ggml_blck_size(t), L.ulspec_ggml_type_size(t)) == (blk, nb), t


KV_ALL = [("u8", G.U8, 200), ("i8", G.I8, -100), ("u16", G.U16, 60000), ("i16", G.I16, -30000),
          ("u32", G.U32, 4000000000), ("i32", G.I32, -2000000000), ("f32", G.F32, 0.5), ("bool", G.BOOL, True),
          ("str", G.STRING, "héllo"), ("u64", G.U64, 2 ** 62), ("i64", G.I64, -2 ** 62), ("f64", G.F64, -1.25),
          ("arr.str", G.ARRAY, (G.STRING, ["x", "", "yz"])), ("arr.f32", G.ARRAY, (G.F32, [1.0, 2.0])),
          ("arr.nested", G.ARRAY, (G.ARRAY, [(G.U8, [1, 2]), (G.U8, [])]))]


@pytest.mark.parametrize("alignment", [32, 64, 256])
def test_writer_round_trip(pkg, tmp_path, alignment):
    rng = np.random.default_rng(alignment)
    shapes = [("f32", 0, (5,)), ("f16", 1, (7, 3)), ("q40", 2, (96, 4)), ("q4k", 12, (512, 3)), ("q6k", 14, (256, 2)),
              ("q80", 8, (64, 5)), ("bf16", 30, (4, 2, 2)), ("q4k3d", 12, (256, 2, 3))]
    tensors = [(n, t, ne, rng.integers(0, 256, G.tensor_nbytes(t, ne), dtype=np.uint8).tobytes())
               for n, t, ne in shapes]
    kv = KV_ALL + [("general.alignment", G.U32, alignment)]
    p = tmp_path / "rt.gguf"
    data_off = G.write(p, kv, tensors, alignment=alignment)
    version, kv_py, tens_py, off_py = G.read(p)
    assert off_py == data_off
    with pkg.GGUFFile(str(p)) as g:
        assert (g.version, g.n_tensors, g.n_kv, g.alignment, g.data_offset) == (3, len(tensors), len(kv), alignment,
                                                                                 data_off)
        for i, (name, t, ne, raw) in enumerate(tensors):
            x = g.tensor(i)
            assert (x.name, x.ggml_type, x.shape, x.nbytes) == (name, t, ne, len(raw))
            assert x.offset == tens_py[i][3] and x.offset % alignment == 0
            assert x.data.tobytes() == raw == tens_py[i][4]
        for key, t, v in KV_ALL:
            if t in (G.U8, G.I8, G.U16, G.I16, G.U32, G.I32, G.U64, G.I64, G.BOOL):
                assert g.get_int(key) == int(v)
            elif t in (G.F32, G.F64):
                assert g.get_float(key) == pytest.approx(v)
            elif t == G.STRING:
                assert g.get_str(key) == v
        keys = {k: (t, at, n) for k, t, at, n in g.keys()}
        assert keys["arr.str"] == (G.ARRAY, G.STRING, 3)
        assert keys["arr.nested"] == (G.ARRAY, G.ARRAY, 2)


def test_llama_cfg_from_metadata(pkg, tmp_path):
    cfg = dict(dim=64, n_layers=2, n_heads=4, n_kv_heads=2, ffn=96, vocab=40, max_ctx=128, rms_eps=1e-6,
               rope_base=500000.0)
    emb = ("token_embd.weight", 2, (64, 40), bytes(G.tensor_nbytes(2, (64, 40))))
    p = tmp_path / "cfg.gguf"
    G.write(p, G.llama_kv(cfg), [emb])
    with pkg.GGUFFile(str(p)) as g:
        c = g.llama_cfg(0)
        assert (c.dim, c.n_layers, c.n_heads, c.n_kv_heads, c.ffn, c.vocab, c.max_ctx) == (64, 2, 4, 2, 96, 40, 128)
        assert c.rms_eps == pytest.approx(1e-6) and c.rope_base == 500000.0
        assert g.llama_cfg(32).max_ctx == 32
    # head_count_kv and rope.freq_base default; a missing key is an error
    kv = [e for e in G.llama_kv(cfg) if e[0] not in ("llama.attention.head_count_kv", "llama.rope.freq_base")]
    G.write(p, kv, [emb])
    with pkg.GGUFFile(str(p)) as g:
        c = g.llama_cfg(0)
        assert c.n_kv_heads == 4 and c.rope_base == 10000.0
    G.write(p, [e for e in kv if e[0] != "llama.block_count"], [emb])
    with pkg.GGUFFile(str(p)) as g:
        with pytest.raises(pkg.UlspecError, match="block_count"):
            g.llama_cfg(0)
    G.write(p, [("general.architecture", G.STRING, "gpt2")] + kv[1:], [emb])
    with pkg.GGUFFile(str(p)) as g:
        with pytest.raises(pkg.UlspecError, match="gpt2"):
            g.llama_cfg(0)


def _expect_open_error(pkg, path, match):
    with pytest.raises(pkg.UlspecError, match=match):
        pkg.GGUFFile(str(path))


def test_malformed_files(pkg, tmp_path):
    p = tmp_path / "bad.gguf"
    good = tmp_path / "good.gguf"
    hand_file(good)
    raw = good.read_bytes()
    p.write_bytes(b"GGUX" + raw[4:])
    _expect_open_error(pkg, p, "magic")
    p.write_bytes(raw[:4] + struct.pack("<I", 1) + raw[8:])
    _expect_open_error(pkg, p, "version")
    _expect_open_error(pkg, tmp_path / "missing.gguf", "cannot open")
    # every truncation fails cleanly (header, metadata, tensor table or data)
    for n in range(0, len(raw) - 1, 3):
        p.write_bytes(raw[:n])
        with pytest.raises(pkg.UlspecError):
            pkg.GGUFFile(str(p))
    # misaligned tensor offset, data past the end, duplicated key, bad alignment
    t = [("a", 0, (4,), bytes(16))]
    G.write(p, [], t)
    b = bytearray(p.read_bytes())
    off_pos = b.index(b"a") + 1 + 4 + 8 + 4
    struct.pack_into("<Q", b, off_pos, 4)
    p.write_bytes(bytes(b))
    _expect_open_error(pkg, p, "aligned")
    struct.pack_into("<Q", b, off_pos, 1 << 20)
    p.write_bytes(bytes(b))
    _expect_open_error(pkg, p, "past the end")
    G.write(p, [("k", G.U8, 1), ("k", G.U8, 2)], t)
    _expect_open_error(pkg, p, "repeated")
    G.write(p, [("general.alignment", G.U32, 48)], t, alignment=32)
    _expect_open_error(pkg, p, "power of two")
    G.write(p, [], [("q", 2, (64, 1), bytes(36))])
    b = bytearray(p.read_bytes())
    struct.pack_into("<Q", b, b.index(b"q") + 1 + 4, 48)  # ne0 no longer a multiple of 32
    p.write_bytes(bytes(b))
    _expect_open_error(pkg, p, "multiple of the block")
    # dimensions whose byte count is 2^128 (4 B x 2^62 x 2^63 x 2): a product
    # wrapped in 128 bits would read 0 bytes and pass the size check
    b = b"GGUF" + struct.pack("<IQQ", 3, 1, 0)
    b += struct.pack("<Q", 1) + b"w" + struct.pack("<I", 3) + struct.pack("<3Q", 1 << 62, 1 << 63, 2)
    b += struct.pack("<IQ", 0, 0)
    b += b"\0" * ((len(b) + 31) // 32 * 32 - len(b)) + bytes(64)
    p.write_bytes(b)
    _expect_open_error(pkg, p, "past the end")


def test_unknown_type_is_listed_without_data(pkg, tmp_path):
    p = tmp_path / "unk.gguf"
    G.write(p, [], [("a", 0, (4,), bytes(16))])
    b = bytearray(p.read_bytes())
    struct.pack_into("<I", b, b.index(b"a") + 1 + 4 + 8, 99)
    p.write_bytes(bytes(b))
    with pkg.GGUFFile(str(p)) as g:
        x = g.tensor(0)
        assert x.ggml_type == 99 and x.nbytes == 0 and x.data is None
