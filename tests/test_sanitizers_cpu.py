"""AddressSanitizer + UBSan builds of the host code that parses untrusted or
test input, on the CPU (no GPU is touched):

  - the GGUF reader (universal-loader_amd/csrc/host/gguf.cpp, host-only C++)
    built with clang++ -fsanitize=address,undefined into tests/cpp/gguf_walk,
    which reads everything the reader exposes from a set of hostile files:
    every truncation of two valid files, the malformed cases of
    test_gguf_cpu.py, and seeded byte and length-field corruptions;
  - the oracle (oracle/*.c, `make -C oracle san`) under the preloaded ASan
    runtime with Python allocating through malloc, running the oracle's own
    CPU tests.

Any out-of-bounds access or undefined behaviour aborts the child process,
which fails the test.
"""
import os
import shutil
import struct
import subprocess
import sys

import numpy as np
import pytest

import gguf_io as G
from conftest import PKG_DIR, REPO
from test_gguf_cpu import hand_file

CLANG = "/opt/rocm/llvm/bin/clang++"
LIBDIR = os.path.join(PKG_DIR, "lib")
SAN_ENV = {"ASAN_OPTIONS": "detect_leaks=0:abort_on_error=0", "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1"}


def _hostile_files(ora, d):
    good = d / "hand.gguf"
    hand_file(good)
    cfg = dict(dim=64, n_layers=1, n_heads=2, n_kv_heads=2, ffn=128, vocab=64, max_ctx=32, rms_eps=1e-5,
               rope_base=10000.0)
    from llama_util import make_tensors
    model = d / "model.gguf"
    G.write(model, G.llama_kv(cfg), G.model_tensors(make_tensors(ora, cfg, 2, seed=5)))
    out = [str(good), str(model)]
    rng = np.random.default_rng(99)
    for base, step in ((good, 1), (model, 97)):
        raw = base.read_bytes()
        for n in range(0, len(raw), step):  # every truncation (a stride through the larger file)
            p = d / f"t_{base.stem}_{n}.gguf"
            p.write_bytes(raw[:n])
            out.append(str(p))
        head = min(len(raw), 4096)  # header, metadata and tensor table
        for i in range(300):  # seeded corruptions of bytes and 8-byte length fields
            b = bytearray(raw)
            for _ in range(int(rng.integers(1, 5))):
                pos = int(rng.integers(4, head))
                if rng.random() < 0.5:
                    b[pos] = int(rng.integers(0, 256))
                elif pos + 8 <= len(b):
                    struct.pack_into("<Q", b, pos, (0, 1, 2 ** 31, 2 ** 62, 2 ** 64 - 1)[int(rng.integers(0, 5))])
            p = d / f"c_{base.stem}_{i}.gguf"
            p.write_bytes(bytes(b))
            out.append(str(p))
    # the 2^128-byte tensor of test_malformed_files
    b = b"GGUF" + struct.pack("<IQQ", 3, 1, 0)
    b += struct.pack("<Q", 1) + b"w" + struct.pack("<I", 3) + struct.pack("<3Q", 1 << 62, 1 << 63, 2)
    b += struct.pack("<IQ", 0, 0)
    b += b"\0" * ((len(b) + 31) // 32 * 32 - len(b)) + bytes(64)
    p = d / "huge.gguf"
    p.write_bytes(b)
    out.append(str(p))
    return out


def test_gguf_reader_under_asan_and_ubsan(ora, tmp_path):
    if not os.path.exists(CLANG) or not os.path.exists(os.path.join(LIBDIR, "libulspec.so")):
        pytest.skip("clang++ or libulspec.so missing")
    obj, exe = str(tmp_path / "gguf_san.o"), str(tmp_path / "gguf_walk")
    flags = ["-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=undefined",
             "-fno-omit-frame-pointer"]
    subprocess.run([CLANG, *flags, "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include", "-c",
                    os.path.join(PKG_DIR, "csrc", "host", "gguf.cpp"), "-o", obj], check=True)
    # the walker's ulspec_gguf_* resolve to the sanitized object; the GGUF
    # type table and the model entry points come from libulspec.so
    subprocess.run([CLANG, *flags, "-I", os.path.join(REPO, "include"), os.path.join(REPO, "tests", "cpp", "gguf_walk.cpp"),
                    obj, "-o", exe, "-L", LIBDIR, "-lulspec", f"-Wl,-rpath,{LIBDIR}"], check=True)
    files = _hostile_files(ora, tmp_path)
    r = subprocess.run([exe, *files], capture_output=True, text=True, timeout=600, env=dict(os.environ, **SAN_ENV))
    print(r.stdout[-2000:], r.stderr[-4000:])
    assert r.returncode == 0 and r.stdout.startswith("OK")
    opened, rejected = map(int, r.stdout.split()[1:3])
    assert opened + rejected == len(files) and opened >= 2 and rejected > len(files) // 2


def test_oracle_under_asan_and_ubsan(tmp_path):
    asan = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True).stdout.strip()
    if not os.path.isabs(asan) or shutil.which("make") is None:
        pytest.skip("no ASan runtime")
    subprocess.run(["make", "-s", "-C", os.path.join(REPO, "oracle"), "san"], check=True)
    env = dict(os.environ, **SAN_ENV, LD_PRELOAD=asan, PYTHONMALLOC="malloc",
               ORACLE_LIB=os.path.join(REPO, "oracle", "_build", "liboracle_san.so"))
    tests = [os.path.join(REPO, "tests", t) for t in
             ("test_oracle_cpu.py", "test_tree_cpu.py", "test_llama_cpu.py", "test_golden_cpu.py")]
    r = subprocess.run([sys.executable, "-m", "pytest", *tests, "-q", "-x", "-p", "no:cacheprovider", "-m", "not gpu"],
                       capture_output=True, text=True, timeout=900, env=env, cwd=str(tmp_path))
    print(r.stdout[-3000:], r.stderr[-4000:])
    assert r.returncode == 0 and " passed" in r.stdout
