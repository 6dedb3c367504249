"""The C++ host classes (include/ulspec_inference.hpp) compile against the C
ABI and link with libulspec.so; on the GPU the mirror test program runs."""
import os
import subprocess

import pytest

from conftest import PKG_DIR, REPO

SRC = os.path.join(REPO, "tests", "cpp", "mirror_test.cpp")
LIBDIR = os.path.join(PKG_DIR, "lib")


def _build(tmp_path):
    exe = str(tmp_path / "mirror_test")
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Wextra", "-I", os.path.join(REPO, "include"), SRC, "-o", exe,
                    "-L", LIBDIR, "-lulspec", f"-Wl,-rpath,{LIBDIR}"], check=True)
    return exe


def test_mirror_compiles_and_links(tmp_path):
    if not os.path.exists(os.path.join(LIBDIR, "libulspec.so")):
        pytest.skip("libulspec.so not built")
    assert os.path.exists(_build(tmp_path))


def _gguf_files(ora, d):
    """A 2-layer target and a 1-layer draft (dim 256, vocabulary strings "▁w<i>")."""
    import gguf_io as G
    from llama_util import make_tensors
    cfg0 = dict(dim=256, n_layers=2, n_heads=4, n_kv_heads=4, ffn=512, vocab=1000, max_ctx=128, rms_eps=1e-5,
                rope_base=10000.0)
    out = []
    for name, seed, layers in (("target", 41, 2), ("draft", 42, 1)):
        cfg = dict(cfg0, n_layers=layers)
        kv = [e if e[0] != "tokenizer.ggml.tokens" else
              ("tokenizer.ggml.tokens", G.ARRAY, (G.STRING, [f"\u2581w{i}" for i in range(cfg0["vocab"])]))
              for e in G.llama_kv(cfg)]
        p = d / f"{name}.gguf"
        G.write(p, kv, G.model_tensors(make_tensors(ora, cfg, 12, seed=seed)))
        out.append(str(p))
    return out


@pytest.mark.gpu
def test_mirror_runs_on_gpu(tmp_path, ora):
    exe = _build(tmp_path)
    r = subprocess.run([exe, *_gguf_files(ora, tmp_path)], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0 and r.stdout.startswith("OK")
