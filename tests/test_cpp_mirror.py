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


@pytest.mark.gpu
def test_mirror_runs_on_gpu(tmp_path):
    exe = _build(tmp_path)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0 and r.stdout.startswith("OK")
