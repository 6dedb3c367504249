"""The C-ABI library loads on the CPU and exports every symbol include/ulspec.h
declares; calls that need a device fail with a status code, not a crash."""
import ctypes as C
import os
import re

import pytest

from conftest import REPO


def _declared():
    text = open(os.path.join(REPO, "include", "ulspec.h")).read()
    return sorted(set(re.findall(r"\b(ulspec_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree(pkg):
    names = {n for n, _, _ in pkg.ABI}
    assert set(_declared()) == names


def test_library_exports_every_declared_symbol(pkg):
    L = pkg.lib()
    for name in _declared():
        assert hasattr(L, name), name


def test_block_sizes(pkg):
    L = pkg.lib()
    assert L.ulspec_ggml_blck_size(2) == 32 and L.ulspec_ggml_type_size(2) == 18
    assert L.ulspec_ggml_blck_size(12) == 256 and L.ulspec_ggml_type_size(12) == 144
    assert L.ulspec_ggml_blck_size(4) == 0 and L.ulspec_ggml_type_size(99) == 0  # removed / unknown ids


def test_null_arguments_are_rejected_without_a_device(pkg):
    L = pkg.lib()
    assert L.ulspec_create(0, None) == pkg.EINVAL
    assert L.ulspec_sync(None) == pkg.EINVAL
    assert L.ulspec_verify_gemm(None, 0, None, 1, None) == pkg.EINVAL
    assert L.ulspec_accept(None, None, 1, 1, 1, None, None, None, None, None, None) == pkg.EINVAL
    assert L.ulspec_last_error(None) == b"null context"
    assert L.ulspec_status_str(pkg.EUNSUPPORTED) == b"unsupported"


def test_create_reports_missing_device(pkg):
    L = pkg.lib()
    h = C.c_void_p()
    st = L.ulspec_create(0, C.byref(h))
    if st == pkg.OK:  # a gfx950 is present: nothing to check here
        L.ulspec_destroy(h)
        pytest.skip("device present")
    assert st == pkg.EDEVICE and not h.value
