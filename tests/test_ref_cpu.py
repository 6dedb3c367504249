"""Cross-checks against the reference's own CPU functions for this path,
compiled from their sources into oracle/_ref/libref.so (see oracle/Makefile,
target `ref`).  Skipped when that library has not been built."""
import ctypes as C
import os

import numpy as np
import pytest

from conftest import REPO

REF = os.path.join(REPO, "oracle", "_ref", "libref.so")
pytestmark = pytest.mark.skipif(not os.path.exists(REF), reason="oracle/_ref not built (needs /root/reference)")


@pytest.fixture(scope="module")
def ref():
    L = C.CDLL(REF)
    P = C.c_void_p
    L.ref_softmax_f32.argtypes = [P, P, C.c_size_t]
    L.ref_silu_f32.argtypes = [P, P, C.c_size_t]
    L.ref_specdec_create.restype = P
    L.ref_specdec_create.argtypes = [C.c_uint32, C.c_uint32, C.c_float]
    L.ref_specdec_update.argtypes = [P, C.c_uint32, C.c_uint32]
    L.ref_specdec_rate.restype = C.c_float
    L.ref_specdec_rate.argtypes = [P]
    L.ref_specdec_free.argtypes = [P]
    L.ref_ggml_blck_size.argtypes = [C.c_uint32]
    L.ref_ggml_type_size.restype = C.c_size_t
    L.ref_ggml_type_size.argtypes = [C.c_uint32]
    return L


def test_reference_softmax_agrees_with_oracle_warp(ref, ora, rng):
    # cpu::softmax_f32 (std::exp, fp32 sums) vs the oracle's fixed-point warp at T = 1
    for V in (17, 1000, 32000):
        x = (rng.standard_normal(V) * 3).astype(np.float32)
        out = np.empty(V, np.float32)
        ref.ref_softmax_f32(out.ctypes.data, x.ctypes.data, V)
        E, Z, _ = ora.warp_row(ora.sampling(1.0), x)
        p = E.astype(np.float64) / Z
        # the reference sums 32000 fp32 terms in order (~3e-5 relative error);
        # the oracle is within ~1e-6 of float64
        big = p > 1e-9
        assert np.allclose(out[big], p[big], rtol=1e-4)
        assert np.allclose(out, p, rtol=0, atol=1e-4 * p.max())


def test_reference_acceptance_rate_bookkeeping(ref):
    # speculative_decoder.cpp:10 (initial 0.5) and :112-116 (cumulative ratio)
    d = ref.ref_specdec_create(32000, 5, 0.5)
    assert ref.ref_specdec_rate(d) == pytest.approx(0.5)
    ref.ref_specdec_update(d, 3, 5)
    assert ref.ref_specdec_rate(d) == pytest.approx(3 / 5)
    ref.ref_specdec_update(d, 1, 5)
    assert ref.ref_specdec_rate(d) == pytest.approx(4 / 10)
    ref.ref_specdec_free(d)


def test_type_ids_and_block_sizes_agree_byte_sizes_corrected(ref, pkg):
    L = pkg.lib()
    for t in (2, 12):
        assert L.ulspec_ggml_blck_size(t) == ref.ref_ggml_blck_size(t)
    # the reference's byte sizes are wrong for the Q4 types (6 / 12 B per block)
    assert ref.ref_ggml_type_size(2) == 6 and ref.ref_ggml_type_size(12) == 12
    assert L.ulspec_ggml_type_size(2) == 18 and L.ulspec_ggml_type_size(12) == 144
