"""Pins the oracle's fp16 conversion.

Known answers from tests/ModelFormatTest.cpp:54-63 (exhaustive round trip of
every non-inf/NaN bit pattern, RNE edge cases) and, where oracle/_ref is built
from the reference's own Quantization.cpp, bit-for-bit agreement with it.
"""
import ctypes as C

import numpy as np
import pytest

import oracle


def test_roundtrip_all_finite_patterns():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    finite = (bits & 0x7C00) != 0x7C00
    back = oracle.f32_to_f16(oracle.f16_to_f32(bits))
    assert np.array_equal(back[finite], bits[finite])


def test_round_half_even_known_answers():
    # ModelFormatTest.cpp:60-63
    vals = np.array([2.0 ** -25, 1.5 * 2.0 ** -24, 1.0 + 2.0 ** -11, 65520.0],
                    dtype=np.float32)
    assert list(oracle.f32_to_f16(vals)) == [0, 2, 0x3C00, 0x7C00]


def test_matches_numpy_half_on_random_floats():
    # numpy's float16 cast is an independent RNE implementation.
    rng = np.random.default_rng(7)
    x = np.concatenate([rng.standard_normal(200000).astype(np.float32) * s
                        for s in (1e-6, 1e-3, 1.0, 1e3, 6e4)])
    assert np.array_equal(oracle.f32_to_f16(x), x.astype(np.float16).view(np.uint16))
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    finite = (bits & 0x7C00) != 0x7C00
    assert np.array_equal(oracle.f16_to_f32(bits)[finite],
                          bits.view(np.float16).astype(np.float32)[finite])


@pytest.fixture(scope="module")
def ref():
    if not oracle.REF_PATH.exists():
        pytest.skip("oracle/_ref not built (needs /root/reference)")
    lib = C.CDLL(str(oracle.REF_PATH))
    lib.ref_float_to_half.restype = C.c_uint16
    lib.ref_float_to_half.argtypes = [C.c_float]
    lib.ref_half_to_float.restype = C.c_float
    lib.ref_half_to_float.argtypes = [C.c_uint16]
    return lib


def test_matches_reference_quantization_cpp(ref):
    rng = np.random.default_rng(11)
    samples = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10,
        (rng.standard_normal(5000) * 1e-5).astype(np.float32),
        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e9, -1e9, 2.0 ** -24,
                  2.0 ** -25, 3 * 2.0 ** -26, np.inf, -np.inf], np.float32)])
    ours = oracle.f32_to_f16(samples)
    theirs = np.array([ref.ref_float_to_half(float(v)) for v in samples], np.uint16)
    assert np.array_equal(ours, theirs)
    bits = np.arange(0, 65536, 7, dtype=np.uint32).astype(np.uint16)
    ours_f = oracle.f16_to_f32(bits)
    theirs_f = np.array([ref.ref_half_to_float(int(b)) for b in bits], np.float32)
    finite = (bits & 0x7C00) != 0x7C00
    assert np.array_equal(ours_f[finite], theirs_f[finite])
