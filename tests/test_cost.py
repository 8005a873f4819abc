"""Pins the algorithmic cost figures (oracle.c: orc_cost_*) that bench.py's
roofline uses.

Known answers from the reference's own tests: KvAppend writes 96 B, CausalGqa
reads 256 B and does 384 MACs for T=3, P=2, Hq=2, Hkv=1, d=8
(tests/GraphIRTest.cpp:99-103); DeltaUpdate does 288 MACs for T=3, Hk=1,
dk=dv=4, Hv=2 (tests/ConverterTest.py:171-179). Where oracle/_ref is built,
the figures must equal the reference's estimateCost (lib/GraphIR/Cost.cpp)
on random shapes, and the published per-configuration FLOP counts of the
benchmark configurations are re-derived.
"""
import ctypes as C

import numpy as np
import pytest

import oracle


def test_reference_known_answers():
    kv = oracle.cost("kv_append", 3, 1, 8)
    g = oracle.cost("causal_gqa", 3, 2, 2, 1, 8)
    assert kv.write_bytes == 96
    assert g.read_bytes == 256 and g.fp_macs == 384
    d = oracle.cost("delta_update", 3, 1, 4, 2, 4)
    assert d.fp_macs == 288


def test_baseline_table_flops():
    # the benchmark configurations' published FLOP counts: FLOPs = 2 x MACs
    assert 2 * oracle.cost("causal_gqa", 128, 0, 16, 4, 256).fp_macs == 135_266_304
    assert 2 * oracle.cost("causal_gqa", 1, 4096, 16, 4, 256).fp_macs == 67_125_248
    assert 2 * oracle.cost("causal_gqa", 2048, 2048, 16, 4, 256).fp_macs == 103_095_992_320
    assert 2 * oracle.cost("delta_update", 1024, 16, 128, 32, 128).fp_macs == 3_221_225_472
    assert 2 * oracle.cost("causal_gqa", 1, 32768, 16, 4, 256).fp_macs == 536_887_296


def test_overflow_rejected():
    with pytest.raises(OverflowError):
        oracle.cost("causal_gqa", 2 ** 40, 2 ** 40, 2 ** 20, 1, 256)


@pytest.fixture(scope="module")
def ref():
    if not oracle.REF_PATH.exists():
        pytest.skip("oracle/_ref not built (needs /root/reference)")
    lib = C.CDLL(str(oracle.REF_PATH))
    u64p = C.POINTER(C.c_uint64)
    lib.ref_gqa_graph.restype = C.c_int
    lib.ref_gqa_graph.argtypes = [C.c_uint64] * 3 + [u64p] * 4 + [C.c_int] * 3 + \
        [u64p, u64p, C.c_char_p, C.c_size_t]
    lib.ref_delta_graph.restype = C.c_int
    lib.ref_delta_graph.argtypes = [C.c_uint64, C.POINTER(C.c_int), u64p, C.POINTER(C.c_int),
                                    u64p, C.c_int, u64p, C.c_char_p, C.c_size_t]
    return lib


def _arr(vals):
    return (C.c_uint64 * len(vals))(*vals)


def test_gqa_cost_matches_reference(ref):
    rng = np.random.default_rng(5)
    for _ in range(200):
        T = int(rng.integers(1, 300))
        P = int(rng.integers(0, 5000))
        hkv = int(rng.integers(1, 5))
        hq = hkv * int(rng.integers(1, 5))
        d = int(rng.integers(1, 300))
        cap = P + T + int(rng.integers(0, 10))
        cost = (C.c_uint64 * 6)()
        eff = (C.c_uint64 * 6)()
        mask = ref.ref_gqa_graph(T, P, cap, _arr([T, hq, d]), _arr([T, hkv, d]),
                                 _arr([T, hkv, d]), _arr([cap, hkv, d]), 2, 2, 0,
                                 cost, eff, None, 0)
        assert mask == 7
        kv = oracle.cost("kv_append", T, hkv, d)
        g = oracle.cost("causal_gqa", T, P, hq, hkv, d)
        assert (cost[0], cost[1]) == (kv.write_bytes, kv.read_bytes)
        assert (cost[2], cost[3], cost[4], cost[5]) == (g.fp_macs, g.read_bytes,
                                                        g.write_bytes, g.exp)


def test_delta_cost_matches_reference(ref):
    rng = np.random.default_rng(6)
    for _ in range(100):
        T = int(rng.integers(1, 2000))
        hk = int(rng.integers(1, 5))
        hv = hk * int(rng.integers(1, 4))
        dk = int(rng.integers(1, 200))
        dv = int(rng.integers(1, 200))
        ranks = (C.c_int * 5)(2, 2, 2, 2, 2)
        dims = _arr([T, hk * dk, 0, 0, T, hk * dk, 0, 0, T, hv * dv, 0, 0,
                     T, hv, 0, 0, T, hv, 0, 0])
        elems = (C.c_int * 5)(3, 3, 2, 3, 3)
        cost = (C.c_uint64 * 4)()
        assert ref.ref_delta_graph(T, ranks, dims, elems, _arr([hv, dk, dv]), 3,
                                   cost, None, 0) == 1
        d = oracle.cost("delta_update", T, hk, dk, hv, dv)
        assert (cost[0], cost[1], cost[2], cost[3]) == (d.fp_macs, d.read_bytes,
                                                        d.write_bytes, d.scalar_ops)
