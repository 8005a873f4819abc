"""Pins the oracle's causal GQA functions (oracle.c: orc_gqa_*).

What fixes each result (no test retypes the oracle's loop):
  * closed forms: T=1,P=0 gives O = V[0]; identical keys give the mean of the
    visible V rows; a dominant logit selects its V row;
  * the KV-head map h -> h/(Hq/Hkv): per-KV-head constant V tags every output;
  * invariance: permuting the past rows (all visible to every query);
  * causality: changing cache rows beyond P+t never changes row t;
  * the reference kernel test's own generator and cases
    (tests/FlashAttentionTest.mm:28-36, 108-109) with its tolerance
    |a-e| <= 2e-4 + 5e-4|e| (:80-81) applied to the fp32 and eager paths.
"""
import numpy as np
import pytest

import oracle


def _f(a):
    return oracle.f16_to_f32(a).astype(np.float64)


def test_single_token_no_past_is_v0():
    x = oracle.make_gqa_inputs(1, 1, 4, 2, 32, 0)
    out = oracle.gqa_dense_f64(x.q, x.k_cache, x.v_cache, 0)
    for h in range(4):
        np.testing.assert_array_equal(out[0, h], _f(x.v_cache[0, h // 2]))


def test_identical_keys_average_visible_values():
    T, P, hq, hkv, d = 5, 7, 4, 2, 16
    x = oracle.make_gqa_inputs(2, T, hq, hkv, d, P)
    kc = x.k_cache.copy()
    kc[:] = kc[0]
    out = oracle.gqa_dense_f64(x.q, kc, x.v_cache, P)
    vf = _f(x.v_cache)
    for t in range(T):
        for h in range(hq):
            np.testing.assert_allclose(out[t, h], vf[:P + t + 1, h // 2].mean(0),
                                       rtol=0, atol=1e-12)


def test_dominant_logit_selects_row():
    T, P, hq, hkv, d = 1, 40, 2, 1, 16
    x = oracle.make_gqa_inputs(3, T, hq, hkv, d, P)
    kc = np.zeros_like(x.k_cache)
    q = np.zeros_like(x.q)
    one8 = oracle.f32_to_f16(np.array([8.0], np.float32))[0]
    kc[17, 0, 0] = one8
    q[0, :, 0] = one8
    out = oracle.gqa_dense_f64(q, kc, x.v_cache, P)
    # score 64/sqrt(16) = 16 against 0 for the other 40 keys
    w = np.exp(16.0) / (np.exp(16.0) + P)
    expect = w * _f(x.v_cache[17, 0]) + (1 - w) * (
        _f(x.v_cache[:P + 1, 0]).sum(0) - _f(x.v_cache[17, 0])) / P
    for h in range(hq):
        np.testing.assert_allclose(out[0, h], expect, atol=1e-12)
        np.testing.assert_allclose(out[0, h], _f(x.v_cache[17, 0]), atol=1e-4 * 8)


def test_kv_head_map():
    T, P, hq, hkv, d = 3, 5, 8, 2, 8
    x = oracle.make_gqa_inputs(4, T, hq, hkv, d, P)
    vc = np.zeros_like(x.v_cache)
    for j in range(hkv):
        vc[:, j, :] = oracle.f32_to_f16(np.float32(j + 1))
    out = oracle.gqa_dense_f64(x.q, x.k_cache, vc, P)
    for h in range(hq):
        np.testing.assert_allclose(out[:, h], h // (hq // hkv) + 1.0, atol=1e-12)


def test_past_permutation_invariance_and_causality():
    T, P, hq, hkv, d = 4, 9, 4, 2, 16
    x = oracle.make_gqa_inputs(5, T, hq, hkv, d, P, capacity=P + T + 3)
    base = oracle.gqa_dense_f64(x.q, x.k_cache, x.v_cache, P)
    perm = np.random.default_rng(0).permutation(P)
    kc, vc = x.k_cache.copy(), x.v_cache.copy()
    kc[:P], vc[:P] = x.k_cache[perm], x.v_cache[perm]
    np.testing.assert_allclose(oracle.gqa_dense_f64(x.q, kc, vc, P), base, atol=1e-12)
    # rows beyond P+t (later tokens and unused capacity) must not matter for row t
    for t in range(T):
        kc2, vc2 = x.k_cache.copy(), x.v_cache.copy()
        kc2[P + t + 1:] = oracle.normal_f16(9, t, kc2[P + t + 1:].shape)
        vc2[P + t + 1:] = oracle.normal_f16(10, t, vc2[P + t + 1:].shape)
        np.testing.assert_array_equal(oracle.gqa_dense_f64(x.q, kc2, vc2, P)[t], base[t])


def _lcg_case(T, hq, hkv, d, P):
    """Inputs exactly as tests/FlashAttentionTest.mm:28-36 fills them."""
    state = 179531
    nq, nc = T * hq * d, (P + T) * hkv * d
    q, state = oracle.lcg_f16(state, nq)
    k, state = oracle.lcg_f16(state, nc)
    v, state = oracle.lcg_f16(state, nc)
    return (q.reshape(T, hq, d), k.reshape(P + T, hkv, d), v.reshape(P + T, hkv, d))


def test_lcg_generator_threads_state():
    a, s1 = oracle.lcg_f16(179531, 10)
    b, s2 = oracle.lcg_f16(s1, 5)
    c, s3 = oracle.lcg_f16(179531, 15)
    assert np.array_equal(np.concatenate([a, b]), c) and s2 == s3
    vals = oracle.f16_to_f32(c)
    assert np.all(np.abs(vals) <= 2.0) and np.all((vals * 64) == np.round(vals * 64))


@pytest.mark.parametrize("case", [(19, 4, 2, 12, 0), (7, 4, 2, 256, 33)])
def test_reference_kernel_cases_fp32_and_eager(case):
    T, hq, hkv, d, P = case
    q, k, v = _lcg_case(T, hq, hkv, d, P)
    e = oracle.gqa_dense_f64(q, k, v, P)
    f32 = _f(oracle.gqa_f32(q, k, v, P, threads=2))
    assert np.all(np.abs(f32 - e) <= 2e-4 + 5e-4 * np.abs(e))
    eager = _f(oracle.gqa_eager_f16(q, k, v, P))
    assert np.max(np.abs(eager - e)) <= 2e-3


@pytest.mark.parametrize("T,P", [(1, 4096), (1, 300), (33, 100), (128, 0)])
def test_fp32_baseline_matches_dense(T, P):
    x = oracle.make_gqa_inputs(6, T, 16, 4, 256, P)
    e = oracle.gqa_dense_f64(x.q, x.k_cache, x.v_cache, P)
    got = _f(oracle.gqa_f32(x.q, x.k_cache, x.v_cache, P, threads=4))
    assert np.max(np.abs(got - e)) <= 1e-3
