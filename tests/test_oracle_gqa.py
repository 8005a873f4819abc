"""Pins the oracle's causal GQA functions (oracle.c: orc_gqa_*).

What fixes each result (no test retypes the oracle's loop):
  * closed forms: T=1,P=0 gives O = V[0]; identical keys give the mean of the
    visible V rows; a dominant logit selects its V row;
  * the KV-head map h -> h/(Hq/Hkv): per-KV-head constant V tags every output;
  * invariance: permuting the past rows (all visible to every query);
  * causality: changing cache rows beyond P+t never changes row t;
  * the reference kernel test's own generator and cases
    (tests/FlashAttentionTest.mm:28-36, 108-109) with its tolerance
    |a-e| <= 2e-4 + 5e-4|e| (:80-81) applied to the fp32 and eager paths;
  * the eager fp16 path's rounding points (gqaScores, Reference.metal:303-323;
    gqaSoftmax/gqaValue, Graph.metal:172-230): Hugging Face's own
    eager_attention_forward (transformers, models/qwen3_5, the attention the
    reference's parity harness compares against) run in fp16 on the CPU, on
    inputs whose sums are exact in fp32 in any order, so both must agree bit
    for bit; the same inputs are checked to change when any one rounding
    point (fp16 dot, fp16 scaled score, fp16 probability) is dropped;
  * KvAppend (cacheAppend, Reference.metal:295-301): numpy slice assignment.
"""
import types

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


# ------------------------------------------------ eager fp16 rounding points

def _hf_eager_f16(q, kc, vc, P):
    """transformers' eager_attention_forward in fp16 on the CPU, with the
    additive causal mask its models build (finfo(fp16).min where masked)."""
    import torch
    from transformers.models.qwen3_5.modeling_qwen3_5 import eager_attention_forward
    T, hq, d = q.shape
    n = P + T
    as16 = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.float16))
    tq = as16(q).permute(1, 0, 2)[None]
    tk = as16(kc[:n]).permute(1, 0, 2)[None]
    tv = as16(vc[:n]).permute(1, 0, 2)[None]
    mask = torch.full((T, n), torch.finfo(torch.float16).min, dtype=torch.float16)
    for t in range(T):
        mask[t, :P + t + 1] = 0
    module = types.SimpleNamespace(num_key_value_groups=hq // kc.shape[1], training=False)
    out, _ = eager_attention_forward(module, tq, tk, tv, mask[None, None], d ** -0.5)
    return out[0].numpy().view(np.uint16)


def _exact_sum_case(seed, T, P, hq=4, hkv=2, d=12):
    """Scores q.k = q0 k0 + q1 k1 with dyadic operands (exact in fp32, not
    in fp16: k1 is an odd multiple of 2^-12 next to k0 in [1.5, 3.5]); every
    V row has two ones, so each output channel sums two probabilities
    exactly. d = 12 makes the 1/sqrt(d) scaling inexact."""
    rng = np.random.default_rng(seed)
    n = P + T
    assert n <= d
    q = np.zeros((T, hq, d), np.float32)
    q[:, :, 0] = rng.choice([0.75, 1.0, 1.25], (T, hq))
    q[:, :, 1] = rng.choice([0.5, 1.0], (T, hq))
    k = np.zeros((n, hkv, d), np.float32)
    k[:, :, 0] = rng.integers(3, 8, (n, hkv)) * 0.5
    k[:, :, 1] = (2 * rng.integers(0, 8, (n, hkv)) + 1) * 2.0 ** -12
    v = np.zeros((n, hkv, d), np.float32)
    for j in range(n):
        v[j, :, j] = 1.0
        v[j, :, (j + 1) % d] = 1.0
    return oracle.f32_to_f16(q), oracle.f32_to_f16(k), oracle.f32_to_f16(v)


def _eager_dropping(q, kc, vc, P, drop):
    """The eager path with one rounding point left out -- only to show that
    the cases above tell the rounding points apart."""
    T, hq, d = q.shape
    g = hq // kc.shape[1]
    rnd = lambda x: _f(oracle.f32_to_f16(np.float32(x))).astype(np.float32)
    rs = np.float32(1) / np.sqrt(np.float32(d))
    out = np.zeros(q.shape, np.uint16)
    for t in range(T):
        n = P + t + 1
        for h in range(hq):
            dot = (_f(kc[:n, h // g]) @ _f(q[t, h])).astype(np.float32)
            dot = dot if drop == "dot" else rnd(dot)
            s = (dot * rs).astype(np.float32)
            s = s if drop == "scale" else rnd(s)
            e = np.exp((s - s.max()).astype(np.float64)).astype(np.float32)
            p = (e / np.float32(e.astype(np.float64).sum())).astype(np.float32)
            p = p if drop == "prob" else rnd(p)
            out[t, h] = oracle.f32_to_f16(
                (p.astype(np.float64) @ _f(vc[:n, h // g])).astype(np.float32))
    return out


@pytest.mark.parametrize("T,P", [(1, 11), (1, 6), (3, 8), (4, 0)])
def test_eager_rounding_points_match_hf(T, P):
    changed = {"dot": 0, "scale": 0, "prob": 0}
    for seed in range(4):
        q, k, v = _exact_sum_case(seed, T, P)
        got = oracle.gqa_eager_f16(q, k, v, P)
        assert np.array_equal(got, _hf_eager_f16(q, k, v, P)), seed
        for drop in changed:
            changed[drop] += int(np.sum(_eager_dropping(q, k, v, P, drop) != got))
    # Each rounding point decides some output bits of these cases.
    assert all(changed[d] > 0 for d in changed), changed


def test_eager_close_to_hf_on_normal_inputs():
    """N(0,1) decode at d=256: the summation order differs (the oracle's
    sequential fma chain against torch's blocked sums), which moves an fp32
    dot product across an fp16 rounding boundary now and then, so outputs
    mostly agree bitwise and otherwise by a few fp16 ulps of |o| < 0.5."""
    x = oracle.make_gqa_inputs(21, 1, 16, 4, 256, 300)
    a = _f(oracle.gqa_eager_f16(x.q, x.k_cache, x.v_cache, 300))
    b = _f(_hf_eager_f16(x.q, x.k_cache, x.v_cache, 300))
    assert np.mean(a == b) > 0.95
    assert np.max(np.abs(a - b)) <= 2.0 ** -12


# ------------------------------------------------------------------ KvAppend

@pytest.mark.parametrize("T,hkv,d,past,cap", [(1, 4, 256, 4096, 8192), (7, 2, 12, 0, 9),
                                              (3, 1, 64, 5, 8)])
def test_kv_append_is_slice_assignment(T, hkv, d, past, cap):
    src = oracle.normal_f16(T, past, (T, hkv, d))
    cache = oracle.normal_f16(cap, 9, (cap, hkv, d))
    want = cache.copy()
    want[past:past + T] = src
    oracle.kv_append(src, cache, past)
    assert np.array_equal(cache, want)
