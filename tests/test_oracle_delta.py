"""Pins the oracle's gated delta rule (oracle.c: orc_delta_*), gates and norm.

What fixes each result:
  * the matrix form of the rule (docs/architecture.md:124-133),
    S_t = a_t (I - b_t k_t k_t^T) S_{t-1} + b_t k_t v_t^T, y_t = S_t^T q_t,
    evaluated with numpy matrix products on tiny shapes -- a different
    formulation from the oracle's per-column loop (Reference.metal:182-197);
  * beta = 0: pure decay, S_T = (prod a) S_0;
  * decay = 1, beta = 1, orthonormal keys, S_0 = 0: exact retrieval q = k_i
    gives y = v_i (the delta rule's defining property);
  * the chunk-wise WY form (a different algorithm) equals the recurrence for
    chunk sizes 1, 16, 64 and a ragged last chunk;
  * linearity in v for S_0 = 0;
  * the fp32 CPU baseline stays within fp32 rounding of the double oracle;
  * gates against numpy's sigmoid / log1p and the fp16 rounding of beta;
    L2 norm against numpy.
"""
import numpy as np
import pytest

import oracle


def _tiny(seed, T, hk, dk, hv, dv, state_std=0.3):
    return oracle.make_delta_inputs(seed, T, hk, dk, hv, dv, state_std)


def _matrix_form(x, hk, dk, hv, dv):
    T = x.q.shape[0]
    S = x.state.astype(np.float64).copy()
    v = oracle.f16_to_f32(x.v).astype(np.float64)
    out = np.zeros((T, hv * dv))
    for t in range(T):
        for h in range(hv):
            kh = h // (hv // hk)
            k = x.k[t, kh * dk:(kh + 1) * dk].astype(np.float64)
            q = x.q[t, kh * dk:(kh + 1) * dk].astype(np.float64)
            a, b = float(x.decay[t, h]), float(x.beta[t, h])
            S[h] = a * (np.eye(dk) - b * np.outer(k, k)) @ S[h] + b * np.outer(k, v[t, h * dv:(h + 1) * dv])
            out[t, h * dv:(h + 1) * dv] = S[h].T @ q
    return out, S


@pytest.mark.parametrize("shape", [(6, 1, 4, 2, 4), (9, 2, 7, 4, 5), (5, 1, 8, 1, 3)])
def test_recurrence_matches_matrix_form(shape):
    T, hk, dk, hv, dv = shape
    x = _tiny(21, *shape)
    out, st = oracle.delta_recurrent_f64(x.q, x.k, x.v, x.beta, x.decay, x.state)
    mo, ms = _matrix_form(x, hk, dk, hv, dv)
    np.testing.assert_allclose(out, mo, atol=1e-12)
    np.testing.assert_allclose(st, ms, atol=1e-12)


def test_beta_zero_is_pure_decay():
    T, hk, dk, hv, dv = 7, 2, 8, 4, 6
    x = _tiny(22, T, hk, dk, hv, dv)
    beta = np.zeros_like(x.beta)
    out, st = oracle.delta_recurrent_f64(x.q, x.k, x.v, beta, x.decay, x.state)
    prod = np.prod(x.decay.astype(np.float64), axis=0)
    np.testing.assert_allclose(st, x.state * prod[:, None, None], rtol=1e-12, atol=0)
    cum = np.cumprod(x.decay.astype(np.float64), axis=0)
    for h in range(hv):
        kh = h // (hv // hk)
        q = x.q[:, kh * dk:(kh + 1) * dk].astype(np.float64)
        want = cum[:, h:h + 1] * (q @ x.state[h].astype(np.float64))
        np.testing.assert_allclose(out[:, h * dv:(h + 1) * dv], want, atol=1e-12)


def test_orthonormal_keys_retrieve_values():
    T, dk, dv = 8, 8, 5
    q = np.zeros((T, dk), np.float32)
    k = np.eye(dk, dtype=np.float32)[:T]
    v = oracle.normal_f16(3, 3, (T, dv))
    ones = np.ones((T, 1), np.float32)
    st0 = np.zeros((1, dk, dv), np.float32)
    _, st = oracle.delta_recurrent_f64(q, k, v, ones, ones, st0)
    np.testing.assert_allclose(st[0], oracle.f16_to_f32(v).astype(np.float64), atol=0)
    # query token t with q = k_i returns v_i once key i is written
    q2 = np.eye(dk, dtype=np.float32)[[3]]
    out, _ = oracle.delta_recurrent_f64(q2, np.zeros_like(q2), np.zeros((1, dv), np.uint16),
                                        np.zeros((1, 1), np.float32), ones[:1], st.astype(np.float32))
    np.testing.assert_allclose(out[0], oracle.f16_to_f32(v[3]), atol=1e-12)


@pytest.mark.parametrize("chunk", [1, 16, 64])
def test_chunked_equals_recurrent(chunk):
    T, hk, dk, hv, dv = 150, 2, 16, 4, 8
    x = _tiny(23, T, hk, dk, hv, dv)
    ro, rs = oracle.delta_recurrent_f64(x.q, x.k, x.v, x.beta, x.decay, x.state)
    co, cs = oracle.delta_chunked_f64(x.q, x.k, x.v, x.beta, x.decay, x.state, chunk)
    np.testing.assert_allclose(co, ro, atol=1e-9)
    np.testing.assert_allclose(cs, rs, atol=1e-9)


def test_chunked_handles_zero_decay():
    T, hk, dk, hv, dv = 40, 1, 8, 2, 4
    x = _tiny(24, T, hk, dk, hv, dv)
    decay = x.decay.copy()
    decay[[3, 17, 18], 0] = 0.0
    ro, rs = oracle.delta_recurrent_f64(x.q, x.k, x.v, x.beta, decay, x.state)
    co, cs = oracle.delta_chunked_f64(x.q, x.k, x.v, x.beta, decay, x.state, 16)
    assert np.all(np.isfinite(co)) and np.all(np.isfinite(cs))
    np.testing.assert_allclose(co, ro, atol=1e-9)
    np.testing.assert_allclose(cs, rs, atol=1e-9)


def test_linear_in_v_from_zero_state():
    T, hk, dk, hv, dv = 12, 1, 8, 2, 4
    x = _tiny(25, T, hk, dk, hv, dv, state_std=0.0)
    rng = np.random.default_rng(1)
    v1 = rng.integers(-8, 8, (T, hv * dv)).astype(np.float16).view(np.uint16)
    v2 = rng.integers(-8, 8, (T, hv * dv)).astype(np.float16).view(np.uint16)
    v12 = (v1.view(np.float16) + v2.view(np.float16)).view(np.uint16)
    args = (x.beta, x.decay, x.state)
    o1, s1 = oracle.delta_recurrent_f64(x.q, x.k, v1, *args)
    o2, s2 = oracle.delta_recurrent_f64(x.q, x.k, v2, *args)
    o12, s12 = oracle.delta_recurrent_f64(x.q, x.k, v12, *args)
    np.testing.assert_allclose(o12, o1 + o2, atol=1e-10)
    np.testing.assert_allclose(s12, s1 + s2, atol=1e-10)


def test_fp32_baseline_close_to_double():
    T, hk, dk, hv, dv = 64, 2, 32, 4, 16
    x = _tiny(26, T, hk, dk, hv, dv)
    ro, rs = oracle.delta_recurrent_f64(x.q, x.k, x.v, x.beta, x.decay, x.state)
    fo, fs = oracle.delta_recurrent_f32(x.q, x.k, x.v, x.beta, x.decay, x.state, threads=2)
    assert np.max(np.abs(oracle.f16_to_f32(fo) - ro)) <= 2e-3
    assert np.max(np.abs(fs - rs)) / np.max(np.abs(rs)) <= 1e-5


def test_gates_and_l2norm():
    T, hv = 64, 8
    a = oracle.normal_f16(1, 1, (T, hv), 0, 3)
    b = oracle.normal_f16(1, 2, (T, hv), 0, 3)
    a_log = np.linspace(-2, 1, hv).astype(np.float32)
    dt_bias = np.linspace(-1, 1, hv).astype(np.float32)
    beta, decay = oracle.delta_gates(a, b, a_log, dt_bias)
    af, bf = oracle.f16_to_f32(a).astype(np.float64), oracle.f16_to_f32(b).astype(np.float64)
    sig = 1 / (1 + np.exp(-bf))
    # beta = fp16(sigmoid(b)), stored as f32 (Graph.metal:142)
    assert np.max(np.abs(beta - sig)) <= 2 ** -12 + 1e-7
    assert np.array_equal(oracle.f16_to_f32(oracle.f32_to_f16(beta)), beta)
    sp = np.log1p(np.exp(-np.abs(af + dt_bias))) + np.maximum(af + dt_bias, 0)
    np.testing.assert_allclose(decay, np.exp(-np.exp(a_log) * sp), rtol=1e-5)
    x = oracle.normal_f16(2, 3, (5, 4 * 16))
    got = oracle.l2norm_f32(x, 16, 1e-6, 0.25)
    xf = oracle.f16_to_f32(x).astype(np.float64).reshape(5, 4, 16)
    want = xf / np.sqrt((xf ** 2).sum(-1, keepdims=True) + 1e-6) * 0.25
    np.testing.assert_allclose(got.reshape(5, 4, 16), want, rtol=1e-6, atol=1e-7)
