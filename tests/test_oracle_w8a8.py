"""The W8A8 projection path of the oracle, pinned without retyping it.

* quantizeActivation (Graph.metal:33-68) against the formula of the
  reference's own test, tests/MetalReferenceTest.py:88-100 (max|x| / 127,
  round half to even, clamp), with exact ties, zero and non-finite groups.
* linearW8A8 (W8A8.metal:28-113) against the same test's formula -- exact
  int32 group dots times the two scales, summed -- evaluated in float64: the
  fp16 outputs agree to one unit in the last place (the fp32 sum order of the
  kernel's lanes is the only difference); bit for bit where the sum is
  exact: one non-zero group (the single term (float(dot) * a) * w, rounded
  twice), or unit scales with integer sums.
* the storeLinear epilogues (Reference.metal:14-47) against oracle functions
  pinned elsewhere: deltaGates (beta and decay), sigmoidMul (the sigmoid
  columns), the SiLU of causalConv with a one-tap unit filter, and numpy for
  the fp16 product of SiluMul and the fp32 SiLU.
* embeddingW8 / embedding (Graph.metal:16-31, Reference.metal:49-58)
  against numpy gathers.
"""
import numpy as np
import pytest

import oracle


def _rng(seed):
    return np.random.default_rng(seed)


def _f16(x):
    return oracle.f32_to_f16(np.asarray(x, np.float32))


def _reference_quantize(x16):
    """tests/MetalReferenceTest.py:88-96 in numpy (float32 throughout)."""
    x = oracle.f16_to_f32(x16)
    rows, width = x.shape
    groups = (width + 31) // 32
    g = np.zeros((rows, groups * 32), np.float32)
    g[:, :width] = x
    g = g.reshape(rows, groups, 32)
    m = np.abs(g).max(axis=-1)
    scales = np.where(m > 0, m / np.float32(127), np.float32(1)).astype(np.float32)
    q = np.clip(np.rint(g / scales[..., None]), -127, 127).astype(np.int8)
    return q.reshape(rows, groups * 32), scales


@pytest.mark.parametrize("rows,width", [(1, 2560), (3, 70), (5, 32), (2, 1)])
def test_quantize_matches_the_reference_test(rows, width):
    x = _f16(_rng(rows * 1000 + width).standard_normal((rows, width)) * 3)
    q, sc, invalid = oracle.quantize_activation(x)
    q_ref, sc_ref = _reference_quantize(x)
    assert invalid == 0
    assert np.array_equal(sc, sc_ref)
    assert np.array_equal(q, q_ref)


def test_quantize_ties_round_to_even():
    # max |x| = 127 makes the scale 1, so x / scale is x itself.
    vals = [127, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -126.5, 3.25]
    x = _f16(np.array([vals + [0] * 22], np.float32))
    q, sc, _ = oracle.quantize_activation(x)
    assert sc[0, 0] == 1.0
    assert list(q[0, :10]) == [127, 0, 2, 2, 0, -2, -2, 126, -126, 3]


def test_quantize_zero_and_non_finite_groups():
    x = _f16(_rng(3).standard_normal((2, 96)))
    x[0, 32:64] = 0
    x[1, 70] = 0x7C00  # +inf in the third group of row 1
    q, sc, invalid = oracle.quantize_activation(x)
    assert invalid == 1
    assert sc[0, 1] == 1.0 and not q[0, 32:64].any()
    assert sc[1, 2] == 1.0 and not q[1, 64:96].any()
    # the other groups quantize as usual
    q_ref, sc_ref = _reference_quantize(x[:1])
    assert np.array_equal(q[0, :32], q_ref[0, :32]) and sc[0, 0] == sc_ref[0, 0]


def _case(seed, rows, columns, groups, scale_spread=1.0):
    r = _rng(seed)
    x = r.integers(-127, 128, (rows, groups * 32), dtype=np.int8)
    w = r.integers(-127, 128, (columns, groups * 32), dtype=np.int8)
    xs = (r.random((rows, groups), np.float32) * 0.05 * scale_spread + 1e-3).astype(np.float32)
    ws = _f16(r.random((columns, groups)) * 0.02 + 1e-3)
    return x, xs, w, ws


def _float64_reference(x, xs, w, ws):
    """tests/MetalReferenceTest.py:97-99: exact int32 dots times both scales,
    summed (here in float64)."""
    rows, groups = xs.shape
    columns = w.shape[0]
    dots = np.einsum("rgj,cgj->rcg", x.reshape(rows, groups, 32).astype(np.int64),
                     w.reshape(columns, groups, 32).astype(np.int64))
    return (dots * xs[:, None, :].astype(np.float64) *
            oracle.f16_to_f32(ws)[None].astype(np.float64)).sum(-1)


def _ulp_diff(a16, b16):
    a = a16.astype(np.int32)
    b = b16.astype(np.int32)
    # fp16 bit patterns of same-sign finite values are ordered like integers
    return np.abs(a - b)


@pytest.mark.parametrize("rows,columns,groups", [(1, 40, 80), (1, 33, 5), (4, 24, 9),
                                                 (7, 19, 16), (1, 8, 1)])
def test_linear_matches_the_reference_test(rows, columns, groups):
    x, xs, w, ws = _case(rows * 31 + columns, rows, columns, groups)
    got = oracle.linear_w8a8(x, xs, w, ws)
    want = _f16(_float64_reference(x, xs, w, ws))
    same_sign = np.signbit(oracle.f16_to_f32(got)) == np.signbit(oracle.f16_to_f32(want))
    assert np.all(same_sign | (np.abs(oracle.f16_to_f32(want)) < 1e-3))
    assert np.max(_ulp_diff(got[same_sign], want[same_sign])) <= 1


@pytest.mark.parametrize("rows", [1, 3])
def test_linear_single_group_is_exact(rows):
    """One non-zero group: the output is fp16(fp32(fp32(dot) * a) * w)."""
    x, xs, w, ws = _case(7 + rows, rows, 12, 20)
    x = x.copy()
    keep = 13
    for g in range(20):
        if g != keep:
            x[:, 32 * g:32 * g + 32] = 0
    got = oracle.linear_w8a8(x, xs, w, ws)
    dots = (x[:, None, 32 * keep:32 * keep + 32].astype(np.int64) *
            w[None, :, 32 * keep:32 * keep + 32].astype(np.int64)).sum(-1)
    term = (dots.astype(np.float32) * xs[:, keep:keep + 1]).astype(np.float32)
    term = (term * oracle.f16_to_f32(ws[:, keep])[None]).astype(np.float32)
    assert np.array_equal(got, _f16(term))


def test_linear_unit_scales_integer_sums_are_exact_in_both_lane_layouts():
    x, _, w, _ = _case(11, 4, 10, 24)
    xs = np.ones((4, 24), np.float32)
    ws = _f16(np.ones((10, 24)))
    want = _f16((x.astype(np.int64) @ w.astype(np.int64).T).astype(np.float32))
    assert np.array_equal(oracle.linear_w8a8(x, xs, w, ws), want)        # 8 lanes
    for r in range(4):                                                   # 16 lanes
        assert np.array_equal(oracle.linear_w8a8(x[r:r + 1], xs[r:r + 1], w, ws), want[r:r + 1])


def test_linear_shard_offset_and_output_width():
    x, xs, w, ws = _case(5, 3, 7, 6)
    full = oracle.linear_w8a8(x, xs, w, ws)
    out = np.full((3, 20), 0x3C00, np.uint16)
    oracle.linear_w8a8(x, xs, w[2:5], ws[2:5], output=out, first_row=9, output_width=20)
    assert np.array_equal(out[:, 9:12], full[:, 2:5])
    assert np.all(out[:, :9] == 0x3C00) and np.all(out[:, 12:] == 0x3C00)


def _projected(x, xs, w, ws):
    return oracle.linear_w8a8(x, xs, w, ws)


def test_epilogue_delta_gates():
    x, xs, w, ws = _case(21, 5, 32, 8, scale_spread=20)
    p = _projected(x, xs, w, ws)
    a_log = (_rng(1).standard_normal(32) * 0.5).astype(np.float32)
    dt_bias = (_rng(2).standard_normal(32) * 0.5).astype(np.float32)
    beta = oracle.linear_w8a8(x, xs, w, ws, oracle.LINEAR_DELTA_BETA)
    decay = oracle.linear_w8a8(x, xs, w, ws, oracle.LINEAR_DELTA_DECAY, aux=a_log, bias=dt_bias)
    b_ref, _ = oracle.delta_gates(p, p, a_log, dt_bias)
    _, d_ref = oracle.delta_gates(p, p, a_log, dt_bias)
    assert np.array_equal(beta, b_ref)
    assert np.array_equal(decay, d_ref)


def test_epilogue_sigmoid_columns():
    x, xs, w, ws = _case(22, 3, 40, 5, scale_spread=20)
    p = _projected(x, xs, w, ws)
    got = oracle.linear_w8a8(x, xs, w, ws, oracle.LINEAR_SIGMOID_COLUMNS, block=8)
    sig = oracle.sigmoid_mul(p, np.full(p.shape, 0x3C00, np.uint16))  # fp16(logistic) * 1
    odd = (np.arange(40) // 8) % 2 == 1
    assert np.array_equal(got[:, odd], sig[:, odd])
    assert np.array_equal(got[:, ~odd], p[:, ~odd])


def test_epilogue_silu_family():
    x, xs, w, ws = _case(23, 4, 24, 6, scale_spread=20)
    p = _projected(x, xs, w, ws)
    rows, cols = p.shape
    # fp16(silu(p)): causalConv with a one-tap unit filter and SiLU
    one = np.full((rows * cols, 1), 0x3C00, np.uint16)
    s16 = oracle.causal_conv(p.reshape(1, -1), one, np.zeros((rows * cols, 0), np.uint16), True)
    s16 = s16.reshape(rows, cols)
    assert np.array_equal(oracle.linear_w8a8(x, xs, w, ws, oracle.LINEAR_SILU), s16)
    aux = _f16(_rng(4).standard_normal((rows, cols)))
    want = _f16(oracle.f16_to_f32(s16) * oracle.f16_to_f32(aux))
    assert np.array_equal(oracle.linear_w8a8(x, xs, w, ws, oracle.LINEAR_SILU_MUL, aux=aux), want)
    pf = oracle.f16_to_f32(p)
    with np.errstate(over="ignore"):
        e = np.exp(-pf.astype(np.float64)).astype(np.float32)  # correctly rounded fp32 exp
    silu32 = (pf * (np.float32(1) / (np.float32(1) + e)).astype(np.float32)).astype(np.float32)
    assert np.array_equal(oracle.linear_w8a8(x, xs, w, ws, oracle.LINEAR_SILU_F32), silu32)


def test_embedding_w8_and_f16():
    r = _rng(9)
    rows, hidden = 50, 70
    groups = (hidden + 31) // 32
    w = r.integers(-127, 128, (rows, groups * 32), dtype=np.int8)
    sc = _f16(r.random((rows, groups)) * 0.05)
    ids = np.array([3, 49, 0, 60, 17, 3], np.uint32)  # 60 is outside [10, 60) shard rows
    out = np.full((ids.size, hidden), 0x7E00, np.uint16)
    oracle.embedding_w8(ids, w, sc, hidden, first_row=10, output=out)
    for t, i in enumerate(ids):
        if 10 <= i < 60:
            row = i - 10
            want = _f16(w[row, :hidden].astype(np.float32) *
                        oracle.f16_to_f32(sc[row, np.arange(hidden) // 32]))
            assert np.array_equal(out[t], want)
        else:
            assert np.all(out[t] == 0x7E00)
    wf = _f16(r.standard_normal((rows, hidden)))
    outf = oracle.embedding(ids, wf)
    for t, i in enumerate(ids):
        assert np.array_equal(outf[t], wf[i] if i < rows else np.zeros(hidden, np.uint16))
