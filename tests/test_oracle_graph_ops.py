"""The graph plan's remaining ops in the oracle, pinned without retyping them.

* residualAdd / multiplyF16 (Reference.metal:119-126, Graph.metal:87-94)
  against numpy: the fp32 sum or product of two fp16 values, rounded to fp16.
* siluF16 (Graph.metal:70-76) against causalConv with a one-tap unit filter
  and SiLU (pinned with the DeltaNet front end); swiGlu (Reference.metal:
  128-135) against that SiLU times the up value in numpy.
* copyHalfView (Graph.metal:1-14) against numpy's strided views.
* linearF16 (Reference.metal:61-103): integer-valued operands whose partial
  sums are exact equal numpy's integer product bit for bit; one non-zero
  term is the single rounded product; random operands stay within an fp32
  rounding bound of the float64 product; the epilogues go through the same
  storeLinear as the W8A8 projections.
"""
import numpy as np
import pytest

import oracle


def _f16(x):
    return oracle.f32_to_f16(np.asarray(x, np.float32))


def _rand16(seed, shape, scale=1.0):
    return _f16(np.random.default_rng(seed).standard_normal(shape) * scale)


def _specials():
    # zeros, subnormals, the fp16 maximum, infinities and a NaN
    return np.array([0x0000, 0x8000, 0x0001, 0x83FF, 0x7BFF, 0xFBFF, 0x7C00, 0xFC00, 0x7E00,
                     0x3C00, 0xBC00, 0x3555], np.uint16)


@pytest.mark.parametrize("kind", ["add", "multiply"])
def test_add_and_multiply_match_numpy(kind):
    a = np.concatenate([_rand16(1, 4000, 100.0), _specials(), _specials()])
    b = np.concatenate([_rand16(2, 4000, 100.0), _specials(), _specials()[::-1]])
    fa, fb = oracle.f16_to_f32(a), oracle.f16_to_f32(b)
    with np.errstate(all="ignore"):
        want = (fa + fb if kind == "add" else fa * fb).astype(np.float32).astype(np.float16)
    got = oracle.elementwise(kind, a, b)
    assert np.array_equal(got, want.view(np.uint16))


def test_silu_and_swiglu_match_the_pinned_silu():
    a = np.concatenate([_rand16(3, 3000, 6.0), _specials()])
    b = _rand16(4, a.size, 2.0)
    one = np.full((a.size, 1), 0x3C00, np.uint16)
    pinned = oracle.causal_conv(a.reshape(1, -1), one, np.zeros((a.size, 0), np.uint16),
                                True).reshape(-1)
    assert np.array_equal(oracle.elementwise("silu", a), pinned)
    with np.errstate(all="ignore"):
        want = (oracle.f16_to_f32(pinned) * oracle.f16_to_f32(b)).astype(np.float16)
    assert np.array_equal(oracle.elementwise("swiglu", a, b), want.view(np.uint16))


@pytest.mark.parametrize("shape,axis,begin,length", [((3, 4, 24), 2, 12, 12), ((3, 4, 24), 2, 0, 12),
                                                     ((5, 33), 1, 7, 9), ((6, 10), 0, 2, 3)])
def test_copy_half_view_matches_numpy(shape, axis, begin, length):
    src = np.arange(int(np.prod(shape)), dtype=np.uint16).reshape(shape)
    index = [slice(None)] * len(shape)
    index[axis] = slice(begin, begin + length)
    view = src[tuple(index)]
    strides = [s // 2 for s in view.strides]
    offset = begin * strides[axis]
    got = oracle.copy_half_view(src, view.shape, strides, offset)
    assert np.array_equal(got, np.ascontiguousarray(view))


def test_linear_f16_integer_sums_are_exact():
    r = np.random.default_rng(5)
    x = r.integers(-8, 9, (5, 70)).astype(np.float32)
    w = r.integers(-8, 9, (13, 70)).astype(np.float32)
    want = _f16((x.astype(np.int64) @ w.astype(np.int64).T).astype(np.float32))
    assert np.array_equal(oracle.linear_f16(_f16(x), _f16(w)), want)


def test_linear_f16_single_term_and_float64_bound():
    r = np.random.default_rng(6)
    x = _rand16(7, (3, 50))
    w = _rand16(8, (9, 50))
    one = np.zeros_like(x)
    one[:, 17] = x[:, 17]
    term = (oracle.f16_to_f32(one[:, 17])[:, None] * oracle.f16_to_f32(w[:, 17])[None]).astype(
        np.float32)
    assert np.array_equal(oracle.linear_f16(one, w), _f16(term))
    got = oracle.f16_to_f32(oracle.linear_f16(x, w)).astype(np.float64)
    exact = oracle.f16_to_f32(x).astype(np.float64) @ oracle.f16_to_f32(w).astype(np.float64).T
    # 50 fp32 fma roundings plus the fp16 rounding of the result
    bound = 50 * 2.0 ** -24 * (np.abs(oracle.f16_to_f32(x)).astype(np.float64) @
                               np.abs(oracle.f16_to_f32(w)).astype(np.float64).T)
    assert np.all(np.abs(got - exact) <= bound + np.abs(exact) * 2.0 ** -11 + 1e-7)
    del r


def test_linear_f16_epilogue_and_shard():
    x = _rand16(9, (4, 40), 2.0)
    w = _rand16(10, (12, 40), 0.5)
    p = oracle.linear_f16(x, w)
    aux = _rand16(11, (4, 12))
    want = oracle.elementwise("swiglu", p, aux)
    assert np.array_equal(oracle.linear_f16(x, w, oracle.LINEAR_SILU_MUL, aux=aux), want)
    out = np.full((4, 30), 0x3C00, np.uint16)
    oracle.linear_f16(x, w[3:7], output=out, first_row=20, output_width=30)
    assert np.array_equal(out[:, 20:24], p[:, 3:7])
    assert np.all(out[:, :20] == 0x3C00) and np.all(out[:, 24:] == 0x3C00)


def test_partial_rope_of_the_rms_norm_is_norm_rope():
    """normRope (Reference.metal:271-293, pinned with the attention rows)
    rounds the normalised value to fp16 before rotatePair, which is exactly
    partialRope applied to rmsNorm's output."""
    T, H, d, past = 5, 3, 24, 17
    x = _rand16(12, (T * H, d), 3.0)
    w = (np.random.default_rng(13).standard_normal(d) * 0.2).astype(np.float32)
    normed = oracle.rms_norm(x, w)
    assert np.array_equal(normed, oracle.norm_rope(x, w, T, H, d, 0, d, 0))
    got = oracle.partial_rope(normed.reshape(T, H, d), 8, past)
    assert np.array_equal(got.reshape(T * H, d), oracle.norm_rope(x, w, T, H, d, 8, d, past))
    assert np.array_equal(got.reshape(T * H, d)[:, 8:], normed[:, 8:])
