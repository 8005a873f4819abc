"""Pins the oracle's causalConv (oracle.c: orc_causal_conv), the DeltaNet
front end's depthwise causal convolution with its history rows.

What fixes each result:
  * numpy float64 convolution over [history, input] (a different
    formulation: a sliding window over one concatenated array), then SiLU in
    float64, within the fp16 roundings of the kernel (a shifted window,
    reversed filter or dropped history term is off by O(1));
  * an impulse through a zero history reproduces the filter reversed, bit
    for bit (fp16 products are exact in fp32);
  * kernel size 1 is an elementwise product with no history;
  * splitting the tokens over two calls, the history carried between them,
    gives the same outputs and final history as one call, bit for bit.

And its gatedRmsNorm (orc_gated_rms_norm): Hugging Face's Qwen3_5RMSNormGated
(what the reference's tests compare against) within one fp16 ulp; with an
activated gate of 1 and unit weight it is the rmsNorm of a zero weight, bit
for bit; a zero gate gives zeros.
"""
import numpy as np
import pytest

import oracle


def _data(seed, T, C, k):
    rng = np.random.default_rng(seed)
    f16 = lambda a: oracle.f32_to_f16(a.astype(np.float32))
    return (f16(rng.standard_normal((T, C))), f16(rng.standard_normal((C, k)) * 0.5),
            f16(rng.standard_normal((C, k - 1))))


@pytest.mark.parametrize("T,C,k", [(7, 33, 4), (1, 64, 4), (20, 8, 3), (2, 16, 4)])
@pytest.mark.parametrize("silu", [False, True])
def test_matches_numpy_window(T, C, k, silu):
    x, w, h = _data(T * 7 + k, T, C, k)
    hist = h.copy()
    got = oracle.f16_to_f32(oracle.causal_conv(x, w, hist, silu)).astype(np.float64)
    xs = np.concatenate([oracle.f16_to_f32(h).T, oracle.f16_to_f32(x)]).astype(np.float64)
    wf = oracle.f16_to_f32(w).astype(np.float64)
    acc = np.stack([(xs[t:t + k] * wf.T).sum(0) for t in range(T)])
    if silu:
        a16 = oracle.f16_to_f32(oracle.f32_to_f16(acc.astype(np.float32))).astype(np.float64)
        ref = a16 / (1 + np.exp(-a16))
        tol = 2.0 ** -10 * np.maximum(np.abs(ref), 2.0 ** -14)
    else:
        ref = acc
        tol = 2.0 ** -11 * np.maximum(np.abs(ref), 2.0 ** -14) + 1e-6
    assert np.all(np.abs(got - ref) <= tol)
    # final history: the last k-1 inputs (or old history then inputs)
    want_h = xs[-(k - 1):].T
    assert np.array_equal(oracle.f16_to_f32(hist).astype(np.float64), want_h)


def test_impulse_response_is_the_filter():
    T, C, k = 9, 5, 4
    _, w, _ = _data(1, T, C, k)
    x = np.zeros((T, C), np.uint16)
    x[2] = 0x3C00                                   # 1.0 at t = 2
    hist = np.zeros((C, k - 1), np.uint16)
    out = oracle.causal_conv(x, w, hist, False)
    for m in range(k):
        assert np.array_equal(out[2 + m], w[:, k - 1 - m])
    assert np.all(out[:2] == 0) and np.all(out[2 + k:] == 0)


def test_kernel_size_one():
    x, w, _ = _data(3, 6, 10, 1)
    hist = np.zeros((10, 0), np.uint16)
    out = oracle.f16_to_f32(oracle.causal_conv(x, w, hist, False))
    want = oracle.f16_to_f32(oracle.f32_to_f16(oracle.f16_to_f32(x) * oracle.f16_to_f32(w)[:, 0]))
    assert np.array_equal(out, want)


@pytest.mark.parametrize("split", [1, 2, 5])
def test_split_calls_carry_the_history(split):
    T, C, k = 8, 12, 4
    x, w, h = _data(4, T, C, k)
    h1, h2 = h.copy(), h.copy()
    whole = oracle.causal_conv(x, w, h1, True)
    parts = np.concatenate([oracle.causal_conv(x[:split], w, h2, True),
                            oracle.causal_conv(x[split:], w, h2, True)])
    assert np.array_equal(whole, parts)
    assert np.array_equal(h1, h2)


def _hf_gated(x, gate, w, eps):
    torch = pytest.importorskip("torch")
    m = pytest.importorskip("transformers.models.qwen3_5.modeling_qwen3_5")
    norm = m.Qwen3_5RMSNormGated(x.shape[1], eps=eps)
    norm.load_state_dict({"weight": torch.from_numpy(w)})
    xt = torch.from_numpy(oracle.f16_to_f32(x)).half()
    gt = torch.from_numpy(oracle.f16_to_f32(gate)).half()
    with torch.no_grad():
        return norm(xt, gt).float().numpy().astype(np.float64)


def test_gated_rms_norm_matches_huggingface():
    """Qwen3_5RMSNormGated (the module the reference's tests compare
    against) on the same fp16 inputs: within one fp16 ulp (its mean and
    rsqrt differ from the sequential fma sum and 1/sqrt)."""
    rng = np.random.default_rng(6)
    x = oracle.f32_to_f16(rng.standard_normal((40, 128)).astype(np.float32))
    g = oracle.f32_to_f16((rng.standard_normal((40, 128)) * 2).astype(np.float32))
    w = (1 + 0.2 * rng.standard_normal(128)).astype(np.float32)
    got = oracle.f16_to_f32(oracle.gated_rms_norm(x, g, w)).astype(np.float64)
    ref = _hf_gated(x, g, w, 1e-6)
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(ref), 2.0 ** -14))) - 10)
    assert np.all(np.abs(got - ref) <= 1.01 * ulp)


def test_gated_rms_norm_exact_cases():
    rng = np.random.default_rng(7)
    x = oracle.f32_to_f16(rng.standard_normal((9, 64)).astype(np.float32))
    # activated gate 1 and weight 1: fp16(x * scale), which is rmsNorm with a
    # zero weight (normRope with no rotation), bit for bit
    one = np.ones((9, 64), np.float32)
    got = oracle.gated_rms_norm(x, one, np.ones(64, np.float32))
    assert np.array_equal(got, oracle.norm_rope(x, np.zeros(64, np.float32), 9, 1, 64, 0, 64, 0))
    # gate 0: silu(0) = 0, output +-0
    z = np.zeros((9, 64), np.uint16)
    out = oracle.gated_rms_norm(x, z, np.ones(64, np.float32))
    assert np.all((out & 0x7FFF) == 0)
