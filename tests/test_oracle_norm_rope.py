"""Pins the oracle's normRope and sigmoidMul (oracle.c: orc_norm_rope,
orc_sigmoid_mul).

What fixes each result:
  * Hugging Face's own Qwen3.5 modules -- Qwen3_5RMSNorm and
    Qwen3_5TextRotaryEmbedding + apply_rotary_pos_emb, the implementation the
    reference's tests compare against (tests/MetalReferenceTest.py:148,
    :222) -- evaluated in float32 on the same fp16 inputs. They use another
    formulation (rotate_half, a frequency table multiplied instead of
    divided, a tree-summed mean) and no fp16 rounding inside, so agreement is
    within a few fp16 ulps of each rotated pair; a wrong sign, a swapped pair
    index, a wrong position or a missing (1 + w) is off by O(1);
  * position 0 rotates by angle 0 (cos = 1, sin = 0 exactly), so the output
    equals the norm with rotaryDim = 0, bit for bit;
  * rows land at (outputStart * heads + row) * headDim and nothing else is
    written; the half of each input row past headDim (the gate, with
    headStride = 2 * headDim) is never read;
  * sigmoidMul against float64 numpy within the final rounding, and its exact
    cases: gate 0 halves the input, a large gate passes it, a very negative
    gate gives 0.
"""
import numpy as np
import pytest

import oracle


def _ulp16(v):
    v = np.maximum(np.abs(v), 2.0 ** -14)
    return 2.0 ** (np.floor(np.log2(v)) - 10)


def _inputs(seed, tokens, heads, head_dim, stride):
    rng = np.random.default_rng(seed)
    x = oracle.f32_to_f16((rng.standard_normal((tokens * heads, stride)) * 0.7).astype(np.float32))
    w = (rng.standard_normal(head_dim) * 0.2).astype(np.float32)
    return x, w


def _hf(x, w, tokens, heads, head_dim, rotary_dim, past, eps, theta):
    torch = pytest.importorskip("torch")
    m = pytest.importorskip("transformers.models.qwen3_5.modeling_qwen3_5")
    cfg_mod = pytest.importorskip("transformers.models.qwen3_5.configuration_qwen3_5")
    cfg = cfg_mod.Qwen3_5TextConfig(
        hidden_size=heads * head_dim, num_attention_heads=heads, num_key_value_heads=heads,
        head_dim=head_dim, rms_norm_eps=eps, max_position_embeddings=4096,
        rope_parameters={"rope_type": "default", "mrope_interleaved": True,
                         "partial_rotary_factor": rotary_dim / head_dim,
                         "mrope_section": [1, 1, 1] if rotary_dim >= 12 else [rotary_dim // 2, 0, 0],
                         "rope_theta": theta})
    norm = m.Qwen3_5RMSNorm(head_dim, eps)
    norm.load_state_dict({"weight": torch.from_numpy(w)})
    rope = m.Qwen3_5TextRotaryEmbedding(cfg)
    xf = torch.from_numpy(oracle.f16_to_f32(x[:, :head_dim]).reshape(tokens, heads, head_dim))
    with torch.no_grad():
        y = norm(xf)                                  # [T, H, d] float32
        positions = torch.arange(past, past + tokens)
        cos, sin = rope(y, positions[None, None])
        q = y.transpose(0, 1)[None]                   # [1, H, T, d]
        q, _ = m.apply_rotary_pos_emb(q, q, cos, sin)
    return q[0].transpose(0, 1).reshape(tokens * heads, head_dim).numpy().astype(np.float64)


@pytest.mark.parametrize("tokens,heads,head_dim,rotary_dim,past",
                         [(5, 4, 256, 64, 0), (3, 2, 128, 64, 37), (4, 3, 64, 32, 250)])
def test_norm_rope_matches_huggingface(tokens, heads, head_dim, rotary_dim, past):
    eps, theta = 1e-6, 1e7
    x, w = _inputs(1, tokens, heads, head_dim, 2 * head_dim)
    got = oracle.f16_to_f32(oracle.norm_rope(x, w, tokens, heads, head_dim, rotary_dim,
                                             2 * head_dim, past, eps, theta)).astype(np.float64)
    ref = _hf(x, w, tokens, heads, head_dim, rotary_dim, past, eps, theta)
    half = rotary_dim // 2
    pair = np.maximum(np.abs(ref[:, :half]), np.abs(ref[:, half:rotary_dim]))
    tol_rot = 4 * _ulp16(np.concatenate([pair, pair], axis=1))
    assert np.all(np.abs(got[:, :rotary_dim] - ref[:, :rotary_dim]) <= tol_rot)
    tol_pass = 1.01 * _ulp16(ref[:, rotary_dim:])
    assert np.all(np.abs(got[:, rotary_dim:] - ref[:, rotary_dim:]) <= tol_pass)


def test_position_zero_is_the_norm():
    x, w = _inputs(2, 1, 8, 256, 256)
    rot = oracle.norm_rope(x, w, 1, 8, 256, 64, 256, 0)
    plain = oracle.norm_rope(x, w, 1, 8, 256, 0, 256, 0)
    assert np.array_equal(rot, plain)
    # ... and positions after 0 do rotate
    assert not np.array_equal(oracle.norm_rope(x, w, 1, 8, 256, 64, 256, 1), plain)


def test_output_placement_and_stride():
    tokens, heads, d, start = 3, 4, 128, 5
    x, w = _inputs(3, tokens, heads, d, 2 * d)
    out = np.full(((start + tokens + 2) * heads, d), 0x7E00, np.uint16)
    oracle.norm_rope(x, w, tokens, heads, d, 64, 2 * d, start, output=out, output_start=start)
    assert np.all(out[:start * heads] == 0x7E00)
    assert np.all(out[(start + tokens) * heads:] == 0x7E00)
    y = x.copy()
    y[:, d:] = 0xFC00                                 # the gate half: never read
    ref = oracle.norm_rope(y, w, tokens, heads, d, 64, 2 * d, start)
    assert np.array_equal(out[start * heads:(start + tokens) * heads], ref)


def test_sigmoid_mul():
    rng = np.random.default_rng(4)
    g = oracle.f32_to_f16((rng.standard_normal(4096) * 4).astype(np.float32))
    x = oracle.f32_to_f16(rng.standard_normal(4096).astype(np.float32))
    got = oracle.f16_to_f32(oracle.sigmoid_mul(g, x)).astype(np.float64)
    gf = oracle.f16_to_f32(g).astype(np.float64)
    s16 = oracle.f16_to_f32(oracle.f32_to_f16((1 / (1 + np.exp(-gf))).astype(np.float32)))
    ref = s16.astype(np.float64) * oracle.f16_to_f32(x)
    assert np.all(np.abs(got - ref) <= 0.5 * _ulp16(ref) + 2.0 ** -25)
    xs = oracle.f32_to_f16(np.array([1.5, -3.25, 0.1, 7.0], np.float32))
    for gate, expect in ((0.0, 0.5), (20.0, 1.0), (-20.0, 0.0)):
        gb = oracle.f32_to_f16(np.full(4, gate, np.float32))
        out = oracle.f16_to_f32(oracle.sigmoid_mul(gb, xs))
        assert np.array_equal(out, (oracle.f16_to_f32(xs) * expect).astype(np.float32))
