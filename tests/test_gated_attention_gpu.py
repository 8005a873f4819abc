"""GPU parity of the fused attention block (llmi_hip_gated_attention).

The reference runs the block as separate dispatches (MetalReferenceGraph.mm:
307-337; Qwen35ModelBuilder.cpp:175-197): normRope of the projected q rows
(headStride 2d, the gate interleaved), normRope of the new keys straight into
the key cache, cacheAppend of the values, the attention, and the sigmoid gate
(applyGqa's, Reference.metal:350-353; sigmoidMul in the graph lowering). The
same sequence through this backend's standalone launches -- each bit-exact
with the oracle in the row-op tests -- must give exactly the fused call's
output and cache bits, at the decode (one launch + merge) and prefill
(K normRope + append, then the MFMA prefill with q normRope in its load and
the gate in its store) shapes. Two cases are also checked end to end against
the oracle: oracle normRope and sigmoidMul around the double-precision
attention, within the north-star 2e-3. The activated form
(llmi_hip_gated_attention_activated: the gate half already holds
fp16(logistic(.)), as the q projection's sigmoid-columns epilogue leaves it)
must equal the same unfused ops with multiplyF16 in place of sigmoidMul.
"""
import numpy as np
import pytest
import torch

import oracle
from llminfer_amd import _lib, ops
from tests.conftest import torch_to_u16, u16_to_torch

pytestmark = pytest.mark.gpu
EPS, THETA = 1e-6, 1e7


def _case(seed, T, hq, hkv, d, past):
    rng = np.random.default_rng(seed)
    x = oracle.make_gqa_inputs(seed, T, hq, hkv, d, past, capacity=past + T + 3)
    q_proj = oracle.normal_f16(seed, 30, (T, hq, 2 * d))
    k_proj = oracle.normal_f16(seed, 31, (T, hkv, d))
    qw = (0.2 * rng.standard_normal(d)).astype(np.float32)
    kw = (0.2 * rng.standard_normal(d)).astype(np.float32)
    return x, q_proj, k_proj, qw, kw


def _run_both(gpu, x, q_proj, k_proj, qw, kw, past, rot):
    T, hq, d2 = q_proj.shape
    d = d2 // 2
    hkv = k_proj.shape[1]
    f32 = lambda a: torch.from_numpy(a).to(gpu)
    qp, kp, vn = u16_to_torch(q_proj, gpu), u16_to_torch(k_proj, gpu), u16_to_torch(x.v_new, gpu)
    base_k, base_v = u16_to_torch(x.k_cache, gpu), u16_to_torch(x.v_cache, gpu)
    base_k[past:] = 0
    base_v[past:] = 0
    # Unfused, in the reference's order.
    kc, vc = base_k.clone(), base_v.clone()
    qn = torch.empty((T, hq, d), dtype=torch.float16, device=gpu)
    ops.norm_rope(qp, f32(qw), qn, past, rot, EPS, THETA, head_dim=d)
    ops.norm_rope(kp, f32(kw), kc, past, rot, EPS, THETA, output_start=past)
    ops.cache_append(vn, vc, past * hkv * d)
    attn = ops.causal_gqa(qn, kc, vc, past)
    gate = qp[:, :, d:].contiguous()
    ref = torch.empty_like(attn)
    ops.sigmoid_mul(gate, attn, ref)
    # Fused.
    kc2, vc2 = base_k.clone(), base_v.clone()
    out = ops.gated_attention(qp, kp, vn, f32(qw), f32(kw), kc2, vc2, past, rot, EPS, THETA)
    torch.cuda.synchronize()
    return ref, out, (kc, vc), (kc2, vc2)


@pytest.mark.parametrize("T,past,shape,rot", [
    (1, 0, (16, 4, 256), 64), (1, 33, (16, 4, 256), 64), (1, 4096, (16, 4, 256), 64),
    (1, 32768, (16, 4, 256), 64), (1, 700, (8, 4, 128), 32), (1, 300, (16, 8, 256), 64),
    (40, 24, (16, 4, 256), 64), (128, 0, (16, 4, 256), 64), (2048, 2048, (16, 4, 256), 64),
    (65, 17, (16, 4, 128), 32), (33, 100, (8, 4, 256), 128),
    (100, 37, (64, 16, 256), 64), (130, 64, (64, 16, 256), 128)])
def test_fused_block_equals_the_unfused_ops(gpu, T, past, shape, rot):
    hq, hkv, d = shape
    print(f"gated attention T={T} past={past} shape={shape} rot={rot}", flush=True)
    x, q_proj, k_proj, qw, kw = _case(500 + T + past, T, hq, hkv, d, past)
    ref, out, caches_ref, caches = _run_both(gpu, x, q_proj, k_proj, qw, kw, past, rot)
    assert torch.equal(caches_ref[0], caches[0]), "key cache differs"
    assert torch.equal(caches_ref[1], caches[1]), "value cache differs"
    assert torch.equal(ref, out), "output differs from the unfused ops"
    names = ops.kernel_names(_lib.OP_GATED_ATTENTION, _lib.GqaParams(T, hq, hkv, d, past))
    if T == 1:
        assert names[0] == "gqaDecodeGated"
    else:
        assert names == ["normRopeTile", "cacheAppend", "gqaPrefillGated"]


@pytest.mark.parametrize("T,past,hq,hkv", [(1, 4096, 16, 4), (40, 24, 16, 4), (100, 37, 64, 16)])
def test_fused_block_against_the_oracle(gpu, T, past, hq, hkv):
    d, rot = 256, 64
    print(f"gated attention vs oracle T={T} past={past}", flush=True)
    x, q_proj, k_proj, qw, kw = _case(900 + T, T, hq, hkv, d, past)
    _, out, _, (kc, vc) = _run_both(gpu, x, q_proj, k_proj, qw, kw, past, rot)
    qn = oracle.norm_rope(q_proj, qw, T, hq, d, rot, 2 * d, past, EPS, THETA).reshape(T, hq, d)
    kcache = x.k_cache.copy()
    oracle.norm_rope(k_proj, kw, T, hkv, d, rot, d, past, EPS, THETA, output=kcache,
                     output_start=past)
    assert np.array_equal(torch_to_u16(kc), kcache)
    attn = oracle.gqa_dense_f64(qn, kcache, x.v_cache, past)
    gate = oracle.f16_to_f32(q_proj[:, :, d:]).astype(np.float64)
    want = attn / (1.0 + np.exp(-gate))
    got = oracle.f16_to_f32(torch_to_u16(out)).astype(np.float64)
    assert np.max(np.abs(got - want)) <= 2e-3


@pytest.mark.parametrize("T,past,shape,rot", [
    (1, 0, (16, 4, 256), 64), (1, 33, (16, 4, 256), 64), (1, 512, (16, 4, 256), 64),
    (1, 4096, (16, 4, 256), 64), (1, 700, (8, 4, 128), 32), (40, 24, (16, 4, 256), 64),
    (65, 17, (16, 4, 128), 32)])
def test_activated_block_equals_the_unfused_ops(gpu, T, past, shape, rot):
    """llmi_hip_gated_attention_activated: the gate half of q_proj already
    holds fp16(logistic(gate)) (here made by sigmoidMul against ones, the
    values the q projection's sigmoid-columns epilogue stores); the output
    must equal multiplyF16(gate, attention) after the same unfused normRope,
    append and attention, bit for bit, with the caches."""
    hq, hkv, d = shape
    print(f"activated gated attention T={T} past={past} shape={shape} rot={rot}", flush=True)
    x, q_proj, k_proj, qw, kw = _case(700 + T + past, T, hq, hkv, d, past)
    f32 = lambda a: torch.from_numpy(a).to(gpu)
    qp = u16_to_torch(q_proj, gpu)
    act = torch.empty((T, hq, d), dtype=torch.float16, device=gpu)
    ops.sigmoid_mul(qp[:, :, d:].contiguous(), torch.ones_like(act), act)
    qp[:, :, d:] = act
    kp, vn = u16_to_torch(k_proj, gpu), u16_to_torch(x.v_new, gpu)
    base_k, base_v = u16_to_torch(x.k_cache, gpu), u16_to_torch(x.v_cache, gpu)
    base_k[past:] = 0
    base_v[past:] = 0
    kc, vc = base_k.clone(), base_v.clone()
    qn = torch.empty((T, hq, d), dtype=torch.float16, device=gpu)
    ops.norm_rope(qp, f32(qw), qn, past, rot, EPS, THETA, head_dim=d)
    ops.norm_rope(kp, f32(kw), kc, past, rot, EPS, THETA, output_start=past)
    ops.cache_append(vn, vc, past * hkv * d)
    attn = ops.causal_gqa(qn, kc, vc, past)
    ref = torch.empty_like(attn)
    ops.elementwise("multiply", act, attn, ref)
    kc2, vc2 = base_k.clone(), base_v.clone()
    out = ops.gated_attention(qp, kp, vn, f32(qw), f32(kw), kc2, vc2, past, rot, EPS, THETA,
                              activated=True)
    torch.cuda.synchronize()
    assert torch.equal(kc, kc2), "key cache differs"
    assert torch.equal(vc, vc2), "value cache differs"
    assert torch.equal(ref, out), "output differs from multiplyF16 after the unfused ops"
    # the plain call on the same rows applies the logistic again: different
    plain = ops.gated_attention(qp, kp, vn, f32(qw), f32(kw), base_k.clone(), base_v.clone(),
                                past, rot, EPS, THETA)
    torch.cuda.synchronize()
    assert not torch.equal(plain, out)
