"""GPU parity of the fused L2Norm -> DeltaUpdate -> GatedRmsNorm chain
(llmi_hip_l2_norm_delta_gated_norm; Qwen35ModelBuilder.cpp:155-166).

The chain as the reference graph emits it, run as separate launches --
llmi_hip_l2_norm_delta_update (itself bit-identical to the L2Norm ->
DeltaUpdate pair, test_delta_fused_gpu.py) and then llmi_hip_gated_rms_norm
(bit-exact with the oracle's orc_gated_rms_norm, test_delta_front_gpu.py)
-- must leave exactly the same output and state bits as the fused call, on
the chunked form (dk 128, T >= 32: the scan normalises the rows at its end)
and the recurrent form (T <= 32: one workgroup per value head). The fused
output is also compared with the oracle's gatedRmsNorm applied to the
unfused DeltaUpdate output.
"""
import numpy as np
import pytest
import torch

import oracle
from llminfer_amd import ops
from tests.conftest import torch_to_u16, u16_to_torch

pytestmark = pytest.mark.gpu


SHAPES = [
    # chunked (T >= 32, dk 128)
    (1024, 16, 128, 32, 128), (100, 16, 128, 32, 128), (64, 2, 128, 4, 64),
    (33, 2, 128, 4, 128), (150, 2, 128, 8, 48), (300, 1, 128, 2, 32),
    # recurrent, one workgroup per value head (T <= 32)
    (1, 16, 128, 32, 128), (5, 16, 128, 32, 128), (31, 2, 128, 4, 128),
    (1, 4, 64, 8, 64), (17, 2, 64, 4, 128), (32, 2, 64, 2, 64),
]


@pytest.mark.parametrize("shape", SHAPES)
def test_fused_equals_chain(gpu, shape):
    T, hk, dk, hv, dv = shape
    print(f"l2norm+delta+gatednorm shape {shape}", flush=True)
    seed = 90 + T + dv
    d = oracle.make_delta_inputs(seed, T, hk, dk, hv, dv, 0.1)
    q16 = oracle.normal_f16(seed, 21, (T, hk * dk))
    k16 = oracle.normal_f16(seed, 22, (T, hk * dk))
    z16 = oracle.normal_f16(seed, 23, (T, hv * dv))
    w = oracle.normal_f32(seed, 24, (dv,), 1.0, 0.2)
    f = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    q, k, v, z = (u16_to_torch(a, gpu) for a in (q16, k16, d.v, z16))
    beta, decay, wt = f(d.beta), f(d.decay), f(w)
    # Unfused: L2Norm+DeltaUpdate, then gatedRmsNorm over rows of dv.
    s_ref = f(d.state)
    x = ops.l2_norm_delta_update(q, k, v, beta, decay, s_ref)
    ref = torch.empty_like(x)
    ops.gated_rms_norm(x.view(T * hv, dv), z.view(T * hv, dv), wt, ref.view(T * hv, dv), 1e-6)
    # Fused.
    s_fused = f(d.state)
    out = ops.l2_norm_delta_gated_norm(q, k, v, beta, decay, s_fused, z, wt)
    torch.cuda.synchronize()
    assert torch.equal(s_ref, s_fused), "states differ from the unfused chain"
    got, want = torch_to_u16(out), torch_to_u16(ref)
    bad = np.flatnonzero(got.reshape(-1) != want.reshape(-1))
    assert bad.size == 0, f"{bad.size} outputs differ from the unfused chain, first at {bad[:4]}"
    if T in (1, 100, 33):
        xo = torch_to_u16(x).reshape(T * hv, dv)
        assert np.array_equal(got.reshape(T * hv, dv),
                              oracle.gated_rms_norm(xo, z16.reshape(T * hv, dv), w))


def test_fused_repeats_and_reuses_counters(gpu):
    """Back-to-back chunked calls on one workspace: the per-head arrival
    counters are re-zeroed by each call's prep."""
    T, hk, dk, hv, dv = 96, 2, 128, 4, 128
    d = oracle.make_delta_inputs(5, T, hk, dk, hv, dv, 0.1)
    q16 = oracle.normal_f16(5, 21, (T, hk * dk))
    k16 = oracle.normal_f16(5, 22, (T, hk * dk))
    z16 = oracle.normal_f16(5, 23, (T, hv * dv))
    f = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    q, k, v, z = (u16_to_torch(a, gpu) for a in (q16, k16, d.v, z16))
    wt = f(np.ones(dv, np.float32))
    outs = []
    for _ in range(3):
        st = f(d.state)
        outs.append(ops.l2_norm_delta_gated_norm(q, k, v, f(d.beta), f(d.decay), st, z, wt))
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[1], outs[2])
