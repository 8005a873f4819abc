"""GPU parity of the fused L2Norm -> DeltaUpdate pair (llmi_hip_l2_norm_delta_update).

The pair as the reference graph emits it (Qwen35ModelBuilder.cpp:155-156:
L2Norm(q, 1e-6, 1/sqrt(dk)), L2Norm(k, 1e-6, 1), then DeltaUpdate) run as
separate launches -- llmi_hip_l2_norm, itself bit-exact with the oracle's
orc_l2norm_f32, then llmi_hip_delta_update -- must give exactly the same
output and state bits as the fused call, which normalises the fp16 q/k rows
inside the update kernels. The fused result is also checked against the
double-precision recurrence on the oracle-normalised operands at the
north-star bar (max-abs 2e-3 on the output, 1e-3 relative on the state).
"""
import numpy as np
import pytest
import torch

import oracle
from llminfer_amd import ops
from tests.conftest import torch_to_u16, u16_to_torch

pytestmark = pytest.mark.gpu


def _inputs(seed, T, hk, dk, hv, dv):
    d = oracle.make_delta_inputs(seed, T, hk, dk, hv, dv, 0.1)
    q16 = oracle.normal_f16(seed, 21, (T, hk * dk))
    k16 = oracle.normal_f16(seed, 22, (T, hk * dk))
    return d, q16, k16


@pytest.mark.parametrize("shape", [(1, 16, 128, 32, 128), (17, 16, 128, 32, 128),
                                   (100, 16, 128, 32, 128), (1024, 16, 128, 32, 128),
                                   (9, 2, 64, 4, 16), (150, 2, 128, 8, 48),
                                   (300, 1, 64, 2, 32)])
def test_fused_equals_l2_norm_then_update(gpu, shape):
    T, hk, dk, hv, dv = shape
    print(f"l2norm+delta shape {shape}", flush=True)
    d, q16, k16 = _inputs(60 + T, T, hk, dk, hv, dv)
    qs = float(np.float32(1.0) / np.sqrt(np.float32(dk)))
    f = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    q, k, v = u16_to_torch(q16, gpu), u16_to_torch(k16, gpu), u16_to_torch(d.v, gpu)
    beta, decay = f(d.beta), f(d.decay)
    # Unfused: the two l2NormF32 launches, then DeltaUpdate on fp32 q/k.
    qf = torch.empty((T, hk * dk), dtype=torch.float32, device=gpu)
    kf = torch.empty_like(qf)
    ops.l2_norm(q, qf, dk, 1e-6, qs)
    ops.l2_norm(k, kf, dk, 1e-6, 1.0)
    s_ref = f(d.state)
    out_ref = ops.delta_update(qf, kf, v, beta, decay, s_ref)
    # Fused.
    s_fused = f(d.state)
    out_fused = ops.l2_norm_delta_update(q, k, v, beta, decay, s_fused)
    torch.cuda.synchronize()
    assert torch.equal(out_ref, out_fused), "outputs differ from the unfused pair"
    assert torch.equal(s_ref, s_fused), "states differ from the unfused pair"
    # The normalised operands are the oracle's, bit for bit.
    assert np.array_equal(qf.cpu().numpy(), oracle.l2norm_f32(q16, dk, 1e-6, qs))
    if T in (1, 100):
        qo = oracle.l2norm_f32(q16, dk, 1e-6, qs)
        ko = oracle.l2norm_f32(k16, dk, 1e-6, 1.0)
        want, want_state = oracle.delta_recurrent_f64(qo, ko, d.v, d.beta, d.decay, d.state)
        got = oracle.f16_to_f32(torch_to_u16(out_fused)).astype(np.float64)
        assert np.max(np.abs(got - want)) <= 2e-3
        st = s_fused.cpu().numpy()
        assert np.max(np.abs(st - want_state)) / np.max(np.abs(want_state)) <= 1e-3

