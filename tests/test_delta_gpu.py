"""GPU parity of DeltaUpdate (gated delta rule) against the CPU oracle.

Bar (north star): max |out - oracle| <= 2e-3 on the fp16 outputs and
max |S - S_ref| / max |S_ref| <= 1e-3 on the fp32 state, the oracle being the
double-precision recurrence of updateDeltaColumn (Reference.metal:182-197,
oracle.delta_recurrent_f64) on identical seeded inputs built the way the
reference graph builds them (oracle.make_delta_inputs).
"""
import numpy as np
import pytest
import torch

import oracle
from llminfer_amd import _lib, ops
from tests.conftest import torch_to_u16, u16_to_torch

pytestmark = pytest.mark.gpu
OUT_TOL = 2e-3
STATE_TOL = 1e-3


def _dev(x, gpu):
    f = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    return (f(x.q), f(x.k), u16_to_torch(x.v, gpu), f(x.beta), f(x.decay), f(x.state))


def _run(x, gpu):
    q, k, v, beta, decay, state = _dev(x, gpu)
    out = ops.delta_update(q, k, v, beta, decay, state)
    torch.cuda.synchronize()
    return oracle.f16_to_f32(torch_to_u16(out)).astype(np.float64), state.cpu().numpy()


def _check(x, got_out, got_state):
    want_out, want_state = oracle.delta_recurrent_f64(x.q, x.k, x.v, x.beta, x.decay, x.state)
    assert np.all(np.isfinite(got_out)) and np.all(np.isfinite(got_state))
    oerr = np.max(np.abs(got_out - want_out))
    serr = np.max(np.abs(got_state - want_state)) / max(np.max(np.abs(want_state)), 1e-30)
    print(f"  out max-abs {oerr:.3g}  state rel {serr:.3g}", flush=True)
    assert oerr <= OUT_TOL, f"out max abs err {oerr:.3g}"
    assert serr <= STATE_TOL, f"state rel err {serr:.3g}"
    return oerr, serr


@pytest.mark.parametrize("state_std", [0.0, 0.1])
def test_decode_step_cfg5_shape(gpu, state_std):
    print(f"delta decode std={state_std}", flush=True)
    x = oracle.make_delta_inputs(5, 1, 16, 128, 32, 128, state_std)
    _check(x, *_run(x, gpu))
    names = ops.kernel_names(_lib.OP_DELTA_UPDATE, _lib.GraphDeltaParams(1, 16, 128, 32, 128))
    assert names == ["deltaRecurrent"]


@pytest.mark.parametrize("T", [2, 17, 31, 32, 64, 65, 127, 200, 1000])
def test_prefill_small(gpu, T):
    print(f"delta prefill T={T}", flush=True)
    x = oracle.make_delta_inputs(40 + T, T, 16, 128, 32, 128, 0.1)
    _check(x, *_run(x, gpu))
    names = ops.kernel_names(_lib.OP_DELTA_UPDATE, _lib.GraphDeltaParams(T, 16, 128, 32, 128))
    assert names == (["deltaChunkPrep", "deltaChunkScan"] if T >= 32 else ["deltaRecurrent"])


@pytest.mark.parametrize("T", [40, 130])
def test_chunked_zero_decay_and_beta(gpu, T):
    """Tokens whose decay is 0 (the chunk form clamps log 0) or whose beta is
    0 (pure decay), in and across chunks."""
    print(f"delta zero decay/beta T={T}", flush=True)
    x = oracle.make_delta_inputs(70 + T, T, 16, 128, 32, 128, 0.1)
    x.decay[5, :] = 0.0
    x.decay[T - 3, 3] = 0.0
    x.beta[7, :] = 0.0
    x.beta[T // 2, 1:9] = 0.0
    x.decay[T // 2 + 1, :] = 1.0
    _check(x, *_run(x, gpu))


def test_chunked_partition_invariance(gpu):
    """Chunk boundaries are an implementation detail: 300 tokens in one call,
    in calls that split chunks (100 + 200) and token by token agree."""
    print("delta chunk partition", flush=True)
    T = 300
    x = oracle.make_delta_inputs(31, T, 16, 128, 32, 128, 0.1)
    q, k, v, beta, decay, state = _dev(x, gpu)
    res = []
    for cuts in ([0, T], [0, 100, T], [0, 37, 101, 299, T]):
        st = state.clone()
        outs = [ops.delta_update(q[a:b], k[a:b], v[a:b], beta[a:b], decay[a:b], st)
                for a, b in zip(cuts, cuts[1:])]
        torch.cuda.synchronize()
        res.append((torch.cat(outs).float().cpu().numpy(), st.cpu().numpy()))
    for o, st in res:
        _check(x, o.astype(np.float64), st)
    for o, st in res[1:]:
        assert np.max(np.abs(o - res[0][0])) <= 1e-3
        assert np.max(np.abs(st - res[0][1])) / np.max(np.abs(res[0][1])) <= 1e-4


def test_prefill_cfg4(gpu):
    """BASELINE cfg4: 1024 tokens, 16x128 key heads, 32x128 value heads, S0 = 0."""
    print("delta prefill cfg4", flush=True)
    x = oracle.make_delta_inputs(4, 1024, 16, 128, 32, 128, 0.0)
    _check(x, *_run(x, gpu))


def test_prefill_long_stage_write_outs(gpu):
    """2100 tokens = 66 chunks of 32: the scan writes its staged output rows
    out after chunk 63 and again at the end (every other test ends within
    its first 64 chunks)."""
    print("delta prefill T=2100", flush=True)
    x = oracle.make_delta_inputs(21, 2100, 1, 128, 2, 32, 0.1)
    _check(x, *_run(x, gpu))


@pytest.mark.parametrize("shape", [(5, 2, 7, 4, 5), (3, 1, 4, 2, 4), (9, 2, 64, 4, 16),
                                   (33, 4, 128, 4, 32), (150, 2, 128, 8, 48),
                                   (100, 1, 128, 2, 256), (70, 2, 128, 4, 144)])
def test_other_shapes(gpu, shape):
    """Reference test-model shapes (MetalReferenceTest.py:37-40,
    ConverterTest.py:43-46) and other head splits; the last three take the
    chunk-wise kernels with 4 value heads per key head, with dv = 256 (two
    staged dv blocks) and with dv = 144 (a partial second block)."""
    T, hk, dk, hv, dv = shape
    print(f"delta shape {shape}", flush=True)
    x = oracle.make_delta_inputs(9, T, hk, dk, hv, dv, 0.2)
    _check(x, *_run(x, gpu))


def test_token_by_token_equals_one_chunk(gpu):
    """Partition invariance (MetalReferenceTest.py:289-295): one call over T
    tokens (the chunk-wise form) and T single-token calls (the recurrence)
    give the same output and state, to the split-fp16 MFMA products' error."""
    print("delta partition invariance", flush=True)
    T = 48
    x = oracle.make_delta_inputs(12, T, 16, 128, 32, 128, 0.1)
    q, k, v, beta, decay, state = _dev(x, gpu)
    whole = ops.delta_update(q, k, v, beta, decay, state.clone())
    s2 = state.clone()
    parts = [ops.delta_update(q[t:t + 1], k[t:t + 1], v[t:t + 1], beta[t:t + 1],
                              decay[t:t + 1], s2) for t in range(T)]
    s1 = state.clone()
    ops.delta_update(q, k, v, beta, decay, s1)
    torch.cuda.synchronize()
    a = whole.float().cpu().numpy()
    b = torch.cat(parts).float().cpu().numpy()
    assert np.max(np.abs(a - b)) <= 1e-3
    rel = (s1 - s2).abs().max().item() / s1.abs().max().item()
    assert rel <= 1e-4
