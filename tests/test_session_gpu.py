"""GPU tests of the session contract (HipSession over llmi_hip_session_*).

Mirrors the reference's session behaviour (MetalExecutor.mm:255-298) and its
parity harness: chunked steps [17, 114, 1, 1] like test_long_attention
(tests/MetalReferenceTest.py:458-472), partition invariance (whole vs chunks,
:289-295), plan-record invariants (op indices sorted, every op covered,
:346-351), and the flash kernel for T > 1 / split-K decode for T == 1
(:465-469). Numerics: outputs within 2e-3 of the double-precision oracle,
the fp32 state within 1e-3 relative.
"""
import numpy as np
import pytest
import torch

import oracle
from llminfer_amd.session import HipSession
from tests.conftest import p_rounding_bound, torch_to_u16, u16_to_torch

pytestmark = pytest.mark.gpu

# A small hybrid layer pair with the north-star head shapes.
HQ, HKV, D = 16, 4, 256
HK, DK, HV, DV = 16, 128, 32, 128


def make_steps(seed, chunks):
    T = sum(chunks)
    dl = oracle.make_delta_inputs(seed, T, HK, DK, HV, DV)
    g = oracle.make_gqa_inputs(seed, T, HQ, HKV, D, 0)
    return dl, g


def run_session(gpu, s, dl, g, chunks, past0=0):
    outs_d, outs_g, plans = [], [], []
    t0 = 0
    f = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    for n in chunks:
        sl = slice(t0, t0 + n)
        r = s.step(f(dl.q[sl]), f(dl.k[sl]), u16_to_torch(dl.v[sl], gpu), f(dl.beta[sl]),
                   f(dl.decay[sl]), u16_to_torch(g.q[sl], gpu), u16_to_torch(g.k_new[sl], gpu),
                   u16_to_torch(g.v_new[sl], gpu))
        assert r.past == past0 + t0 + n
        outs_d.append(oracle.f16_to_f32(torch_to_u16(r.delta_out)))
        outs_g.append(oracle.f16_to_f32(torch_to_u16(r.gqa_out)))
        plans.append(r.dispatches)
        t0 += n
    return np.concatenate(outs_d), np.concatenate(outs_g), plans


def test_chunked_session_matches_oracle(gpu):
    chunks = [17, 114, 1, 1]
    print(f"session chunks {chunks}", flush=True)
    T = sum(chunks)
    dl, g = make_steps(31, chunks)
    s = HipSession.open(capacity=160)
    d_out, g_out, plans = run_session(gpu, s, dl, g, chunks)
    want_d, want_state = oracle.delta_recurrent_f64(dl.q, dl.k, dl.v, dl.beta, dl.decay,
                                                    dl.state)
    want_g = oracle.gqa_dense_f64(g.q, g.k_cache, g.v_cache, 0)
    assert np.max(np.abs(d_out - want_d)) <= 2e-3
    assert np.max(np.abs(g_out.reshape(T, HQ, D) - want_g)) <= 2e-3
    st = s.recurrent_state().cpu().numpy()
    assert np.max(np.abs(st - want_state)) / np.max(np.abs(want_state)) <= 1e-3
    kc = torch_to_u16(s.key_cache())
    assert np.array_equal(kc[:T], g.k_cache[:T]) and not kc[T:].any()
    assert np.array_equal(torch_to_u16(s.value_cache())[:T], g.v_cache[:T])
    # Plan records: the reference's own invariant, written as
    # MetalReferenceTest.py:346-351 writes it -- op indices sorted and, with
    # the fused indices of records that carry an epilogue, covering every
    # op. The split-K decode appends inside its own launch for short chunks
    # (recorded under op 1 and op 2), the flash path follows an append.
    for n, plan in zip(chunks, plans):
        check_plan(plan, n)
    s.close()


def check_plan(lowered, n):
    indices = [dispatch["op_index"] for dispatch in lowered]
    assert indices == sorted(indices)
    fused_indices = {d["fused_op_index"] for d in lowered if "epilogue" in d}
    assert set(indices) | fused_indices == {0, 1, 2}
    assert not [d for d in lowered if "epilogue" in d]  # no projection epilogues here
    by_op = {i: [d["kernel"] for d in lowered if d["op_index"] == i] for i in (0, 1, 2)}
    if n > 1:
        assert by_op[1] == ["kvAppend"] and by_op[2] == ["gqaPrefillMfma"]
    else:
        assert by_op[0] == ["deltaRecurrent"]
        assert by_op[1] == ["gqaDecodeSplitK"]
        assert by_op[2] in (["gqaDecodeSplitK"], ["gqaDecodeSplitK", "gqaDecodeMerge"])


def test_hybrid_decode_cfg5_session(gpu):
    """BASELINE cfg5 as a session workload: a DeltaNet state seeded N(0, 0.1)
    and a 32,768-row N(0,1) KV cache, then 32 steps of one DeltaNet decode
    update + KvAppend + GQA decode, each step appending its own K/V row
    (P = 32768 .. 32799). Every step's outputs within 2e-3 of the oracle,
    the final state within 1e-3 relative, the appended rows bit-exact --
    the reference's chunked-steps check (MetalReferenceTest.py:458-472) at
    the north-star context length."""
    P0, steps = 32768, 32
    print(f"session cfg5: {steps} decode steps from P={P0}", flush=True)
    dl = oracle.make_delta_inputs(41, steps, HK, DK, HV, DV, 0.1)
    g = oracle.make_gqa_inputs(42, steps, HQ, HKV, D, P0)
    s = HipSession.open(capacity=P0 + steps)
    kc, vc, st = s.writable_views()
    kc[:P0].copy_(u16_to_torch(g.k_cache[:P0], gpu))
    vc[:P0].copy_(u16_to_torch(g.v_cache[:P0], gpu))
    st.copy_(torch.from_numpy(dl.state))
    torch.cuda.synchronize()
    s.restore(P0)
    d_out, g_out, plans = run_session(gpu, s, dl, g, [1] * steps, past0=P0)
    want_d, want_state = oracle.delta_recurrent_f64(dl.q, dl.k, dl.v, dl.beta, dl.decay,
                                                    dl.state)
    # The 32 decode queries see keys [0, P0 + j], which is a causal chunk of
    # 32 tokens after P0 past rows.
    want_g = oracle.gqa_dense_f64(g.q, g.k_cache, g.v_cache, P0)
    e_d = np.max(np.abs(d_out - want_d), axis=1)
    e_g = np.max(np.abs(g_out.reshape(steps, HQ * D) - want_g.reshape(steps, HQ * D)), axis=1)
    print(f"  per-step max err: delta {e_d.max():.3g}, gqa {e_g.max():.3g}")
    assert np.all(e_d <= 2e-3) and np.all(e_g <= 2e-3)
    stf = s.recurrent_state().cpu().numpy()
    rel = np.max(np.abs(stf - want_state)) / np.max(np.abs(want_state))
    print(f"  final state rel err {rel:.3g}")
    assert rel <= 1e-3
    assert np.array_equal(torch_to_u16(s.key_cache())[P0:], g.k_new)
    assert np.array_equal(torch_to_u16(s.value_cache())[P0:], g.v_new)
    assert np.array_equal(torch_to_u16(s.key_cache()[:P0]), g.k_cache[:P0])
    for plan in plans:
        check_plan(plan, 1)
    s.close()


def test_partition_invariance(gpu):
    """Whole prompt in one step vs chunks vs token by token (the reference
    checks whole vs [2,1,5,11] at 1e-5 for same-precision paths). The
    DeltaNet path keeps the state in fp32 between steps, so it must agree
    exactly; attention switches between the MFMA prefill and the split-K
    decode kernels, so it agrees to fp16 output rounding."""
    print("session partition invariance", flush=True)
    parts = [[19], [2, 1, 5, 11], [1] * 19]
    dl, g = make_steps(77, [19])
    res = []
    for chunks in parts:
        s = HipSession.open(capacity=32)
        res.append(run_session(gpu, s, dl, g, chunks)[:2] + (s.recurrent_state().cpu(),))
        s.close()
    # Attention: every partition within the north-star 2e-3 of the dense
    # oracle, and within two fp16 output ulps plus the fp16-P rounding bound
    # of each other.
    want = oracle.gqa_dense_f64(g.q, g.k_cache, g.v_cache, 0).reshape(19, HQ * D)
    a = res[0][1].reshape(19, HQ * D)
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(a), 2.0 ** -14))) - 10)
    pb = p_rounding_bound(g.q, g.k_cache, g.v_cache, 0).reshape(19, HQ * D)
    for d_out, g_out, st in res[1:]:
        assert np.array_equal(d_out, res[0][0])
        assert torch.equal(st, res[0][2])
        b = g_out.reshape(19, HQ * D)
        assert np.max(np.abs(b - want)) <= 2e-3
        assert np.all(np.abs(b - a) <= 2 * ulp + pb)


def test_validation_leaves_session_unchanged(gpu):
    print("session validation", flush=True)
    dl, g = make_steps(5, [8])
    s = HipSession.open(capacity=10)
    run_session(gpu, s, dl, g, [8])
    before = s.recurrent_state()
    with pytest.raises(Exception, match="exceeds session capacity"):
        run_session(gpu, s, dl, g, [3])  # 8 + 3 > 10
    assert s.past == 8 and not s.invalid
    assert torch.equal(s.recurrent_state(), before)
    with pytest.raises(ValueError):
        s.step(*(torch.zeros(1, device=gpu),) * 8)
    s.reset()
    assert s.past == 0 and not s.invalid
    assert not s.recurrent_state().any() and not s.key_cache().any()
    # After reset the session replays identically.
    d1, g1, _ = run_session(gpu, s, dl, g, [8])
    s.close()
    s2 = HipSession.open(capacity=10)
    d2, g2, _ = run_session(gpu, s2, dl, g, [8])
    assert np.array_equal(d1, d2) and np.array_equal(g1, g2)
    s2.close()
