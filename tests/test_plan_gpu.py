"""The whole-graph plan on the GPU.

* Bit for bit against the same graph run op by op through the per-op entry
  points (tests/graph_runner.py, backend "gpu": every projection unfused,
  every view copied): the fused epilogues, the arena's reuse, the in-place
  views and the launch order change nothing. Logits of every step and the
  conv, recurrent and KV states after the last step are compared.
* Against the CPU oracle runner (pinned to HF transformers in test_plan.py)
  at that test's bound, over chunked steps.
* The reference's tiny model (generic attention and DeltaNet kernels), a
  small model at the real head widths (MFMA GQA prefill, split-K decode,
  chunked and recurrent DeltaNet, the MFMA W8A8 GEMM), both precisions,
  and one Qwen3.5-4B decode step.
"""
import numpy as np
import pytest
import torch

import oracle
from graph_runner import GraphRunner
from llminfer_amd import graph as G
from llminfer_amd.plan import ModelSession, random_weights
from test_plan import TOKENS, oracle_states, run_oracle, tiny_weights

pytestmark = pytest.mark.gpu


def small_qwen35() -> G.Qwen35Config:
    """Two layers at Qwen3.5's head widths: GQA d 256 (4 query / 2 KV heads,
    64-wide RoPE), DeltaNet dk = dv = 128 (2 key / 4 value heads)."""
    return G.Qwen35Config(hidden=512, intermediate=1024, vocabulary=1000, head_dim=256,
                          q_heads=4, kv_heads=2, rotary_width=64, key_heads=2, value_heads=4,
                          key_dim=128, value_dim=128, conv_kernel=4, layers=("delta", "gqa"),
                          max_positions=4096)


def device_weights(weights, gpu):
    out = {}
    for tid, (data, scales) in weights.items():
        if data.dtype == np.uint16:
            d = torch.from_numpy(data.view(np.int16)).to(gpu).view(torch.float16)
        else:
            d = torch.from_numpy(np.ascontiguousarray(data)).to(gpu)
        s = None if scales is None else \
            torch.from_numpy(scales.view(np.int16)).to(gpu).view(torch.float16)
        out[tid] = (d, s)
    return out


def _u16(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _f16_logits(x):
    return oracle.f16_to_f32(x) if x.dtype == np.uint16 else x


def run_plan_and_ops(c, weights, chunks, w8, gpu, capacity=64):
    """Per step: the plan's logits and the op-by-op GPU run's (fp16 bits),
    then both sides' states."""
    dw = device_weights(weights, gpu)
    session = ModelSession(c, dw, capacity, w8, gpu)
    states = None
    plan_logits, op_logits = [], []
    past = 0
    for chunk in chunks:
        print(f"plan step tokens={len(chunk)} past={past} w8={w8}", flush=True)
        r = session.step(chunk, "all", trace=True)
        plan_logits.append(r.logits)
        g = G.build_qwen35(c, len(chunk), past, capacity, "all", w8)
        if states is None:
            states = [torch.zeros(s.shape, dtype=torch.float32 if s.element == G.Element.F32
                                  else torch.float16, device=gpu) for s in g.states]
        ids = torch.from_numpy(np.asarray(chunk, np.uint32).view(np.int32)).to(gpu)
        got = GraphRunner(g, dw, states, "gpu").run(ids)
        torch.cuda.synchronize()
        op_logits.append(got[0].float().cpu().numpy())
        past += len(chunk)
    return session, plan_logits, op_logits, states


def _same_state(a: torch.Tensor, b: torch.Tensor) -> bool:
    return torch.equal(a.view(torch.int16) if a.dtype == torch.float16 else a.view(torch.int32),
                       b.view(torch.int16) if b.dtype == torch.float16 else b.view(torch.int32))


def _f16_weights(c, seed):
    """fp16 weights for the LinearF16 path: the int8 rows dequantized."""
    w8 = tiny_weights(c, seed) if c is not None else None
    out = {}
    for tid, (element, shape) in G.qwen35_tensors(c, False).items():
        data, scales = w8[tid]
        if element == G.Element.F16 and data.dtype == np.int8:
            rows, width = shape
            groups = data.shape[1] // 32
            deq = data.astype(np.float32).reshape(rows, groups, 32) * \
                oracle.f16_to_f32(scales)[..., None]
            out[tid] = (oracle.f32_to_f16(deq.reshape(rows, -1)[:, :width]), None)
        else:
            out[tid] = (data, scales)
    return out


@pytest.mark.parametrize("w8", [True, False])
def test_tiny_plan_is_the_op_by_op_graph(gpu, w8):
    c = G.tiny_qwen35()
    weights = tiny_weights(c, 1597) if w8 else _f16_weights(c, 1597)
    chunks = [TOKENS[:2], TOKENS[2:3], TOKENS[3:]]
    session, plan_logits, op_logits, states = run_plan_and_ops(c, weights, chunks, w8, gpu)
    for p, o in zip(plan_logits, op_logits):
        assert np.array_equal(p.view(np.uint32), o.view(np.uint32))
    for a, b in zip(session.states, states):
        assert _same_state(a, b)


def test_tiny_plan_matches_the_oracle(gpu):
    """The reference's tiny model through the plan against the oracle model
    (itself pinned to HF transformers in test_plan.py), over chunked steps."""
    c = G.tiny_qwen35()
    weights = tiny_weights(c, 7)
    chunks = [TOKENS[:2], TOKENS[2:3], TOKENS[3:]]
    session = ModelSession(c, device_weights(weights, gpu), 64, True, gpu)
    want, _ = run_oracle(c, weights, chunks)
    for chunk, w_ in zip(chunks, want):
        got = session.step(chunk, "all").logits
        rel = np.linalg.norm(got - w_) / np.linalg.norm(w_)
        print(f"  tiny plan vs oracle: rel L2 {rel:.3g}, max {np.abs(got - w_).max():.3g}, "
              f"identical {np.mean(got == w_):.3f}", flush=True)
        # measured: bit-identical (the tiny model's generic attention and
        # DeltaNet kernels round like the float64 oracle here); the bound
        # leaves room for a single int8 rounding flip
        assert rel <= 2e-3
        assert np.abs(got - w_).max() < 0.02


def _small_weights(c, seed):
    r = np.random.default_rng(seed)
    out = {}
    for tid, (element, shape) in G.qwen35_tensors(c, True).items():
        if element == G.Element.I8:
            rows, width = shape
            groups = (width + 31) // 32
            data = np.zeros((rows, groups * 32), np.int8)
            data[:, :width] = r.integers(-127, 128, (rows, width))
            scale = 0.6 / 127 / np.sqrt(width)
            out[tid] = (data, oracle.f32_to_f16((r.random((rows, groups)) * 2 * scale)
                                                .astype(np.float32)))
        elif element == G.Element.F16:
            out[tid] = (oracle.f32_to_f16((r.standard_normal(shape) * 0.3).astype(np.float32)),
                        None)
        else:
            v = (r.standard_normal(shape) * 0.1).astype(np.float32)
            if tid.endswith("linear_attn.norm.weight"):
                v = v + 1
            out[tid] = (v, None)
    return out


def test_small_plan_on_the_hot_kernels(gpu):
    c = small_qwen35()
    weights = _small_weights(c, 3)
    rng = np.random.default_rng(4)
    chunks = [list(rng.integers(0, c.vocabulary, 40)), [5], [999], list(rng.integers(0, 1000, 33))]
    session, plan_logits, op_logits, states = run_plan_and_ops(c, weights, chunks, True, gpu,
                                                               capacity=256)
    for p, o in zip(plan_logits, op_logits):
        assert np.array_equal(p.view(np.uint32), o.view(np.uint32))
    for a, b in zip(session.states, states):
        assert _same_state(a, b)
    kernels = {d["kernel"] for d in session.plan(1, "last").dispatches}
    # the one-row attention block in one call (llmi_hip_gated_attention_activated),
    # and the DeltaNet tail (llmi_hip_l2_norm_delta_gated_norm_activated_quantize)
    assert {"gqaDecodeGated", "deltaRecurrentNormQuantize", "linearW8A8Gemv"} <= kernels
    assert "gqaDecodeSplitK" not in kernels
    want, _ = run_oracle(c, weights, chunks, capacity=256)
    for p, w_ in zip(plan_logits, want):
        # measured 0.8-1.0 % (max 0.022): the MFMA attention and chunked
        # delta rule sum in fp32 where the oracle sums in float64, and a
        # rounding flip ahead of an int8 quantization moves the activation by
        # a whole step, which the later layers carry; a wrong term, sign or
        # head order is O(1)
        rel = np.linalg.norm(p - w_) / np.linalg.norm(w_)
        print(f"  small plan vs oracle: rel L2 {rel:.3g}, max {np.abs(p - w_).max():.3g}",
              flush=True)
        assert rel <= 0.02 and np.abs(p - w_).max() < 0.05


def test_session_rejects_bad_steps_and_resets(gpu):
    c = G.tiny_qwen35()
    session = ModelSession(c, device_weights(tiny_weights(c), gpu), 8, True, gpu)
    with pytest.raises(ValueError):
        session.step([c.vocabulary])
    with pytest.raises(ValueError):
        session.step(list(range(9)))
    a = session.step(TOKENS[:4]).logits
    session.step(TOKENS[4:6])
    session.reset()
    assert session.past == 0
    assert np.array_equal(session.step(TOKENS[:4]).logits, a)


def test_qwen35_4b_decode_step(gpu):
    """Qwen3.5-4B (32 layers, random W8A8 weights of its shapes): a 64-token
    prefill and a decode step through the session equal, bit for bit, the
    same two graphs run op by op through the per-op entry points (logits and
    every state), and the decode step's records name the fused kernels."""
    c = G.qwen35_4b()
    print("qwen3.5-4b random weights", flush=True)
    weights = random_weights(c, True, gpu, seed=1)
    session = ModelSession(c, weights, 1024, True, gpu)
    prompt = list(range(100, 164))
    r = session.step(prompt, "last")
    assert r.logits.shape == (1, c.vocabulary) and np.isfinite(r.logits).all()
    first = r.logits
    r = session.step([7], "last", trace=True)
    assert r.past == 65 and np.isfinite(r.logits).all()
    print("qwen3.5-4b op by op", flush=True)
    states = None
    want = []
    for past, chunk in ((0, prompt), (64, [7])):
        g = G.build_qwen35(c, len(chunk), past, 1024, "last", True)
        if states is None:
            states = [torch.zeros(s.shape, dtype=torch.float32 if s.element == G.Element.F32
                                  else torch.float16, device=gpu) for s in g.states]
        ids = torch.tensor(chunk, dtype=torch.int32, device=gpu)
        want.append(GraphRunner(g, weights, states, "gpu").run(ids)[0].float().cpu().numpy())
    torch.cuda.synchronize()
    assert np.array_equal(first.view(np.uint32), want[0].view(np.uint32))
    assert np.array_equal(r.logits.view(np.uint32), want[1].view(np.uint32))
    for a, b in zip(session.states, states):
        assert _same_state(a, b)
    kinds = [d["kernel"] for d in r.dispatches]
    # deltaRecurrentNormQuantize: the update, its fused q / k L2Norms, the
    # gated norm of its output and the quantization of the norm's rows, a
    # record each
    # gqaDecodeGated: the attention block's seven ops (q / k RMSNorm and
    # PartialRope, KvAppend, CausalGqa, SigmoidMul) in one call, a record each
    assert kinds.count("gqaDecodeGated") == 8 * 7
    assert kinds.count("deltaRecurrentNormQuantize") == 24 * 5


def test_nonfinite_activation_invalidates_until_reset(gpu):
    """A non-finite activation found by a quantization fails the step after
    its launches and leaves the session invalid until reset
    (MetalExecutor.mm:180-187, 283-298); past does not advance, and the
    session is clean again after reset."""
    c = G.tiny_qwen35()
    weights = tiny_weights(c, 11)
    dw = device_weights(weights, gpu)
    session = ModelSession(c, dw, 8, True, gpu)
    good = session.step(TOKENS[:2], "all").logits
    # an infinite embedding row: its token's hidden row is non-finite
    table, scales = dw[G.EMBEDDING_ID]
    saved = scales[TOKENS[2]].clone()
    scales[TOKENS[2]] = float("inf")
    print("nonfinite activation step", flush=True)
    with pytest.raises(RuntimeError):
        session.step(TOKENS[2:3])
    assert session.invalid and session.past == 2
    with pytest.raises(RuntimeError):
        session.step(TOKENS[3:4])        # refused before any launch
    scales[TOKENS[2]] = saved
    session.reset()
    assert not session.invalid and session.past == 0
    again = session.step(TOKENS[:2], "all").logits
    assert np.array_equal(good.view(np.uint32), again.view(np.uint32))


def test_session_states_read_back(gpu):
    """The state copies the session hands out are its buffers after the
    step: the KV cache rows of the step are written, rows past it zero."""
    c = G.tiny_qwen35()
    session = ModelSession(c, device_weights(tiny_weights(c, 5), gpu), 8, True, gpu)
    session.step(TOKENS[:3], "none")
    states = session.states
    kinds = [s.kind for s in G.build_qwen35(c, 1, 0, 8, "none", True).states]
    assert len(states) == len(kinds)
    for st, kind in zip(states, kinds):
        if kind in (G.StateKind.KEY_CACHE, G.StateKind.VALUE_CACHE):
            assert torch.count_nonzero(st[:3]) > 0 and torch.count_nonzero(st[3:]) == 0
