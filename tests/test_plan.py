"""The whole-graph plan on the CPU: lowering records and the oracle model.

* Lowering (llmi_hip_plan_lower is host-only) of the reference's tiny
  two-layer model is checked with the predicates of the reference's own
  test_graph_lowering (tests/MetalReferenceTest.py:321-377): records in op
  order, every non-view op covered by a launch or a fused epilogue, a
  copyHalfView for the interleaved query / gate halves, the epilogue
  multiset {sigmoid x2, silu, softplus_decay, swiglu x2}, no unfused
  swiGlu / deltaGates / sigmoidMul, the head on linearW8A8Gemm / Gemv by
  row count, and fewer launches without logits. Where the reference keeps
  an unfused siluF16 after the convolution, the SiLU here runs in the
  convolution's launch (causalConv with applySilu: the same bits) and is
  recorded under it. Qwen3.5-4B's one-row attention blocks lower to one
  gated-attention call each, recorded under every op of the block.
* The oracle runner (oracle/graph_runner.py) executes the same graphs op by
  op on the CPU oracle; its logits are pinned against HF transformers'
  Qwen3.5 decoder layers with the reference test's W8A8 projection
  (quantized_linear, MetalReferenceTest.py:88-100) over chunked steps that
  carry the conv, recurrent and KV states: within 2 % relative L2 and 0.1
  absolute (the reason is in the test), and partition invariant.
"""
import ctypes as C
from collections import Counter
from dataclasses import replace
from functools import partial

import numpy as np
import pytest
import torch

import oracle
from graph_runner import GraphRunner
from llminfer_amd import _lib
from llminfer_amd import graph as G
from llminfer_amd.plan import Plan, marshal

TOKENS = [3, 17, 29, 5, 11, 36, 0, 22, 9]


def _fake_table(c, w8):
    names = sorted(G.qwen35_tensors(c, w8))
    return [(0x10000 * (i + 1), 0x1000000 * (i + 1)) for i in range(len(names))], \
        {n: i for i, n in enumerate(names)}


def _lower(c, tokens, past, cap, logits, w8):
    g = G.build_qwen35(c, tokens, past, cap, logits, w8)
    table, index = _fake_table(c, w8)
    return g, Plan(g, table, index)


@pytest.mark.parametrize("w8", [True, False])
def test_lowering_matches_the_reference_predicates(w8):
    c = G.tiny_qwen35()
    n = len(TOKENS)
    chunks = [TOKENS[:2], TOKENS[2:3], TOKENS[3:]]
    past = 0
    steps = []
    for chunk in chunks:
        g, p = _lower(c, len(chunk), past, 64, "all", w8)
        steps.append((g, p))
        past += len(chunk)
    g, full = _lower(c, n, 0, 64, "all", w8)
    lowered = full.dispatches
    indices = [d["op_index"] for d in lowered]
    assert indices == sorted(indices)
    fused = {d["fused_op_index"] for d in lowered if "epilogue" in d}
    assert set(indices) | fused == {i for i, op in enumerate(g.ops)
                                    if op.kind not in (G.OpKind.RESHAPE, G.OpKind.SLICE)}
    assert any(d["kernel"] == "copyHalfView" for d in lowered)
    assert lowered[-1]["kernel"] == ("linearW8A8Gemm" if w8 else "linearF16")
    for gs, p in [(g, full), *steps]:
        ds = p.dispatches
        assert sorted(d["epilogue"] for d in ds if "epilogue" in d) == [
            "sigmoid", "sigmoid", "silu", "softplus_decay", "swiglu", "swiglu"]
        assert not {"swiGlu", "deltaGates", "sigmoidMul"} & {d["kernel"] for d in ds}
        assert "siluF16" not in {d["kernel"] for d in ds}
        conv = [i for i, op in enumerate(gs.ops) if op.kind == G.OpKind.CAUSAL_CONV1D]
        assert conv and all(gs.ops[i + 1].kind == G.OpKind.SILU for i in conv)
        by_op = {}
        for d in ds:
            by_op.setdefault(d["op_index"], []).append(d["kernel"])
        # one launch for the convolution and its SiLU; in a one-row W8A8 step
        # the launch of the norm and the projection whose row it reads
        fused = "rmsNormLinearW8A8" if w8 and gs.tokens == 1 else "causalConv"
        assert all(by_op[i] == by_op[i + 1] == [fused] for i in conv), (w8, gs.tokens)
        assert p.scratch_bytes > 0 and p.scratch_bytes % 256 == 0
    if w8:
        assert [p.dispatches[-1]["kernel"] for _, p in steps] == [
            "linearW8A8Gemm", "linearW8A8Gemv", "linearW8A8Gemm"]
    _, last = _lower(c, n, 0, 64, "last", w8)
    assert last.logit_rows == 1 and last.logit_elements == c.vocabulary
    if w8:
        assert last.dispatches[-1]["kernel"] == "linearW8A8Gemv"
    _, skipped = _lower(c, 1, n, 64, "none", w8)
    assert skipped.logit_rows == 0
    assert len(skipped.dispatches) < len(steps[-1][1].dispatches)


def test_qwen35_4b_lowers_with_the_hot_kernels():
    c = G.qwen35_4b()
    g, decode = _lower(c, 1, 4096, 8192, "last", True)
    kinds = Counter(d["kernel"] for d in decode.dispatches)
    # every hidden-width norm, its quantization and the residual Add before
    # it (all but the first layer's) in one launch, and in decode the
    # projections right after it too (DeltaNet qkv, z, a and b — a and b
    # launched at their own ops in a one-row step, recorded as fused into
    # DeltaGates —, attention q, k and v, the MLP's up and its SwiGLU gate),
    # each op recorded: the first layer's norm with its four projections
    # alone, 23 DeltaNet, 8 attention and 32 MLP norms with their Add
    # (3 + 4, 3 + 3, 3 + 2 records; DeltaNet's with the convolution and its
    # SiLU, 2 more); the final norm before the head, whose GEMV stays its
    # own launch
    assert kinds["rmsNormLinearW8A8"] == 2 + 4 + 2
    assert kinds["addRmsNormLinearW8A8"] == 23 * 9 + 8 * 6 + 32 * 5
    assert kinds["addRmsNormQuantize"] == 3 and kinds["rmsNormQuantize"] == 0
    # the rest: the DeltaNet and attention out projections, the MLP's down,
    # the head
    assert kinds["linearW8A8Gemv"] == 24 + 8 + 32 + 1
    # each DeltaNet layer's tail in one call
    # (llmi_hip_l2_norm_delta_gated_norm_activated_quantize): the q and k
    # L2Norms run inside the one-row DeltaUpdate's loads, and the gated norm
    # of its output and the quantization of the norm's rows at its end; the
    # five ops recorded under its kernel
    assert kinds["deltaRecurrentNormQuantize"] == 24 * 5
    assert kinds["gatedRmsNormQuantize"] == 0 and kinds["quantizeActivation"] == 40
    # each attention layer's block -- the q and k RMSNorms and PartialRopes,
    # KvAppend, CausalGqa and the SigmoidMul with the gate the q projection
    # activated -- in one call (llmi_hip_gated_attention_activated), its
    # seven ops recorded under its split and merge kernels
    assert kinds["gqaDecodeGated"] == kinds["gqaDecodeMergeGated"] == 8 * 7
    assert not {"gqaDecodeSplitK", "kvAppend", "normRopeTile", "partialRopeTile",
                "copyHalfView", "multiplyF16"} & set(kinds)
    assert kinds["deltaRecurrent"] == 0 and kinds["l2NormF32"] == 0
    # each DeltaNet layer's convolution with its SiLU, the epilogue of the
    # qkv projection in its norm + projections launch (its two records
    # counted above with the launch's)
    assert kinds["causalConv"] == 0 and kinds["siluF16"] == 0
    # a launch that serves several ops (the Adds, norms, quantizations,
    # projections, SiLUs and attention blocks above) has a record for each:
    # 764 records, 211 launches
    assert len(decode.dispatches) == 764 and decode.launches == 211
    assert kinds["residualAdd"] == 0
    assert "quantizeActivation" in kinds     # the others (after GQA / gated norms, SwiGLU)
    indices = [d["op_index"] for d in decode.dispatches]
    assert indices == sorted(indices)
    assert set(indices) | {d["fused_op_index"] for d in decode.dispatches if "epilogue" in d} \
        == {i for i, op in enumerate(g.ops) if op.kind not in (G.OpKind.RESHAPE, G.OpKind.SLICE)}
    _, prefill = _lower(c, 512, 0, 8192, "last", True)
    kinds = Counter(d["kernel"] for d in prefill.dispatches)
    assert kinds["gqaPrefillMfma"] == 8
    # several rows: the norms keep their quantization launch (the final
    # norm takes the last row, a view, without its Add); the head stays a GEMV
    assert kinds["rmsNormQuantize"] == 2 + 2 and kinds["addRmsNormQuantize"] == 63 * 3
    assert "addRmsNormLinearW8A8" not in kinds and kinds["linearW8A8Gemv"] == 1
    assert kinds["l2NormF32"] == 48
    # several rows: the chunked DeltaUpdate, then the gated norm with its
    # quantization
    assert kinds["gatedRmsNormQuantize"] == 24 * 2
    # the MLP down projection and the head: at most a few hundred MB of scratch
    assert prefill.scratch_bytes < 512 << 20


@pytest.mark.parametrize("past", [0, 5, 31, 32, 100, 4096])
def test_fused_decode_output_never_covers_the_new_rows(past):
    """The fused one-token KvAppend + CausalGqa launch reads the new K / V
    rows while it writes the attention output (in the same launch when there
    is one split, i.e. P + 1 <= 32). The lowering keeps the new rows live
    until the attention op, so the arena never places the output over them,
    and it fuses only when neither the output nor the workspace overlaps the
    new rows (a clash leaves KvAppend as its own launch). So a fused decode
    in every attention layer at every past, with no kvAppend launch, shows
    that no output of a fused decode covers its new rows. (Qwen3.5-4B with a
    40-wide rotation, which the whole-block call does not take, so that the
    plan uses this pair.)"""
    c = replace(G.qwen35_4b(), rotary_width=40)
    _, decode = _lower(c, 1, past, 8192, "last", True)
    kinds = Counter(d["kernel"] for d in decode.dispatches)
    assert kinds["kvAppend"] == 0
    assert kinds["gqaDecodeSplitK"] == 8 * 2
    assert kinds["gqaDecodeMerge"] == (0 if past + 1 <= 32 else 8 * 2)


@pytest.mark.parametrize("past", [0, 5, 31, 32, 100, 4096])
def test_gated_block_output_never_covers_its_rows(past):
    """The one-row attention block call reads the projected q / gate rows,
    the new key and value rows while it writes its output (in the split
    launch itself when there is one split). The lowering keeps those rows
    live until the block's SigmoidMul, where the call is made, and refuses
    to lower (an error, not a silent overlap) if the output or the workspace
    covered them; so the block in all 8 attention layers at every past shows
    that they never do."""
    c = G.qwen35_4b()
    _, decode = _lower(c, 1, past, 8192, "last", True)
    kinds = Counter(d["kernel"] for d in decode.dispatches)
    assert kinds["gqaDecodeGated"] == 8 * 7
    assert kinds["gqaDecodeMergeGated"] == (0 if past + 1 <= 32 else 8 * 7)
    assert "kvAppend" not in kinds and "gqaDecodeSplitK" not in kinds


@pytest.mark.parametrize("past", [0, 5, 31, 32, 100, 4096])
def test_delta_tail_and_conv_launches_never_cover_what_they_read(past):
    """The DeltaNet tail in one launch (llmi_hip_l2_norm_delta_gated_norm_
    activated_quantize) writes the normalised and quantized rows while other
    workgroups still read q, k, v and the gates, and the qkv projection's
    convolution epilogue writes its output while other workgroups still read
    the norm's operands. The lowering keeps those operands live until the
    last op of each merged launch and merges only when no output overlaps
    what the launch reads; so both merges in all 24 DeltaNet layers at every
    past show that no such output covers them."""
    c = G.qwen35_4b()
    _, decode = _lower(c, 1, past, 8192, "last", True)
    kinds = Counter(d["kernel"] for d in decode.dispatches)
    assert kinds["deltaRecurrentNormQuantize"] == 24 * 5
    assert kinds["causalConv"] == 0 and kinds["deltaRecurrent"] == 0
    assert kinds["rmsNormLinearW8A8"] + kinds["addRmsNormLinearW8A8"] == 8 + 415


def test_malformed_graphs_are_rejected_before_any_launch():
    c = G.tiny_qwen35()
    g = G.build_qwen35(c, 2, 0, 8, "all", True)
    table, index = _fake_table(c, True)
    desc, keep = marshal(g, index)
    lib = _lib.load()
    handle = C.c_void_p()
    values, states, ops, outputs = keep
    ops[3].inputs[0] = len(g.values) + 5                       # a missing operand
    assert lib.llmi_hip_plan_lower(C.byref(desc), None, 0, C.byref(handle)) != 0
    from llminfer_amd.plan import WeightDesc
    weights = (WeightDesc * len(table))(*[WeightDesc(d, s) for d, s in table])
    assert lib.llmi_hip_plan_lower(C.byref(desc), weights, len(table), C.byref(handle)) == \
        _lib.INVALID_ARGUMENT
    assert b"missing value" in lib.llmi_hip_last_error()
    assert not handle.value


# ----------------------------------------------------- the oracle model

def quantized_linear(input, weight):
    """tests/MetalReferenceTest.py:88-100."""
    data, weight_scales, width = weight
    rows = input.reshape(-1, width).float()
    groups = data.size(1)
    grouped = torch.nn.functional.pad(rows, (0, 32 * groups - width))
    grouped = grouped.reshape(rows.size(0), groups, 32)
    maximum = grouped.abs().amax(dim=-1)
    scales = torch.where(maximum > 0, maximum / 127, 1.0)
    quantized = torch.round(grouped / scales[..., None]).clamp(-127, 127).int()
    dots = (quantized[:, None] * data[None]).sum(dim=-1, dtype=torch.int32)
    result = (dots.float() * scales[:, None] * weight_scales[None]).sum(dim=-1)
    return result.half().reshape(*input.shape[:-1], data.size(0))


def tiny_weights(c: G.Qwen35Config, seed: int = 1597):
    """Random weights of the tiny model as numpy arrays (oracle layout):
    int8 rows padded to whole groups with fp16 scales, fp16 conv filters,
    fp32 vectors."""
    r = np.random.default_rng(seed)
    out = {}
    for tid, (element, shape) in G.qwen35_tensors(c, True).items():
        if element == G.Element.I8:
            rows, width = shape
            groups = (width + 31) // 32
            data = np.zeros((rows, groups * 32), np.int8)
            data[:, :width] = r.integers(-127, 128, (rows, width))
            scale = 0.25 / 127 if tid == G.EMBEDDING_ID else 0.12 / 127
            scales = oracle.f32_to_f16((r.random((rows, groups)) * 2 * scale + scale / 4)
                                       .astype(np.float32))
            out[tid] = (data, scales)
        elif element == G.Element.F16:
            out[tid] = (oracle.f32_to_f16((r.standard_normal(shape) * 0.12).astype(np.float32)),
                        None)
        else:
            v = (r.standard_normal(shape) * 0.1).astype(np.float32)
            if tid.endswith("linear_attn.norm.weight"):
                v = v + 1
            out[tid] = (v, None)
    return out


def oracle_states(g: G.Graph):
    return [np.zeros(s.shape, np.float32 if s.element == G.Element.F32 else np.uint16)
            for s in g.states]


def run_oracle(c, weights, chunks, logits="all", capacity=64):
    states, past, out = None, 0, []
    for chunk in chunks:
        g = G.build_qwen35(c, len(chunk), past, capacity, logits, True)
        if states is None:
            states = oracle_states(g)
        got = GraphRunner(g, weights, states, "oracle").run(np.asarray(chunk, np.uint32))
        out.append(oracle.f16_to_f32(got[0]) if got else None)
        past += len(chunk)
    return out, states


def transformers_logits(c, weights, chunks):
    """HF Qwen3.5 decoder layers with the reference test's W8A8 projection."""
    from transformers.cache_utils import DynamicCache
    from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig
    from transformers.models.qwen3_5.modeling_qwen3_5 import (Qwen3_5DecoderLayer,
                                                              Qwen3_5RMSNorm,
                                                              Qwen3_5TextRotaryEmbedding)
    text = {
        "model_type": "qwen3_5_text", "tie_word_embeddings": True, "attention_bias": False,
        "attn_output_gate": True, "attention_dropout": 0.0, "hidden_act": "silu",
        "mlp_only_layers": [], "hidden_size": c.hidden, "intermediate_size": c.intermediate,
        "vocab_size": c.vocabulary, "num_hidden_layers": len(c.layers),
        "head_dim": c.head_dim, "num_attention_heads": c.q_heads,
        "num_key_value_heads": c.kv_heads, "linear_num_key_heads": c.key_heads,
        "linear_num_value_heads": c.value_heads, "linear_key_head_dim": c.key_dim,
        "linear_value_head_dim": c.value_dim, "linear_conv_kernel_dim": c.conv_kernel,
        "max_position_embeddings": c.max_positions, "rms_norm_eps": c.epsilon,
        "rope_parameters": {"rope_type": "default", "mrope_interleaved": True,
                            "partial_rotary_factor": c.rotary_width / c.head_dim,
                            "mrope_section": [1, 1, 1], "rope_theta": c.theta},
        "layer_types": ["linear_attention" if k == "delta" else "full_attention"
                        for k in c.layers],
    }
    config = Qwen3_5TextConfig(**text)
    config._attn_implementation = "eager"

    def w8(tid):
        data, scales = weights[tid]
        rows, width = G.qwen35_tensors(c, True)[tid][1]
        groups = data.shape[1] // 32
        return (torch.from_numpy(data.astype(np.int32)).reshape(rows, groups, 32),
                torch.from_numpy(oracle.f16_to_f32(scales)), width)

    layers = []
    for index, kind in enumerate(c.layers):
        layer = Qwen3_5DecoderLayer(config, index).eval()
        state = {}
        for name, tensor in layer.state_dict().items():
            tid = f"layers.{index}.{name}"
            data, _ = weights[tid]
            if data.dtype == np.int8:
                continue
            if data.dtype == np.uint16:
                state[name] = torch.from_numpy(oracle.f16_to_f32(data)).half().reshape(tensor.shape)
            else:
                state[name] = torch.from_numpy(data).reshape(tensor.shape)
        layer.load_state_dict(state, strict=False)
        for name, module in layer.named_modules():
            if isinstance(module, torch.nn.Linear):
                module.forward = partial(quantized_linear, weight=w8(f"layers.{index}.{name}.weight"))
        layers.append(layer)
    emb = w8(G.EMBEDDING_ID)
    table = (emb[0].float() * emb[1][..., None]).reshape(emb[0].size(0), -1)[:, :c.hidden].half()
    norm = Qwen3_5RMSNorm(c.hidden, c.epsilon)
    norm.load_state_dict({"weight": torch.from_numpy(weights["norm.weight"][0])})
    rope = Qwen3_5TextRotaryEmbedding(config)
    cache = DynamicCache(config=config)
    past, out = 0, []
    with torch.inference_mode():
        for chunk in chunks:
            end = past + len(chunk)
            positions = torch.arange(past, end)
            hidden = table[torch.tensor(chunk)][None]
            visible = torch.arange(end)[None, :] <= positions[:, None]
            mask = torch.zeros(visible.shape, dtype=torch.float16)
            mask.masked_fill_(~visible, float("-inf"))
            for layer, kind in zip(layers, c.layers):
                if kind == "delta":
                    hidden = layer(hidden, position_embeddings=None, past_key_values=cache)
                else:
                    hidden = layer(hidden, position_embeddings=rope(hidden, positions[None, None]),
                                   position_ids=positions[None], attention_mask=mask[None, None],
                                   past_key_values=cache)
            out.append(quantized_linear(norm(hidden), emb).float().reshape(len(chunk), -1).numpy())
            past = end
    return out


@pytest.mark.parametrize("seed", [1597, 7, 11])
def test_oracle_model_matches_transformers(seed):
    """Logits within 2 % relative L2 and 0.1 absolute of HF's. The oracle
    keeps attention and the delta rule in float64, HF in fp16 (eager
    attention) and fp32 (its chunked delta rule); an fp16 rounding flip
    ahead of a W8A8 projection moves its int8 activation by one step, which
    the later layers amplify, so the elementwise bound of the reference test
    (atol 0.003, rtol 0.008) holds for some weights and not others (measured
    over five seeds: relative L2 0 - 1.3 %, max |diff| <= 0.056; many steps
    are bit-identical). A wrong term, sign, head order or position puts the
    logits O(1) apart."""
    pytest.importorskip("transformers.models.qwen3_5")
    c = G.tiny_qwen35()
    weights = tiny_weights(c, seed)
    chunks = [TOKENS[:2], TOKENS[2:3], TOKENS[3:]]
    got, _ = run_oracle(c, weights, chunks)
    want = transformers_logits(c, weights, chunks)
    for g_, w_ in zip(got, want):
        assert g_.shape == w_.shape
        assert np.linalg.norm(g_ - w_) <= 0.02 * np.linalg.norm(w_)
        assert np.abs(g_ - w_).max() < 0.1
    # one chunk against three: the oracle is partition invariant bit for bit
    full, _ = run_oracle(c, weights, [TOKENS])
    assert np.array_equal(full[0], np.concatenate(got))
