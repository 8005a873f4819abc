"""The C++ Qwen3.5 graph builder behind the model session (csrc/model.cpp).

Its graphs are compared field by field with the Python builder's
(llminfer_amd/graph.py), whose graphs test_graph_builder.py replays through
the reference's own Graph.cpp: every value (element, kind, shape, strides,
view base and offset, defining op, tensor), state and op attribute, and the
outputs, for the reference's tiny model, the real head widths and
Qwen3.5-4B, prefill and decode shapes, every logits mode, W8A8 and fp16.
Host only: nothing runs on a device.
"""
import ctypes as C

import pytest

from llminfer_amd import _lib
from llminfer_amd import graph as G
from llminfer_amd.plan import LOGITS, GraphDesc, GraphOp, GraphState, GraphValue, c_config, \
    marshal


def small_qwen35() -> G.Qwen35Config:
    return G.Qwen35Config(hidden=512, intermediate=1024, vocabulary=1000, head_dim=256,
                          q_heads=4, kv_heads=2, rotary_width=64, key_heads=2, value_heads=4,
                          key_dim=128, value_dim=128, conv_kernel=4, layers=("delta", "gqa"),
                          max_positions=4096)


def cpp_graph(c, tokens, past, capacity, logits, w8):
    lib = _lib.load()
    cfg, kinds = c_config(c, w8)
    h = C.c_void_p()
    rc = lib.llmi_qwen35_build(C.byref(cfg), tokens, past, capacity, LOGITS[logits],
                               C.byref(h))
    if rc != _lib.OK:
        raise _lib.HipError(rc, lib.llmi_hip_last_error().decode())
    try:
        d = C.cast(lib.llmi_qwen35_graph_view(h), C.POINTER(GraphDesc)).contents
        tensors = [lib.llmi_qwen35_graph_tensor(h, i).decode()
                   for i in range(lib.llmi_qwen35_graph_tensor_count(h))]
        copy = lambda p, n, t: bytes(C.string_at(p, n * C.sizeof(t))) if n else b""
        return {"step": (d.tokens, d.past, d.capacity),
                "values": copy(d.values, d.value_count, GraphValue),
                "states": copy(d.states, d.state_count, GraphState),
                "ops": copy(d.ops, d.op_count, GraphOp),
                "outputs": [d.outputs[i] for i in range(d.output_count)],
                "tensors": tensors}
    finally:
        lib.llmi_qwen35_graph_destroy(h)


def py_graph(c, tokens, past, capacity, logits, w8, tensors):
    g = G.build_qwen35(c, tokens, past, capacity, logits, w8)
    desc, keep = marshal(g, {t: i for i, t in enumerate(tensors)})
    raw = lambda arr, n, t: bytes(C.string_at(arr, n * C.sizeof(t))) if n else b""
    return {"step": (g.tokens, g.past, g.capacity),
            "values": raw(keep[0], len(g.values), GraphValue),
            "states": raw(keep[1], len(g.states), GraphState),
            "ops": raw(keep[2], len(g.ops), GraphOp),
            "outputs": list(g.outputs),
            "tensors": [v.tensor_id for v in g.values if v.tensor_id]}


CASES = [(G.tiny_qwen35, 3, 0, 8), (G.tiny_qwen35, 1, 5, 8), (small_qwen35, 40, 0, 256),
         (small_qwen35, 1, 77, 256), (G.qwen35_4b, 1, 512, 1024), (G.qwen35_4b, 64, 0, 64)]


@pytest.mark.parametrize("make,tokens,past,capacity", CASES)
@pytest.mark.parametrize("logits", ["none", "last", "all"])
@pytest.mark.parametrize("w8", [True, False])
def test_cpp_graph_is_the_python_graph(make, tokens, past, capacity, logits, w8):
    c = make()
    want_tensors = cpp_graph(c, tokens, past, capacity, logits, w8)
    got = want_tensors
    want = py_graph(c, tokens, past, capacity, logits, w8, got["tensors"])
    assert got["tensors"] == want["tensors"]  # first-use order, the tied head once
    for key in ("step", "states", "ops", "outputs", "values"):
        assert got[key] == want[key], key


def test_capacity_zero_is_past_plus_tokens():
    c = G.tiny_qwen35()
    assert cpp_graph(c, 3, 2, 0, "last", True)["step"] == (3, 2, 5)


@pytest.mark.parametrize("tokens,past,capacity", [(0, 0, 8), (5, 4, 8), (1, 0, 257)])
def test_cpp_builder_rejects_bad_steps(tokens, past, capacity):
    c = G.tiny_qwen35()   # max_positions 256
    with pytest.raises(_lib.HipError) as e:
        cpp_graph(c, tokens, past, capacity, "last", True)
    assert e.value.status == _lib.INVALID_ARGUMENT
    with pytest.raises(G.GraphError):
        G.build_qwen35(c, tokens, past, capacity, "last", True)


def test_cpp_builder_rejects_a_bad_config():
    c = G.tiny_qwen35()
    bad = G.Qwen35Config(**{**c.__dict__, "kv_heads": 3})   # 4 query heads over 3
    with pytest.raises(_lib.HipError):
        cpp_graph(bad, 1, 0, 4, "last", True)
