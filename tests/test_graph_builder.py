"""The GraphIR builder (llminfer_amd/graph.py) against the reference's own
Graph.cpp: every graph is replayed through Graph::create / addWeight /
addState / append of lib/GraphIR/Graph.cpp, compiled from the reference's
sources into oracle/_ref, and each value's kind, element type, shape,
strides, view base and offset, defining op and group, and each op's state
effects and versions must be the reference's. Rejections must come at the
same op with the same message. The Qwen3.5 op sequence itself follows
Qwen35ModelBuilder.cpp:127-230 and is checked here by its op counts."""
import ctypes as C
from collections import Counter

import numpy as np
import pytest

import oracle
from llminfer_amd import graph as G


@pytest.fixture(scope="module")
def ref():
    if not oracle.REF_PATH.exists():
        pytest.skip("oracle/_ref not built (needs /root/reference)")
    lib = C.CDLL(str(oracle.REF_PATH))
    lib.ref_graph_replay.restype = C.c_int
    lib.ref_graph_replay.argtypes = [C.c_char_p, C.c_char_p, C.c_size_t]
    return lib


def _f(x):
    return float(np.float32(x)).hex()


def _op_line(op) -> str:
    a = op.attrs
    k = op.kind
    if k == G.OpKind.QUANTIZE_ACTIVATION:
        attr = f"quant {a['group_size']}"
    elif k in (G.OpKind.RMS_NORM, G.OpKind.GATED_RMS_NORM):
        attr = f"norm {_f(a['epsilon'])}"
    elif k == G.OpKind.L2_NORM:
        attr = f"l2 {a['group_width']} {_f(a['epsilon'])} {_f(a['scale'])}"
    elif k == G.OpKind.RESHAPE:
        attr = f"reshape {len(a['shape'])} " + " ".join(map(str, a["shape"]))
    elif k == G.OpKind.SLICE:
        attr = f"slice {a['axis']} {a['begin']} {a['length']}"
    elif k == G.OpKind.PARTIAL_ROPE:
        attr = f"rope {a['rotary_width']} {_f(a['theta'])}"
    elif k in (G.OpKind.CAUSAL_CONV1D, G.OpKind.DELTA_UPDATE):
        attr = f"state {a['state']}"
    elif k in (G.OpKind.KV_APPEND, G.OpKind.CAUSAL_GQA):
        attr = f"kv {a['keys']} {a['values']}"
    else:
        attr = "none"
    layer = -1 if op.layer is None else op.layer
    return f"op {int(k)} {layer} {len(op.inputs)} " + " ".join(map(str, op.inputs)) + " " + attr


def program(g: G.Graph, extra=None) -> str:
    """The replay program of g, in the order g was built; `extra`, an
    Operation, is appended last (a probe the reference may reject)."""
    lines = [f"step {g.tokens} {g.past} {g.capacity}"]
    for what, i in g.order:
        if what == "input":
            v = g.values[i]
            lines.append(f"input {int(v.element)} {len(v.shape)} " + " ".join(map(str, v.shape)))
        elif what == "weight":
            v = g.values[i]
            lines.append(f"weight {v.tensor_id} {int(v.element)} {v.group_size} {len(v.shape)} "
                         + " ".join(map(str, v.shape)))
        elif what == "state":
            s = g.states[i]
            lines.append(f"state {int(s.kind)} {s.layer} {int(s.element)} {len(s.shape)} "
                         + " ".join(map(str, s.shape)))
        else:
            lines.append(_op_line(g.ops[i]))
    if extra is not None:
        lines.append(_op_line(extra))
    return "\n".join(lines) + "\n"


def report(g: G.Graph) -> list[str]:
    out = []
    for v in g.values:
        out.append(" ".join(map(str, [
            "value", int(v.kind), int(v.element), len(v.shape), *v.shape, *v.strides,
            -1 if v.view_of is None else v.view_of, v.view_offset,
            -1 if v.defining_op is None else v.defining_op, v.group_size])))
    for i, op in enumerate(g.ops):
        fields = ["effects", i, len(op.effects)]
        for e in op.effects:
            fields += [e.state, int(e.access), e.begin, e.length, e.version_before, e.version_after]
        out.append(" ".join(map(str, fields)))
    return out


def replay(ref, text: str) -> list[str]:
    buf = C.create_string_buffer(8 << 20)
    assert ref.ref_graph_replay(text.encode(), buf, len(buf)) == 0
    return buf.value.decode().splitlines()


@pytest.mark.parametrize("w8", [True, False])
@pytest.mark.parametrize("tokens,past,capacity,logits", [
    (5, 0, 16, "all"), (1, 5, 16, "all"), (3, 2, 8, "last"), (1, 0, 1, "none"), (4, 0, 4, "last")])
def test_tiny_graph_matches_reference(ref, w8, tokens, past, capacity, logits):
    g = G.build_qwen35(G.tiny_qwen35(), tokens, past, capacity, logits, w8)
    assert replay(ref, program(g)) == report(g)


def test_qwen35_4b_graph_matches_reference(ref):
    g = G.build_qwen35(G.qwen35_4b(), 1, 4096, 4200, "last", True)
    assert replay(ref, program(g)) == report(g)
    kinds = Counter(G.OP_NAMES[op.kind] for op in g.ops)
    # per DeltaNet layer 4 + per GQA layer 4 + per MLP 3 projections, and the head
    assert kinds["LinearW8A8"] == 24 * 5 + 8 * 4 + 32 * 3 + 1
    assert kinds["CausalGqa"] == kinds["KvAppend"] == 8
    assert kinds["DeltaUpdate"] == kinds["CausalConv1d"] == 24
    assert kinds["RmsNorm"] == 32 * 2 + 8 * 2 + 1


def _bad(g, kind, inputs, layer=None, **attrs):
    """Append to both builders; both must reject with one message."""
    with pytest.raises(G.GraphError) as e:
        g.append(kind, inputs, layer, **attrs)
    return str(e.value)


def test_rejections_match_reference(ref):
    cases = []
    # a W8A8 projection whose scales come from another quantization
    g = G.Graph(2, 0, 4)
    x = g.add_input(G.Element.U32, (2,))
    w = g.add_weight("e", G.Element.F16, (10, 64))
    h = g.append(G.OpKind.EMBEDDING_GATHER, [x, w])[0]
    q1 = g.append(G.OpKind.QUANTIZE_ACTIVATION, [h], group_size=32)
    q2 = g.append(G.OpKind.QUANTIZE_ACTIVATION, [h], group_size=32)
    m = g.add_weight("m", G.Element.I8, (8, 64), 32)
    cases.append((g, G.OpKind.LINEAR_W8A8, [q1[0], q2[1], m], None, {}))
    # CausalGqa before the KvAppend; KvAppend twice
    for twice in (False, True):
        g = G.Graph(2, 1, 8)
        q = g.add_input(G.Element.F16, (2, 4, 16))
        k = g.add_input(G.Element.F16, (2, 2, 16))
        ks = g.add_state(G.StateKind.KEY_CACHE, 0, G.Element.F16, (8, 2, 16))
        vs = g.add_state(G.StateKind.VALUE_CACHE, 0, G.Element.F16, (8, 2, 16))
        if twice:
            g.append(G.OpKind.KV_APPEND, [k, k], 0, keys=ks, values=vs)
            cases.append((g, G.OpKind.KV_APPEND, [k, k], 0, {"keys": ks, "values": vs}))
        else:
            cases.append((g, G.OpKind.CAUSAL_GQA, [q], 0, {"keys": ks, "values": vs}))
    # a state of another layer; a slice past the end; an odd RoPE width
    g = G.Graph(3, 0, 3)
    a = g.add_input(G.Element.F16, (3, 12))
    cw = g.add_weight("c", G.Element.F16, (12, 1, 4))
    hs = g.add_state(G.StateKind.CONV_HISTORY, 1, G.Element.F16, (12, 3))
    cases.append((g, G.OpKind.CAUSAL_CONV1D, [a, cw], 0, {"state": hs}))
    cases.append((g, G.OpKind.SLICE, [a], None, {"axis": 1, "begin": 8, "length": 5}))
    r3 = g.append(G.OpKind.RESHAPE, [a], None, shape=(3, 3, 4))[0]
    cases.append((g, G.OpKind.PARTIAL_ROPE, [r3], None, {"rotary_width": 3, "theta": 1e4}))
    for g, kind, inputs, layer, attrs in cases:
        mine = _bad(g, kind, inputs, layer, **attrs)
        lines = replay(ref, program(g, G.Operation(G.OpKind(kind), layer, tuple(inputs), attrs)))
        errors = [line for line in lines if line.startswith("error")]
        assert errors == [f"error {len(g.ops)} {mine}"], (errors, mine)
