"""A typed SSA graph for one step shape, and the Qwen3.5 graph builder.

The graph is the input of the whole-graph HIP plan (llminfer_amd/plan.py,
csrc/plan.cpp). Its vocabulary is the reference's GraphIR
(include/llminfer/GraphIR/Graph.h:22-88): element types, value kinds,
state kinds and op kinds in the same order, since the plan's C ABI takes
them by number. append() infers each op's results and checks its operands,
layer-local states and state versions with the contracts of
lib/GraphIR/Graph.cpp:140-380, before the graph changes, so a graph that the
reference would reject is rejected here with the same cause.

build_qwen35() emits the op sequence of lib/Models/Qwen35/
Qwen35ModelBuilder.cpp:127-230 for a config of
lib/ModelFormat/Qwen35Schema.cpp:40-130's fields.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from enum import IntEnum

import numpy as np


class Element(IntEnum):
    I8 = 0
    U32 = 1
    F16 = 2
    F32 = 3


class ValueKind(IntEnum):
    INPUT = 0
    WEIGHT = 1
    RESULT = 2
    VIEW = 3


class StateKind(IntEnum):
    CONV_HISTORY = 0
    DELTA_RECURRENT = 1
    KEY_CACHE = 2
    VALUE_CACHE = 3


class OpKind(IntEnum):
    EMBEDDING_GATHER = 0
    QUANTIZE_ACTIVATION = 1
    LINEAR_F16 = 2
    LINEAR_W8A8 = 3
    RMS_NORM = 4
    GATED_RMS_NORM = 5
    L2_NORM = 6
    ADD = 7
    SILU = 8
    SILU_MUL = 9
    SIGMOID_MUL = 10
    RESHAPE = 11
    SLICE = 12
    PARTIAL_ROPE = 13
    CAUSAL_CONV1D = 14
    DELTA_GATES = 15
    DELTA_UPDATE = 16
    KV_APPEND = 17
    CAUSAL_GQA = 18


OP_NAMES = ("EmbeddingGather", "QuantizeActivation", "LinearF16", "LinearW8A8", "RmsNorm",
            "GatedRmsNorm", "L2Norm", "Add", "Silu", "SiluMul", "SigmoidMul", "Reshape", "Slice",
            "PartialRoPE", "CausalConv1d", "DeltaGates", "DeltaUpdate", "KvAppend", "CausalGqa")


class Access(IntEnum):
    READ = 0
    WRITE = 1
    READ_WRITE = 2


class GraphError(ValueError):
    pass


@dataclass
class Value:
    element: Element
    shape: tuple
    strides: tuple
    kind: ValueKind
    tensor_id: str = ""
    group_size: int = 0
    defining_op: int | None = None
    view_of: int | None = None
    view_offset: int = 0          # elements, relative to view_of


@dataclass
class State:
    kind: StateKind
    layer: int
    element: Element
    shape: tuple


@dataclass
class Effect:
    state: int
    access: Access
    begin: int
    length: int
    version_before: int
    version_after: int


@dataclass
class Operation:
    kind: OpKind
    layer: int | None
    inputs: tuple
    attrs: dict
    outputs: list = field(default_factory=list)
    effects: list = field(default_factory=list)


def dense_strides(shape) -> tuple:
    if not shape:
        raise GraphError("A tensor must have positive rank")
    strides, stride = [0] * len(shape), 1
    for i in range(len(shape) - 1, -1, -1):
        strides[i] = stride
        stride *= shape[i]
    return tuple(strides)


def is_dense(v: Value) -> bool:
    stride = 1
    for dim, st in zip(reversed(v.shape), reversed(v.strides)):
        if dim > 1 and st != stride:
            return False
        stride *= dim
    return True


def _positive(x: float) -> bool:
    return math.isfinite(x) and x > 0


def _make_value(element: Element, shape, kind: ValueKind, group: int = 0) -> Value:
    shape = tuple(int(d) for d in shape)
    if any(d == 0 for d in shape):
        raise GraphError("Value dimensions must be positive")
    strides = list(dense_strides(shape))
    if group:
        if element != Element.I8 or len(shape) != 2:
            raise GraphError("Invalid grouped INT8 storage")
        strides[0] = (shape[1] + group - 1) // group * group
    return Value(element, shape, tuple(strides), kind, group_size=group)


class Graph:
    """One step's graph: tokens new rows after past cached ones, caches of
    capacity rows (Graph.cpp:380-386)."""

    def __init__(self, tokens: int, past: int, capacity: int):
        if not tokens or past > capacity or tokens > capacity - past:
            raise GraphError("Invalid graph step: expected 0 < tokens <= capacity - past")
        self.tokens, self.past, self.capacity = tokens, past, capacity
        self.values: list[Value] = []
        self.states: list[State] = []
        self.versions: list[int] = []
        self.ops: list[Operation] = []
        self.outputs: list[int] = []
        self.order: list[tuple[str, int]] = []   # ("input" | "weight" | "state" | "op", index)

    # ---------------------------------------------------------- sources
    def add_input(self, element: Element, shape) -> int:
        self.values.append(_make_value(element, shape, ValueKind.INPUT))
        self.order.append(("input", len(self.values) - 1))
        return len(self.values) - 1

    def add_weight(self, tensor_id: str, element: Element, shape, group: int = 0) -> int:
        if not tensor_id or (element == Element.I8) != (group != 0) or element == Element.U32:
            raise GraphError("Invalid graph weight declaration")
        shape = tuple(int(d) for d in shape)
        for i, v in enumerate(self.values):
            if v.kind == ValueKind.WEIGHT and v.tensor_id == tensor_id:
                if v.element != element or v.shape != shape or v.group_size != group:
                    raise GraphError("Conflicting type for weight " + tensor_id)
                return i
        v = _make_value(element, shape, ValueKind.WEIGHT, group)
        v.tensor_id = tensor_id
        self.values.append(v)
        self.order.append(("weight", len(self.values) - 1))
        return len(self.values) - 1

    def add_state(self, kind: StateKind, layer: int, element: Element, shape) -> int:
        shape = tuple(int(d) for d in shape)
        history = kind == StateKind.CONV_HISTORY
        recurrent = kind == StateKind.DELTA_RECURRENT
        if len(shape) != (2 if history else 3) or \
                element != (Element.F32 if recurrent else Element.F16) or not shape[0] or \
                (not history and 0 in shape) or \
                (not history and not recurrent and shape[0] != self.capacity):
            raise GraphError("Invalid graph state type")
        if any(s.kind == kind and s.layer == layer for s in self.states):
            raise GraphError("Duplicate state slot in layer")
        self.states.append(State(kind, layer, element, shape))
        self.versions.append(0)
        self.order.append(("state", len(self.states) - 1))
        return len(self.states) - 1

    def set_outputs(self, outputs) -> None:
        for v in outputs:
            if v >= len(self.values):
                raise GraphError("Graph output has no definition")
        self.outputs = list(outputs)

    # -------------------------------------------------------------- ops
    def append(self, kind: OpKind, inputs, layer: int | None = None, **attrs) -> list[int]:
        for i in inputs:
            if i >= len(self.values):
                raise GraphError("Graph operand has no preceding definition")
        op = Operation(OpKind(kind), layer, tuple(inputs), attrs)
        try:
            results = _Inference(self, op).run()
        except GraphError as e:
            raise GraphError(f"{OP_NAMES[kind]}: {e}") from None
        for v in results:
            v.defining_op = len(self.ops)
            op.outputs.append(len(self.values))
            self.values.append(v)
        for e in op.effects:
            self.versions[e.state] = e.version_after
        self.ops.append(op)
        self.order.append(("op", len(self.ops) - 1))
        return list(op.outputs)


class _Inference:
    """Result inference and operand checks of Graph.cpp:140-380."""

    def __init__(self, g: Graph, op: Operation):
        self.g, self.op = g, op
        self.results: list[Value] = []

    def arg(self, i) -> Value:
        return self.g.values[self.op.inputs[i]]

    def shape(self, i) -> tuple:
        return self.arg(i).shape

    def signature(self, n, *attrs) -> bool:
        return len(self.op.inputs) == n and all(a in self.op.attrs for a in attrs)

    def tensor(self, i, element, rank) -> bool:
        return self.arg(i).element == element and len(self.shape(i)) == rank

    def weight(self, i, element, rank) -> bool:
        return self.arg(i).kind == ValueKind.WEIGHT and self.tensor(i, element, rank)

    def result(self, element, shape, group=0):
        self.results.append(_make_value(element, shape, ValueKind.RESULT, group))

    def view(self, shape, strides, offset):
        a = self.arg(0)
        self.results.append(Value(a.element, tuple(shape), tuple(strides), ValueKind.VIEW,
                                  view_of=self.op.inputs[0], view_offset=offset))

    def state(self, sid, kind) -> State | None:
        if sid is None or sid >= len(self.g.states):
            return None
        s = self.g.states[sid]
        if s.kind != kind or self.op.layer != s.layer:
            return None
        return s

    def effect(self, sid, access, begin, length):
        v = self.g.versions[sid]
        self.op.effects.append(Effect(sid, access, begin, length, v,
                                      v + (access != Access.READ)))

    def run(self) -> list[Value]:
        k, g, a = self.op.kind, self.g, self.op.attrs
        if k == OpKind.EMBEDDING_GATHER:
            if not self.signature(2) or not self.tensor(0, Element.U32, 1) or \
                    self.shape(0)[0] != g.tokens or \
                    not (self.weight(1, Element.I8, 2) or self.weight(1, Element.F16, 2)):
                raise GraphError("Expected step token IDs and an embedding table")
            self.result(Element.F16, (self.shape(0)[0], self.shape(1)[1]))
        elif k == OpKind.QUANTIZE_ACTIVATION:
            if not self.signature(1, "group_size") or not self.tensor(0, Element.F16, 2) or \
                    not a["group_size"]:
                raise GraphError("Invalid activation quantization")
            rows, width = self.shape(0)
            self.result(Element.I8, (rows, width), a["group_size"])
            self.result(Element.F32, (rows, 1 + (width - 1) // a["group_size"]))
        elif k in (OpKind.LINEAR_F16, OpKind.LINEAR_W8A8):
            self.linear()
        elif k in (OpKind.RMS_NORM, OpKind.GATED_RMS_NORM, OpKind.L2_NORM):
            self.normalize()
        elif k in (OpKind.ADD, OpKind.SILU_MUL, OpKind.SIGMOID_MUL):
            if not self.signature(2) or self.arg(0).element != Element.F16 or \
                    self.arg(1).element != Element.F16 or self.shape(0) != self.shape(1):
                raise GraphError("Expected two matching FP16 operands")
            self.result(Element.F16, self.shape(0))
        elif k == OpKind.SILU:
            if not self.signature(1) or self.arg(0).element != Element.F16:
                raise GraphError("Expected a single FP16 operand")
            self.result(Element.F16, self.shape(0))
        elif k in (OpKind.RESHAPE, OpKind.SLICE):
            self.views()
        elif k == OpKind.PARTIAL_ROPE:
            if not self.signature(1, "rotary_width", "theta") or \
                    not self.tensor(0, Element.F16, 3) or self.shape(0)[0] != g.tokens or \
                    not a["rotary_width"] or a["rotary_width"] % 2 or \
                    a["rotary_width"] > self.shape(0)[-1] or not _positive(a["theta"]):
                raise GraphError("Invalid partial RoPE parameters")
            self.result(Element.F16, self.shape(0))
        elif k == OpKind.CAUSAL_CONV1D:
            if not self.signature(2, "state") or not self.tensor(0, Element.F16, 2) or \
                    not self.weight(1, Element.F16, 3) or self.shape(1)[1] != 1 or \
                    self.shape(0) != (g.tokens, self.shape(1)[0]):
                raise GraphError("Expected a step activation and depthwise filter")
            s = self.state(a["state"], StateKind.CONV_HISTORY)
            if s is None or g.versions[a["state"]] != 0 or \
                    s.shape != (self.shape(1)[0], self.shape(1)[2] - 1):
                raise GraphError("Invalid convolution history")
            self.effect(a["state"], Access.READ_WRITE, 0, self.shape(1)[0])
            self.result(Element.F16, self.shape(0))
        elif k == OpKind.DELTA_GATES:
            if not self.signature(4) or not self.tensor(0, Element.F16, 2) or \
                    not self.tensor(1, Element.F16, 2) or self.shape(0) != self.shape(1) or \
                    self.shape(0)[0] != g.tokens or not self.weight(2, Element.F32, 1) or \
                    not self.weight(3, Element.F32, 1) or self.shape(2) != self.shape(3) or \
                    self.shape(2)[0] != self.shape(0)[1]:
                raise GraphError("Invalid DeltaNet gate inputs")
            self.result(Element.F32, self.shape(0))
            self.result(Element.F32, self.shape(0))
        elif k == OpKind.DELTA_UPDATE:
            self.delta_update()
        elif k in (OpKind.KV_APPEND, OpKind.CAUSAL_GQA):
            self.kv()
        else:
            raise GraphError("Unknown GraphIR operation")
        return self.results

    def linear(self):
        if self.op.kind == OpKind.LINEAR_F16:
            if not self.signature(2) or not self.tensor(0, Element.F16, 2) or \
                    not self.weight(1, Element.F16, 2) or self.shape(0)[1] != self.shape(1)[1]:
                raise GraphError("Expected compatible FP16 activation and weight matrices")
            self.result(Element.F16, (self.shape(0)[0], self.shape(1)[0]))
            return
        if not self.signature(3) or not self.tensor(0, Element.I8, 2) or \
                not self.tensor(1, Element.F32, 2) or not self.weight(2, Element.I8, 2) or \
                self.shape(0)[1] != self.shape(2)[1] or self.arg(0).defining_op is None or \
                self.arg(0).defining_op != self.arg(1).defining_op:
            raise GraphError("Expected a matching quantized activation and weight")
        q = self.g.ops[self.arg(0).defining_op]
        if q.kind != OpKind.QUANTIZE_ACTIVATION or q.outputs[0] != self.op.inputs[0] or \
                q.outputs[1] != self.op.inputs[1] or \
                self.arg(0).group_size != self.arg(2).group_size:
            raise GraphError("Activation data and scales must come from the same matching "
                             "quantization")
        self.result(Element.F16, (self.shape(0)[0], self.shape(2)[0]))

    def normalize(self):
        a = self.op.attrs
        if self.op.kind == OpKind.L2_NORM:
            if not self.signature(1, "group_width", "epsilon", "scale") or \
                    not self.tensor(0, Element.F16, 2) or not a["group_width"] or \
                    self.shape(0)[-1] % a["group_width"] or not _positive(a["epsilon"]) or \
                    not _positive(a["scale"]):
                raise GraphError("Invalid grouped L2 normalization")
            self.result(Element.F32, self.shape(0))
            return
        gated = self.op.kind == OpKind.GATED_RMS_NORM
        w = 2 if gated else 1
        if not self.signature(3 if gated else 2, "epsilon") or not _positive(a["epsilon"]) or \
                self.arg(0).element != Element.F16 or not self.weight(w, Element.F32, 1):
            raise GraphError("Invalid RMS normalization")
        width = self.shape(w)[0]
        if gated:
            if self.arg(1).element != Element.F16 or self.shape(1) != self.shape(0) or \
                    self.shape(0)[-1] % width:
                raise GraphError("Invalid gated RMS normalization shapes")
        elif self.shape(0)[-1] != width:
            raise GraphError("RMS normalization weight does not match the last axis")
        self.result(Element.F16, self.shape(0))

    def views(self):
        a = self.op.attrs
        if len(self.op.inputs) != 1 or self.arg(0).kind == ValueKind.WEIGHT or \
                self.arg(0).group_size:
            raise GraphError("Expected a single ungrouped activation")
        if self.op.kind == OpKind.SLICE:
            if not self.signature(1, "axis", "begin", "length") or \
                    a["axis"] >= len(self.shape(0)):
                raise GraphError("Invalid slice axis")
            width = self.shape(0)[a["axis"]]
            if a["begin"] > width or not a["length"] or a["length"] > width - a["begin"]:
                raise GraphError("Slice is outside the operand")
            dims = list(self.shape(0))
            dims[a["axis"]] = a["length"]
            self.view(dims, self.arg(0).strides, a["begin"] * self.arg(0).strides[a["axis"]])
            return
        shape = tuple(int(d) for d in a.get("shape", ()))
        if "shape" not in a or not is_dense(self.arg(0)) or 0 in shape:
            raise GraphError("Reshape requires contiguous storage and positive dimensions")
        if math.prod(shape) != math.prod(self.shape(0)):
            raise GraphError("Reshape changes the element count")
        self.view(shape, dense_strides(shape), 0)

    def delta_update(self):
        a, g = self.op.attrs, self.g
        if not self.signature(5, "state"):
            raise GraphError("DeltaUpdate expects Q, K, V, beta and decay")
        s = self.state(a["state"], StateKind.DELTA_RECURRENT)
        if s is None or g.versions[a["state"]] != 0:
            raise GraphError("Expected an unwritten recurrent state in this layer")
        hv, dk, dv = s.shape
        t = g.tokens
        if not self.tensor(0, Element.F32, 2) or not self.tensor(1, Element.F32, 2) or \
                self.shape(0)[0] != t or self.shape(1) != self.shape(0) or \
                self.shape(0)[1] % dk or hv % (self.shape(0)[1] // dk) or \
                not self.tensor(2, Element.F16, 2) or self.shape(2) != (t, hv * dv) or \
                not self.tensor(3, Element.F32, 2) or self.shape(3) != (t, hv) or \
                not self.tensor(4, Element.F32, 2) or self.shape(4) != self.shape(3):
            raise GraphError("DeltaUpdate operand shapes do not match its recurrent state")
        self.effect(a["state"], Access.READ_WRITE, 0, hv)
        self.result(Element.F16, self.shape(2))

    def kv(self):
        a, g = self.op.attrs, self.g
        append = self.op.kind == OpKind.KV_APPEND
        if not self.signature(2 if append else 1, "keys", "values"):
            raise GraphError("Expected key and value cache slots")
        keys = self.state(a["keys"], StateKind.KEY_CACHE)
        vals = self.state(a["values"], StateKind.VALUE_CACHE)
        if keys is None or vals is None or keys.shape != vals.shape:
            raise GraphError("Expected compatible key and value caches in this layer")
        dims = keys.shape
        if not self.tensor(0, Element.F16, 3) or self.shape(0)[0] != g.tokens or \
                self.shape(0)[2] != dims[2] or self.shape(0)[1] % dims[1]:
            raise GraphError("Invalid attention head shape")
        version = 0 if append else 1
        if g.versions[a["keys"]] != version or g.versions[a["values"]] != version:
            raise GraphError("KV cache is already appended" if append
                             else "Attention requires the appended KV version")
        if append:
            if not self.tensor(1, Element.F16, 3) or self.shape(0) != self.shape(1) or \
                    self.shape(0)[1] != dims[1]:
                raise GraphError("New keys and values must match the cache layout")
            self.effect(a["keys"], Access.WRITE, g.past, g.tokens)
            self.effect(a["values"], Access.WRITE, g.past, g.tokens)
            return
        self.effect(a["keys"], Access.READ, 0, g.past + g.tokens)
        self.effect(a["values"], Access.READ, 0, g.past + g.tokens)
        self.result(Element.F16, self.shape(0))


# ----------------------------------------------------------------- Qwen3.5

EMBEDDING_ID = "embed_tokens.weight"   # Qwen35Schema.h:10
HEAD_ID = "lm_head.weight"             # Qwen35Schema.h:11 (tied: resolves to the embedding)
WEIGHT_GROUP = 32


@dataclass
class Qwen35Config:
    """The text config fields the graph uses (Qwen35Schema.h:16-23)."""
    hidden: int
    intermediate: int
    vocabulary: int
    head_dim: int
    q_heads: int
    kv_heads: int
    rotary_width: int
    key_heads: int
    value_heads: int
    key_dim: int
    value_dim: int
    conv_kernel: int
    layers: tuple          # "delta" or "gqa" per layer
    epsilon: float = 1e-6
    theta: float = 1e7
    max_positions: int = 262144

    @property
    def query_width(self):
        return self.q_heads * self.head_dim

    @property
    def kv_width(self):
        return self.kv_heads * self.head_dim

    @property
    def linear_key_width(self):
        return self.key_heads * self.key_dim

    @property
    def linear_value_width(self):
        return self.value_heads * self.value_dim

    @property
    def linear_qkv_width(self):
        return 2 * self.linear_key_width + self.linear_value_width


def qwen35_4b() -> Qwen35Config:
    """Qwen3.5-4B's text backbone (docs/architecture.md:115): 32 layers,
    24 Gated DeltaNet and 8 Gated GQA (every fourth), hidden 2560, MLP 9216,
    vocabulary 248320; GQA 16 query / 4 KV heads of 256 with a 64-wide
    partial RoPE; DeltaNet 16 key / 32 value heads of 128, conv kernel 4."""
    return Qwen35Config(hidden=2560, intermediate=9216, vocabulary=248320, head_dim=256,
                        q_heads=16, kv_heads=4, rotary_width=64, key_heads=16, value_heads=32,
                        key_dim=128, value_dim=128, conv_kernel=4,
                        layers=tuple("gqa" if i % 4 == 3 else "delta" for i in range(32)))


def tiny_qwen35() -> Qwen35Config:
    """The reference's two-layer test model (tests/MetalReferenceTest.py:19-53):
    odd widths everywhere, one DeltaNet and one GQA layer."""
    return Qwen35Config(hidden=33, intermediate=19, vocabulary=37, head_dim=12, q_heads=4,
                        kv_heads=2, rotary_width=6, key_heads=2, value_heads=4, key_dim=7,
                        value_dim=5, conv_kernel=4, layers=("delta", "gqa"), max_positions=256)


def qwen35_tensors(c: Qwen35Config, w8: bool) -> dict[str, tuple]:
    """Tensor id -> (Element, shape) of the model (Qwen35Schema.cpp:133-178)."""
    matrix = Element.I8 if w8 else Element.F16
    t = {EMBEDDING_ID: (matrix, (c.vocabulary, c.hidden)), "norm.weight": (Element.F32, (c.hidden,))}
    for i, kind in enumerate(c.layers):
        p = f"layers.{i}."
        t[p + "input_layernorm.weight"] = (Element.F32, (c.hidden,))
        t[p + "post_attention_layernorm.weight"] = (Element.F32, (c.hidden,))
        t[p + "mlp.gate_proj.weight"] = (matrix, (c.intermediate, c.hidden))
        t[p + "mlp.up_proj.weight"] = (matrix, (c.intermediate, c.hidden))
        t[p + "mlp.down_proj.weight"] = (matrix, (c.hidden, c.intermediate))
        if kind == "delta":
            q = p + "linear_attn."
            t[q + "in_proj_qkv.weight"] = (matrix, (c.linear_qkv_width, c.hidden))
            t[q + "in_proj_z.weight"] = (matrix, (c.linear_value_width, c.hidden))
            t[q + "in_proj_a.weight"] = (matrix, (c.value_heads, c.hidden))
            t[q + "in_proj_b.weight"] = (matrix, (c.value_heads, c.hidden))
            t[q + "out_proj.weight"] = (matrix, (c.hidden, c.linear_value_width))
            t[q + "conv1d.weight"] = (Element.F16, (c.linear_qkv_width, 1, c.conv_kernel))
            t[q + "norm.weight"] = (Element.F32, (c.value_dim,))
            t[q + "A_log"] = (Element.F32, (c.value_heads,))
            t[q + "dt_bias"] = (Element.F32, (c.value_heads,))
        else:
            q = p + "self_attn."
            t[q + "q_proj.weight"] = (matrix, (2 * c.query_width, c.hidden))
            t[q + "k_proj.weight"] = (matrix, (c.kv_width, c.hidden))
            t[q + "v_proj.weight"] = (matrix, (c.kv_width, c.hidden))
            t[q + "o_proj.weight"] = (matrix, (c.hidden, c.query_width))
            t[q + "q_norm.weight"] = (Element.F32, (c.head_dim,))
            t[q + "k_norm.weight"] = (Element.F32, (c.head_dim,))
    return t


def build_qwen35(c: Qwen35Config, tokens: int, past: int = 0, capacity: int | None = None,
                 logits: str = "all", w8: bool = True) -> Graph:
    """The Qwen3.5 graph of one step (Qwen35ModelBuilder.cpp:127-230); logits
    "all" (every row), "last" (the last row) or "none"."""
    if capacity is None:
        capacity = past + tokens
    if capacity > c.max_positions:
        raise GraphError("Graph capacity exceeds the model context limit")
    g = Graph(tokens, past, capacity)
    tensors = qwen35_tensors(c, w8)
    layer: list[int | None] = [None]

    def emit(kind, inputs, **attrs):
        return g.append(kind, inputs, layer[0], **attrs)

    def op(kind, inputs, **attrs):
        return emit(kind, inputs, **attrs)[0]

    def weight(name):
        tid = EMBEDDING_ID if name == HEAD_ID else name
        element, shape = tensors[tid]
        return g.add_weight(tid, element, shape, WEIGHT_GROUP if element == Element.I8 else 0)

    def prepare(x):
        if w8:
            return x, emit(OpKind.QUANTIZE_ACTIVATION, [x], group_size=WEIGHT_GROUP)
        return x, None

    def project(prep, name):
        x, q = prep
        m = weight(name)
        if w8:
            return op(OpKind.LINEAR_W8A8, [q[0], q[1], m])
        return op(OpKind.LINEAR_F16, [x, m])

    def norm(x, name):
        return op(OpKind.RMS_NORM, [x, weight(name)], epsilon=c.epsilon)

    def delta(x, pre):
        history = g.add_state(StateKind.CONV_HISTORY, layer[0], Element.F16,
                              (c.linear_qkv_width, c.conv_kernel - 1))
        recurrent = g.add_state(StateKind.DELTA_RECURRENT, layer[0], Element.F32,
                                (c.value_heads, c.key_dim, c.value_dim))
        prep = prepare(x)
        qkv = project(prep, pre + "in_proj_qkv.weight")
        z = project(prep, pre + "in_proj_z.weight")
        a = project(prep, pre + "in_proj_a.weight")
        b = project(prep, pre + "in_proj_b.weight")
        qkv = op(OpKind.CAUSAL_CONV1D, [qkv, weight(pre + "conv1d.weight")], state=history)
        qkv = op(OpKind.SILU, [qkv])
        kw, vw = c.linear_key_width, c.linear_value_width
        q = op(OpKind.SLICE, [qkv], axis=1, begin=0, length=kw)
        k = op(OpKind.SLICE, [qkv], axis=1, begin=kw, length=kw)
        v = op(OpKind.SLICE, [qkv], axis=1, begin=2 * kw, length=vw)
        # 1 / sqrt(dk) in fp32 arithmetic, as the builder computes it
        scale = float(np.float32(1.0) / np.sqrt(np.float32(c.key_dim)))
        q = op(OpKind.L2_NORM, [q], group_width=c.key_dim, epsilon=1e-6, scale=scale)
        k = op(OpKind.L2_NORM, [k], group_width=c.key_dim, epsilon=1e-6, scale=1.0)
        gates = emit(OpKind.DELTA_GATES, [a, b, weight(pre + "A_log"), weight(pre + "dt_bias")])
        mixed = op(OpKind.DELTA_UPDATE, [q, k, v, gates[0], gates[1]], state=recurrent)
        gated = op(OpKind.GATED_RMS_NORM, [mixed, z, weight(pre + "norm.weight")],
                   epsilon=c.epsilon)
        return project(prepare(gated), pre + "out_proj.weight")

    def gqa(x, pre):
        shape = (capacity, c.kv_heads, c.head_dim)
        keys = g.add_state(StateKind.KEY_CACHE, layer[0], Element.F16, shape)
        values = g.add_state(StateKind.VALUE_CACHE, layer[0], Element.F16, shape)
        prep = prepare(x)
        q_gate = project(prep, pre + "q_proj.weight")
        k = project(prep, pre + "k_proj.weight")
        v = project(prep, pre + "v_proj.weight")
        q_gate = op(OpKind.RESHAPE, [q_gate], shape=(tokens, c.q_heads, 2 * c.head_dim))
        q = op(OpKind.SLICE, [q_gate], axis=2, begin=0, length=c.head_dim)
        gate = op(OpKind.SLICE, [q_gate], axis=2, begin=c.head_dim, length=c.head_dim)
        k = op(OpKind.RESHAPE, [k], shape=(tokens, c.kv_heads, c.head_dim))
        v = op(OpKind.RESHAPE, [v], shape=(tokens, c.kv_heads, c.head_dim))
        q = norm(q, pre + "q_norm.weight")
        k = norm(k, pre + "k_norm.weight")
        q = op(OpKind.PARTIAL_ROPE, [q], rotary_width=c.rotary_width, theta=c.theta)
        k = op(OpKind.PARTIAL_ROPE, [k], rotary_width=c.rotary_width, theta=c.theta)
        emit(OpKind.KV_APPEND, [k, v], keys=keys, values=values)
        mixed = op(OpKind.CAUSAL_GQA, [q], keys=keys, values=values)
        mixed = op(OpKind.SIGMOID_MUL, [gate, mixed])
        mixed = op(OpKind.RESHAPE, [mixed], shape=(tokens, c.query_width))
        return project(prepare(mixed), pre + "o_proj.weight")

    def mlp(x, pre):
        prep = prepare(x)
        gate = project(prep, pre + "gate_proj.weight")
        up = project(prep, pre + "up_proj.weight")
        return project(prepare(op(OpKind.SILU_MUL, [gate, up])), pre + "down_proj.weight")

    ids = g.add_input(Element.U32, (tokens,))
    hidden = op(OpKind.EMBEDDING_GATHER, [ids, weight(EMBEDDING_ID)])
    for i, kind in enumerate(c.layers):
        layer[0] = i
        pre = f"layers.{i}."
        x = norm(hidden, pre + "input_layernorm.weight")
        mixed = delta(x, pre + "linear_attn.") if kind == "delta" else gqa(x, pre + "self_attn.")
        residual = op(OpKind.ADD, [hidden, mixed])
        x = norm(residual, pre + "post_attention_layernorm.weight")
        hidden = op(OpKind.ADD, [residual, mlp(x, pre + "mlp.")])
    layer[0] = None
    outputs = []
    if logits != "none":
        if logits == "last" and tokens > 1:
            hidden = op(OpKind.SLICE, [hidden], axis=0, begin=tokens - 1, length=1)
        hidden = norm(hidden, "norm.weight")
        outputs.append(project(prepare(hidden), HEAD_ID))
    g.set_outputs(outputs)
    return g
