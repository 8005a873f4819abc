"""Bindings of the whole-graph HIP plan and of the C++ model session.

Plan lowers one step's graph (llminfer_amd.graph.Graph) through the C ABI
(llmi_hip_plan_lower, csrc/plan.cpp) and runs it, or wraps a plan the model
session lowered. ModelSession binds the C++ session (llmi_hip_model_*,
csrc/model.cpp), the part of the reference's MetalSession
(include/llminfer/Backend/Metal/MetalSession.h:26-50, MetalExecutor.mm:
212-298): the session owns the per-layer states, builds the Qwen3.5 graph of
each step in C++, lowers and runs it, and returns the logits with the plan
records.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np
import torch

from . import _lib
from .graph import (EMBEDDING_ID, Element, Graph, OpKind, Qwen35Config, StateKind, build_qwen35,
                    qwen35_tensors)

_MAX_RANK = 4


class GraphValue(C.Structure):
    _fields_ = [("element", C.c_uint32), ("kind", C.c_uint32), ("rank", C.c_uint32),
                ("reserved", C.c_uint32), ("shape", C.c_uint64 * _MAX_RANK),
                ("strides", C.c_uint64 * _MAX_RANK), ("view_of", C.c_int64),
                ("defining_op", C.c_int64), ("weight", C.c_int64), ("view_offset", C.c_uint64),
                ("group_size", C.c_uint64)]


class GraphState(C.Structure):
    _fields_ = [("kind", C.c_uint32), ("layer", C.c_uint32), ("element", C.c_uint32),
                ("rank", C.c_uint32), ("shape", C.c_uint64 * _MAX_RANK)]


class GraphOp(C.Structure):
    _fields_ = [("kind", C.c_uint32), ("layer", C.c_int32), ("input_count", C.c_uint32),
                ("output_count", C.c_uint32), ("inputs", C.c_uint32 * 5),
                ("outputs", C.c_uint32 * 2), ("state", C.c_uint32), ("keys", C.c_uint32),
                ("values", C.c_uint32), ("group_size", C.c_uint64), ("group_width", C.c_uint64),
                ("axis", C.c_uint64), ("begin", C.c_uint64), ("length", C.c_uint64),
                ("rotary_width", C.c_uint64), ("epsilon", C.c_float), ("scale", C.c_float),
                ("theta", C.c_float), ("reserved", C.c_float)]


class GraphDesc(C.Structure):
    _fields_ = [("tokens", C.c_uint64), ("past", C.c_uint64), ("capacity", C.c_uint64),
                ("values", C.POINTER(GraphValue)), ("value_count", C.c_size_t),
                ("states", C.POINTER(GraphState)), ("state_count", C.c_size_t),
                ("ops", C.POINTER(GraphOp)), ("op_count", C.c_size_t),
                ("outputs", C.POINTER(C.c_uint32)), ("output_count", C.c_size_t)]


class WeightDesc(C.Structure):
    _fields_ = [("data", C.c_void_p), ("scales", C.c_void_p)]


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise _lib.HipError(rc, f"{what}: {_lib.load().llmi_hip_last_error().decode()}")


def marshal(g: Graph, weight_index: dict[str, int]):
    """The flat llmi_graph of g; weight values refer to weight_index[tensor_id]."""
    values = (GraphValue * len(g.values))()
    for i, v in enumerate(g.values):
        d = values[i]
        d.element, d.kind, d.rank = int(v.element), int(v.kind), len(v.shape)
        for k, (n, s) in enumerate(zip(v.shape, v.strides)):
            d.shape[k], d.strides[k] = n, s
        d.view_of = -1 if v.view_of is None else v.view_of
        d.defining_op = -1 if v.defining_op is None else v.defining_op
        d.weight = weight_index[v.tensor_id] if v.tensor_id else -1
        d.view_offset, d.group_size = v.view_offset, v.group_size
    states = (GraphState * max(1, len(g.states)))()
    for i, s in enumerate(g.states):
        d = states[i]
        d.kind, d.layer, d.element, d.rank = int(s.kind), s.layer, int(s.element), len(s.shape)
        for k, n in enumerate(s.shape):
            d.shape[k] = n
    ops = (GraphOp * len(g.ops))()
    for i, op in enumerate(g.ops):
        d, a = ops[i], op.attrs
        d.kind = int(op.kind)
        d.layer = -1 if op.layer is None else op.layer
        d.input_count, d.output_count = len(op.inputs), len(op.outputs)
        for k, x in enumerate(op.inputs):
            d.inputs[k] = x
        for k, x in enumerate(op.outputs):
            d.outputs[k] = x
        d.state = a.get("state", 0)
        d.keys, d.values = a.get("keys", 0), a.get("values", 0)
        d.group_size = a.get("group_size", 0)
        d.group_width = a.get("group_width", 0)
        d.axis, d.begin, d.length = a.get("axis", 0), a.get("begin", 0), a.get("length", 0)
        d.rotary_width = a.get("rotary_width", 0)
        d.epsilon, d.scale, d.theta = a.get("epsilon", 0.0), a.get("scale", 0.0), \
            a.get("theta", 0.0)
    outputs = (C.c_uint32 * max(1, len(g.outputs)))(*g.outputs)
    desc = GraphDesc(g.tokens, g.past, g.capacity, values, len(g.values), states, len(g.states),
                     ops, len(g.ops), outputs, len(g.outputs))
    return desc, (values, states, ops, outputs)


class Plan:
    """A lowered step: llmi_hip_plan_lower's result, owned here."""

    def __init__(self, g: Graph | None, weight_table: list[tuple[int, int]] | None = None,
                 weight_index: dict[str, int] | None = None, handle=None):
        lib = _lib.load()
        if handle is None:
            desc, self._keep = marshal(g, weight_index)
            table = (WeightDesc * max(1, len(weight_table)))(
                *[WeightDesc(d, s) for d, s in weight_table])
            self._table = table
            handle = C.c_void_p()
            _check(lib.llmi_hip_plan_lower(C.byref(desc), table, len(weight_table),
                                           C.byref(handle)), "plan lowering")
        self._h = handle
        self.scratch_bytes = lib.llmi_hip_plan_scratch_bytes(handle)
        rows, elements = C.c_uint64(), C.c_uint64()
        lib.llmi_hip_plan_logits(handle, C.byref(rows), C.byref(elements))
        self.logit_rows, self.logit_elements = rows.value, elements.value
        self.launches = lib.llmi_hip_plan_launches(handle)  # kernel launches a step
        self.dispatches = records(lib.llmi_hip_plan_dispatches, handle)
        self.graph = g

    def execute(self, scratch: torch.Tensor, states: list[torch.Tensor], ids: torch.Tensor,
                logits: torch.Tensor | None, invalid: torch.Tensor | None) -> None:
        ptrs = (C.c_void_p * max(1, len(states)))(*[s.data_ptr() for s in states])
        _check(_lib.load().llmi_hip_plan_execute(
            self._h, scratch.data_ptr(), scratch.numel(), ptrs, len(states), ids.data_ptr(),
            None if logits is None else logits.data_ptr(),
            None if invalid is None else invalid.data_ptr(),
            torch.cuda.current_stream().cuda_stream), "plan execution")

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value and _lib is not None and _lib._lib is not None:
            _lib._lib.llmi_hip_plan_destroy(h)
            self._h = None


def records(query, handle) -> list[dict]:
    """Plan records {op_index, kernel[, epilogue, fused_op_index]}
    (tools/run/Main.cpp:244-255) from a (handle, records, cap) query."""
    n = query(handle, None, 0)
    recs = (_lib.Dispatch * max(1, n))()
    query(handle, recs, n)
    out = []
    for r in recs[:n]:
        d = {"op_index": r.op_index, "kernel": r.kernel.decode()}
        if r.epilogue:
            d["epilogue"] = r.epilogue.decode()
            d["fused_op_index"] = r.fused_op_index
        out.append(d)
    return out


_TORCH = {Element.I8: torch.int8, Element.U32: torch.int32, Element.F16: torch.float16,
          Element.F32: torch.float32}


@dataclass
class StepResult:
    """MetalStepResult (MetalSession.h:18-24)."""
    past: int
    logit_rows: int
    scratch_bytes: int
    dispatch_count: int
    logits: np.ndarray | None
    dispatches: list = field(default_factory=list)


def random_weights(c: Qwen35Config, w8: bool, device, seed: int = 0) -> dict:
    """Random device weights of the model's shapes: int8 matrices with fp16
    group scales (rows padded to whole groups), fp16 matrices, fp32 vectors
    (norm weights near 0, the zero-centred RMSNorm; A_log and dt_bias small)."""
    g = torch.Generator(device=device).manual_seed(seed)
    out = {}
    for tid, (element, shape) in qwen35_tensors(c, w8).items():
        if element == Element.I8:
            rows, width = shape
            groups = (width + 31) // 32
            data = torch.zeros(rows, groups * 32, dtype=torch.int8, device=device)
            data[:, :width] = torch.randint(-127, 128, (rows, width), generator=g, device=device,
                                            dtype=torch.int8)
            scales = (torch.rand(rows, groups, generator=g, device=device) * 2e-3 + 2e-4).half()
            out[tid] = (data, scales)
        elif element == Element.F16:
            out[tid] = ((torch.randn(shape, generator=g, device=device) * 0.1).half(), None)
        else:
            v = torch.randn(shape, generator=g, device=device) * 0.1
            if tid.endswith("linear_attn.norm.weight"):
                v = v + 1.0    # gatedRmsNorm multiplies by the weight directly
            out[tid] = (v.float(), None)
    return out


class Qwen35Config_C(C.Structure):
    """llmi_qwen35_config (include/llminfer_hip.h)."""
    _fields_ = [(n, C.c_uint64) for n in (
        "hidden", "intermediate", "vocabulary", "max_positions", "head_dim", "q_heads",
        "kv_heads", "rotary_width", "key_heads", "value_heads", "key_dim", "value_dim",
        "conv_kernel")] + [("epsilon", C.c_double), ("theta", C.c_double), ("w8", C.c_uint32),
                          ("layer_count", C.c_uint32), ("layer_kinds", C.POINTER(C.c_uint8))]


class NamedWeight(C.Structure):
    _fields_ = [("name", C.c_char_p), ("data", C.c_void_p), ("scales", C.c_void_p)]


class StepResult_C(C.Structure):
    _fields_ = [("past", C.c_uint64), ("logit_rows", C.c_uint64), ("scratch_bytes", C.c_uint64),
                ("dispatch_count", C.c_size_t)]


LOGITS = {"none": 0, "last": 1, "all": 2}   # LogitsMode (Qwen35ModelBuilder.h:10)


def c_config(c: Qwen35Config, w8: bool):
    """The C config of c, and the layer-kind array it points to (keep both)."""
    kinds = (C.c_uint8 * len(c.layers))(*[1 if k == "gqa" else 0 for k in c.layers])
    cfg = Qwen35Config_C(c.hidden, c.intermediate, c.vocabulary, c.max_positions, c.head_dim,
                         c.q_heads, c.kv_heads, c.rotary_width, c.key_heads, c.value_heads,
                         c.key_dim, c.value_dim, c.conv_kernel, c.epsilon, c.theta, int(w8),
                         len(c.layers), kinds)
    return cfg, kinds


class ModelSession:
    """One sequence through the Qwen3.5 graph: a binding of the C++ model
    session (llmi_hip_model_*, csrc/model.cpp), which plays MetalSession
    (MetalSession.h:26-50, MetalExecutor.mm:212-298): it owns the per-layer
    states, builds and lowers each step's graph and runs it with one host
    sync. The weights stay owned here (the session borrows their device
    pointers). Calls on one session must be serialised."""

    def __init__(self, config: Qwen35Config, weights: dict, capacity: int, w8: bool = True,
                 device=None):
        lib = _lib.load()
        self.config, self.w8, self.capacity = config, w8, capacity
        self.device = torch.device(device) if device is not None else torch.device("cuda", 0)
        self.weights = weights
        names = sorted(weights)
        self._names = [n.encode() for n in names]
        table = (NamedWeight * max(1, len(names)))(
            *[NamedWeight(self._names[i], weights[n][0].data_ptr(),
                          weights[n][1].data_ptr() if weights[n][1] is not None else None)
              for i, n in enumerate(names)])
        self._cfg, self._kinds = c_config(config, w8)
        h = C.c_void_p()
        rc = lib.llmi_hip_model_open(C.byref(self._cfg), table, len(names), capacity,
                                     torch.cuda.current_stream(self.device).cuda_stream,
                                     C.byref(h))
        if rc != _lib.OK:
            msg = lib.llmi_hip_last_error().decode()
            raise (ValueError if rc == _lib.INVALID_ARGUMENT else _lib.HipError)(
                *((msg,) if rc == _lib.INVALID_ARGUMENT else (rc, msg)))
        self._h = h
        self.vocabulary = lib.llmi_hip_model_vocabulary(h)

    @property
    def past(self) -> int:
        return _lib.load().llmi_hip_model_past(self._h)

    @property
    def invalid(self) -> bool:
        return bool(_lib.load().llmi_hip_model_invalid(self._h))

    @property
    def states(self) -> list[torch.Tensor]:
        """Copies of the session's state buffers, in graph order."""
        lib = _lib.load()
        out = []
        for i in range(lib.llmi_hip_model_state_count(self._h)):
            d, n = GraphState(), C.c_size_t()
            _check(lib.llmi_hip_model_state(self._h, i, C.byref(d), None, C.byref(n)), "state")
            dtype = torch.float32 if d.element == Element.F32 else torch.float16
            t = torch.empty(tuple(d.shape[:d.rank]), dtype=dtype, device=self.device)
            _check(lib.llmi_hip_model_read_state(self._h, i, t.data_ptr(), n.value), "state")
            out.append(t)
        return out

    def plan(self, tokens: int, logits: str = "last", past: int | None = None) -> Plan:
        """The lowered step of `tokens` rows at `past` (default: the session's)."""
        h = C.c_void_p()
        _check(_lib.load().llmi_hip_model_plan(self._h, tokens, self.past if past is None
                                               else past, LOGITS[logits], C.byref(h)),
               "model plan")
        return Plan(None, handle=h)

    def run(self, plan: Plan, ids: torch.Tensor, logits: torch.Tensor | None) -> None:
        """Enqueues one lowered step (no sync, no checks, past unchanged): for timing."""
        _check(_lib.load().llmi_hip_model_run(self._h, plan._h, ids.data_ptr(),
                                              None if logits is None else logits.data_ptr()),
               "model run")

    def step(self, ids, logits: str = "last", trace: bool = False) -> StepResult:
        lib = _lib.load()
        ids = np.ascontiguousarray(np.asarray(ids, np.int64).reshape(-1))
        if ids.size and (ids.min() < 0 or ids.max() >= 2 ** 32):
            raise ValueError("Token ID is outside the vocabulary")
        ids = ids.astype(np.uint32)
        rows = 0 if logits == "none" else (ids.size if logits == "all" else 1)
        out = np.empty((rows, self.vocabulary), np.float32)
        res = StepResult_C()
        rc = lib.llmi_hip_model_step(self._h, ids.ctypes.data, ids.size, LOGITS[logits],
                                     out.ctypes.data if rows else None, out.size,
                                     C.byref(res))
        if rc != _lib.OK:
            msg = lib.llmi_hip_last_error().decode()
            if rc == _lib.INVALID_ARGUMENT and not self.invalid:
                raise ValueError(msg)
            raise RuntimeError(f"{msg} (status {rc})")
        disp = records(lib.llmi_hip_model_dispatches, self._h) if trace else []
        return StepResult(res.past, res.logit_rows, res.scratch_bytes, res.dispatch_count,
                          out if rows else None, disp)

    def reset(self) -> None:
        _lib.load().llmi_hip_model_reset(self._h)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value and _lib is not None and _lib._lib is not None:
            _lib._lib.llmi_hip_model_close(h)
            self._h = None


__all__ = ["Plan", "ModelSession", "StepResult", "random_weights", "marshal", "OpKind",
           "StateKind"]
