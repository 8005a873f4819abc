"""The whole-graph HIP plan and a model session over it.

Plan lowers one step's graph (llminfer_amd.graph.Graph) through the C ABI
(llmi_hip_plan_lower, csrc/plan.cpp) and runs it; ModelSession plays the
part of the reference's MetalSession (include/llminfer/Backend/Metal/
MetalSession.h:26-50, MetalExecutor.mm:212-298): it owns the model's
device weights and the per-layer states, builds the Qwen3.5 graph of each
step, lowers and runs it, and returns the logits with the plan records.
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

    def __init__(self, g: Graph, weight_table: list[tuple[int, int]],
                 weight_index: dict[str, int]):
        lib = _lib.load()
        desc, self._keep = marshal(g, weight_index)
        table = (WeightDesc * max(1, len(weight_table)))(
            *[WeightDesc(d, s) for d, s in weight_table])
        self._table = table
        handle = C.c_void_p()
        _check(lib.llmi_hip_plan_lower(C.byref(desc), table, len(weight_table), C.byref(handle)),
               "plan lowering")
        self._h = handle
        self.scratch_bytes = lib.llmi_hip_plan_scratch_bytes(handle)
        rows, elements = C.c_uint64(), C.c_uint64()
        lib.llmi_hip_plan_logits(handle, C.byref(rows), C.byref(elements))
        self.logit_rows, self.logit_elements = rows.value, elements.value
        n = lib.llmi_hip_plan_dispatches(handle, None, 0)
        recs = (_lib.Dispatch * max(1, n))()
        lib.llmi_hip_plan_dispatches(handle, recs, n)
        self.launches = lib.llmi_hip_plan_launches(handle)  # kernel launches a step
        self.dispatches = []  # plan records, one per op a launch serves
        for r in recs[:n]:
            d = {"op_index": r.op_index, "kernel": r.kernel.decode()}
            if r.epilogue:
                d["epilogue"] = r.epilogue.decode()
                d["fused_op_index"] = r.fused_op_index
            self.dispatches.append(d)
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


class ModelSession:
    """One sequence through the Qwen3.5 graph on the HIP plan (MetalSession,
    MetalExecutor.mm:212-298): states persist across steps; every step
    builds the graph of its shape, lowers it and runs it with one host sync.
    Calls on one session must be serialised."""

    def __init__(self, config: Qwen35Config, weights: dict, capacity: int, w8: bool = True,
                 device=None):
        if not capacity or capacity > min(config.max_positions, 2 ** 32 - 1):
            raise ValueError("Invalid session capacity")
        self.config, self.w8, self.capacity = config, w8, capacity
        self.device = torch.device(device) if device is not None else torch.device("cuda", 0)
        names = sorted(weights)
        self.weight_index = {n: i for i, n in enumerate(names)}
        self.weights = weights
        self.weight_table = [(weights[n][0].data_ptr(),
                              weights[n][1].data_ptr() if weights[n][1] is not None else 0)
                             for n in names]
        self.vocabulary = weights[EMBEDDING_ID][0].shape[0]
        layout = build_qwen35(config, 1, 0, capacity, "none", w8)
        self.states = [torch.zeros(s.shape, dtype=_TORCH[s.element], device=self.device)
                       for s in layout.states]
        self._layout = [(s.kind, s.layer, s.shape) for s in layout.states]
        self.scratch = torch.empty(0, dtype=torch.uint8, device=self.device)
        self.invalid_flag = torch.zeros(1, dtype=torch.int32, device=self.device)
        self.past = 0
        self.invalid = False

    def plan(self, tokens: int, logits: str = "last") -> Plan:
        g = build_qwen35(self.config, tokens, self.past, self.capacity, logits, self.w8)
        if [(s.kind, s.layer, s.shape) for s in g.states] != self._layout:
            raise RuntimeError("Graph state layout changed within the session")
        return Plan(g, self.weight_table, self.weight_index)

    def run(self, plan: Plan, ids: torch.Tensor, logits: torch.Tensor | None) -> None:
        """Enqueues one lowered step (no sync, no state checks): for timing."""
        if self.scratch.numel() < plan.scratch_bytes:
            self.scratch = torch.empty(plan.scratch_bytes, dtype=torch.uint8, device=self.device)
        plan.execute(self.scratch, self.states, ids, logits, self.invalid_flag)

    def step(self, ids, logits: str = "last", trace: bool = False) -> StepResult:
        if self.invalid:
            raise RuntimeError("Session is invalid after a failed GPU step")
        ids = np.asarray(ids, np.uint32).reshape(-1)
        if ids.size == 0 or ids.size > self.capacity - self.past:
            raise ValueError("Token chunk is empty or exceeds session capacity")
        if np.any(ids >= self.vocabulary):
            raise ValueError("Token ID is outside the vocabulary")
        plan = self.plan(ids.size, logits)
        dev_ids = torch.from_numpy(ids.view(np.int32)).to(self.device)
        out = None
        if plan.logit_rows:
            out = torch.empty(plan.logit_rows, plan.logit_elements // plan.logit_rows,
                              dtype=torch.float16, device=self.device)
        self.invalid_flag.zero_()
        try:
            self.run(plan, dev_ids, out)
            torch.cuda.synchronize(self.device)
        except Exception:
            self.invalid = True
            raise
        if int(self.invalid_flag.item()):
            self.invalid = True
            raise RuntimeError("Non-finite activation during W8A8 quantization")
        self.past += ids.size
        return StepResult(self.past, plan.logit_rows, plan.scratch_bytes, len(plan.dispatches),
                          out.float().cpu().numpy() if out is not None else None,
                          plan.dispatches if trace else [])

    def reset(self) -> None:
        for s in self.states:
            s.zero_()
        self.past = 0
        self.invalid = False


__all__ = ["Plan", "ModelSession", "StepResult", "random_weights", "marshal", "OpKind",
           "StateKind"]
