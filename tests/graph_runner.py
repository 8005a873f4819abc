"""Executes a graph (llminfer_amd.graph) op by op, unfused, for checking the
whole-graph plan: on the CPU oracle (backend "oracle": oracle/graph_runner.py)
or through the per-op GPU entry points (backend "gpu": the same kernels the
plan launches, called one op at a time with every projection unfused and
every view copied). Test infrastructure only."""
from __future__ import annotations

import torch

from llminfer_amd import ops
from llminfer_amd.graph import Element, Graph
from oracle.graph_runner import GraphRunner as OracleRunner

_TORCH = {Element.I8: torch.int8, Element.U32: torch.int32, Element.F16: torch.float16,
          Element.F32: torch.float32}


def GraphRunner(g: Graph, weights: dict, states: list, backend: str):
    """weights: tensor id -> (data, scales or None) as numpy arrays (oracle)
    or device tensors (gpu); states: one array per graph state, updated in
    place."""
    if backend == "oracle":
        return OracleRunner(g, weights, states)
    if backend == "gpu":
        return GpuRunner(g, weights, states)
    raise ValueError(f"unknown backend {backend}")


class GpuRunner(OracleRunner):
    """The oracle runner's walk over the graph, each op on its GPU entry point."""

    def window(self, root, shape, strides, offset):
        return root.reshape(-1).as_strided(shape, strides, offset).contiguous()

    def _f16(self, shape):
        return torch.empty(shape, dtype=torch.float16, device="cuda")

    def _f32(self, shape):
        return torch.empty(shape, dtype=torch.float32, device="cuda")

    def _embedding_gather(self, op):
        ids, wv = self.get(op.inputs[0]), self.g.values[op.inputs[1]]
        data, scales = self.w[wv.tensor_id]
        out = self._f16((ids.numel(), wv.shape[1]))
        if scales is not None:
            ops.embedding_w8(ids, data, scales, out)
        else:
            ops.embedding(ids, data, out)
        self.put(op.outputs[0], out)

    def _quantize_activation(self, op):
        x = self.get(op.inputs[0])
        rows, width = x.shape
        groups = (width + 31) // 32
        q = torch.empty(rows, groups * 32, dtype=torch.int8, device="cuda")
        s = self._f32((rows, groups))
        ops.quantize_activation(x, q, s)
        self.put(op.outputs[0], q)
        self.put(op.outputs[1], s)

    def _linear_w8a8(self, op):
        q = self.roots[self._root(op.inputs[0])]
        data, scales = self.w[self.g.values[op.inputs[2]].tensor_id]
        out = self._f16((q.shape[0], data.shape[0]))
        ops.linear_w8a8(q, self.get(op.inputs[1]), data, scales, out)
        self.put(op.outputs[0], out)

    def _linear_f16(self, op):
        x = self.get(op.inputs[0])
        w = self.w[self.g.values[op.inputs[1]].tensor_id][0]
        out = self._f16((x.shape[0], w.shape[0]))
        ops.linear_f16(x, w, out)
        self.put(op.outputs[0], out)

    def _rms_norm(self, op):
        x, w = self.get(op.inputs[0]), self.get(op.inputs[1])
        out = self._f16(tuple(x.shape))
        ops.rms_norm(x, w, out, op.attrs["epsilon"])
        self.put(op.outputs[0], out)

    def _gated_rms_norm(self, op):
        x, gate, w = (self.get(i) for i in op.inputs)
        width = w.shape[0]
        out = self._f16(tuple(x.shape))
        ops.gated_rms_norm(x.reshape(-1, width), gate.reshape(-1, width), w,
                           out.reshape(-1, width), op.attrs["epsilon"])
        self.put(op.outputs[0], out)

    def _l2_norm(self, op):
        x, a = self.get(op.inputs[0]), op.attrs
        out = self._f32(tuple(x.shape))
        ops.l2_norm(x, out, a["group_width"], a["epsilon"], a["scale"])
        self.put(op.outputs[0], out)

    def _binary(self, op, kind):
        a, b = self.get(op.inputs[0]), self.get(op.inputs[1])
        out = self._f16(tuple(a.shape))
        if kind == "sigmoid":
            ops.sigmoid_mul(a, b, out)
        else:
            ops.elementwise(kind, a, b, out)
        self.put(op.outputs[0], out)

    def _silu(self, op):
        x = self.get(op.inputs[0])
        out = self._f16(tuple(x.shape))
        ops.elementwise("silu", x, None, out)
        self.put(op.outputs[0], out)

    def _partial_rope(self, op):
        x, a = self.get(op.inputs[0]), op.attrs
        out = self._f16(tuple(x.shape))
        ops.partial_rope(x, out, self.g.past, a["rotary_width"], a["theta"])
        self.put(op.outputs[0], out)

    def _causal_conv1d(self, op):
        x = self.get(op.inputs[0])
        w = self.w[self.g.values[op.inputs[1]].tensor_id][0]
        C, k = w.shape[0], w.shape[2]
        out = self._f16(tuple(x.shape))
        ops.causal_conv(x, w.reshape(C, k), self.states[op.attrs["state"]], out, False)
        self.put(op.outputs[0], out)

    def _delta_gates(self, op):
        a, b, a_log, dt = (self.get(i) for i in op.inputs)
        beta, decay = self._f32(tuple(a.shape)), self._f32(tuple(a.shape))
        ops.delta_gates(a, b, a_log, dt, beta, decay)
        self.put(op.outputs[0], beta)
        self.put(op.outputs[1], decay)

    def _delta_update(self, op):
        q, k, v, beta, decay = (self.get(i) for i in op.inputs)
        self.put(op.outputs[0], ops.delta_update(q, k, v, beta, decay,
                                                 self.states[op.attrs["state"]]))

    def _kv_append(self, op):
        k, v = self.get(op.inputs[0]), self.get(op.inputs[1])
        kc, vc = self.states[op.attrs["keys"]], self.states[op.attrs["values"]]
        ops.kv_append(k, v, kc, vc, self.g.past)

    def _causal_gqa(self, op):
        kc, vc = self.states[op.attrs["keys"]], self.states[op.attrs["values"]]
        self.put(op.outputs[0], ops.causal_gqa(self.get(op.inputs[0]), kc, vc, self.g.past))
