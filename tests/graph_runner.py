"""Executes a graph (llminfer_amd.graph) op by op, unfused, for checking the
whole-graph plan: on the CPU oracle (backend "oracle": every op through its
oracle.c function, attention and DeltaUpdate in float64 then fp16), or
through the per-op GPU entry points (backend "gpu": the same kernels the
plan launches, called one op at a time with every projection unfused and
every view copied). Test infrastructure only.

Values are held dense per root (fp16 as uint16 bits on the oracle side);
views are strided windows of their root, copied before use."""
from __future__ import annotations

import numpy as np
import torch

import oracle
from llminfer_amd import ops
from llminfer_amd.graph import Element, Graph, OpKind, ValueKind

_NP = {Element.I8: np.int8, Element.U32: np.uint32, Element.F16: np.uint16,
       Element.F32: np.float32}
_TORCH = {Element.I8: torch.int8, Element.U32: torch.int32, Element.F16: torch.float16,
          Element.F32: torch.float32}


class GraphRunner:
    def __init__(self, g: Graph, weights: dict, states: list, backend: str):
        """weights: tensor id -> (data, scales or None) as numpy arrays
        (oracle) or device tensors (gpu); states: one array per graph state,
        updated in place."""
        self.g, self.w, self.states, self.backend = g, weights, states, backend
        self.roots: dict[int, object] = {}

    # ------------------------------------------------------------ values
    def _root(self, vid):
        v = self.g.values[vid]
        while v.view_of is not None:
            vid = v.view_of
            v = self.g.values[vid]
        return vid

    def _offset(self, vid):
        off, v = 0, self.g.values[vid]
        while v.view_of is not None:
            off += v.view_offset
            vid = v.view_of
            v = self.g.values[vid]
        return off

    def get(self, vid):
        """The value as a dense array of its shape (a copy for views)."""
        v = self.g.values[vid]
        if v.kind == ValueKind.WEIGHT:
            return self.w[v.tensor_id][0]
        root = self.roots[self._root(vid)]
        if v.kind != ValueKind.VIEW:
            return root
        off = self._offset(vid)
        if self.backend == "oracle":
            flat = root.reshape(-1)
            item = flat.itemsize
            return np.ascontiguousarray(np.lib.stride_tricks.as_strided(
                flat[off:], v.shape, [s * item for s in v.strides]))
        return root.reshape(-1).as_strided(v.shape, v.strides, off).contiguous()

    def put(self, vid, array):
        self.roots[vid] = array

    def _f16(self, shape):
        if self.backend == "oracle":
            return np.zeros(shape, np.uint16)
        return torch.empty(shape, dtype=torch.float16, device="cuda")

    def _f32(self, shape):
        if self.backend == "oracle":
            return np.zeros(shape, np.float32)
        return torch.empty(shape, dtype=torch.float32, device="cuda")

    # --------------------------------------------------------------- run
    def run(self, ids):
        g = self.g
        for vid, v in enumerate(g.values):
            if v.kind == ValueKind.INPUT:
                self.put(vid, ids)
        for op in g.ops:
            getattr(self, "_" + OpKind(op.kind).name.lower())(op)
        return [self.get(o) for o in g.outputs]

    def _embedding_gather(self, op):
        ids, wv = self.get(op.inputs[0]), self.g.values[op.inputs[1]]
        data, scales = self.w[wv.tensor_id]
        hidden = wv.shape[1]
        if self.backend == "oracle":
            out = (oracle.embedding_w8(ids, data, scales, hidden) if scales is not None
                   else oracle.embedding(ids, data))
        else:
            out = self._f16((ids.numel(), hidden))
            if scales is not None:
                ops.embedding_w8(ids, data, scales, out)
            else:
                ops.embedding(ids, data, out)
        self.put(op.outputs[0], out)

    def _quantize_activation(self, op):
        x = self.get(op.inputs[0])
        rows, width = x.shape
        groups = (width + 31) // 32
        if self.backend == "oracle":
            q, s, _ = oracle.quantize_activation(x)
        else:
            q = torch.empty(rows, groups * 32, dtype=torch.int8, device="cuda")
            s = self._f32((rows, groups))
            ops.quantize_activation(x, q, s)
        self.put(op.outputs[0], q)
        self.put(op.outputs[1], s)

    def _linear_w8a8(self, op):
        q = self.roots[self._root(op.inputs[0])]
        s = self.get(op.inputs[1])
        data, scales = self.w[self.g.values[op.inputs[2]].tensor_id]
        if self.backend == "oracle":
            out = oracle.linear_w8a8(q, s, data, scales)
        else:
            out = self._f16((q.shape[0], data.shape[0]))
            ops.linear_w8a8(q, s, data, scales, out)
        self.put(op.outputs[0], out)

    def _linear_f16(self, op):
        x = self.get(op.inputs[0])
        w = self.w[self.g.values[op.inputs[1]].tensor_id][0]
        if self.backend == "oracle":
            out = oracle.linear_f16(x, w)
        else:
            out = self._f16((x.shape[0], w.shape[0]))
            ops.linear_f16(x, w, out)
        self.put(op.outputs[0], out)

    def _rms_norm(self, op):
        x, w = self.get(op.inputs[0]), self.get(op.inputs[1])
        eps = op.attrs["epsilon"]
        if self.backend == "oracle":
            out = oracle.rms_norm(x, w, eps)
        else:
            out = self._f16(tuple(x.shape))
            ops.rms_norm(x, w, out, eps)
        self.put(op.outputs[0], out)

    def _gated_rms_norm(self, op):
        x, gate, w = (self.get(i) for i in op.inputs)
        width, eps = w.shape[0], op.attrs["epsilon"]
        if self.backend == "oracle":
            out = oracle.gated_rms_norm(x.reshape(-1, width), gate.reshape(-1, width), w,
                                        eps).reshape(x.shape)
        else:
            out = self._f16(tuple(x.shape))
            ops.gated_rms_norm(x.reshape(-1, width), gate.reshape(-1, width), w,
                               out.reshape(-1, width), eps)
        self.put(op.outputs[0], out)

    def _l2_norm(self, op):
        x, a = self.get(op.inputs[0]), op.attrs
        if self.backend == "oracle":
            out = oracle.l2norm_f32(x, a["group_width"], a["epsilon"], a["scale"])
        else:
            out = self._f32(tuple(x.shape))
            ops.l2_norm(x, out, a["group_width"], a["epsilon"], a["scale"])
        self.put(op.outputs[0], out)

    def _binary(self, op, kind):
        a, b = self.get(op.inputs[0]), self.get(op.inputs[1])
        if self.backend == "oracle":
            out = oracle.sigmoid_mul(a, b) if kind == "sigmoid" else \
                oracle.elementwise(kind, a, b)
        else:
            out = self._f16(tuple(a.shape))
            if kind == "sigmoid":
                ops.sigmoid_mul(a, b, out)
            else:
                ops.elementwise(kind, a, b, out)
        self.put(op.outputs[0], out)

    def _add(self, op):
        self._binary(op, "add")

    def _silu_mul(self, op):
        self._binary(op, "swiglu")

    def _sigmoid_mul(self, op):
        self._binary(op, "sigmoid")

    def _silu(self, op):
        x = self.get(op.inputs[0])
        if self.backend == "oracle":
            out = oracle.elementwise("silu", x)
        else:
            out = self._f16(tuple(x.shape))
            ops.elementwise("silu", x, None, out)
        self.put(op.outputs[0], out)

    def _reshape(self, op):
        pass

    def _slice(self, op):
        pass

    def _partial_rope(self, op):
        x, a = self.get(op.inputs[0]), op.attrs
        if self.backend == "oracle":
            out = oracle.partial_rope(x, a["rotary_width"], self.g.past, a["theta"])
        else:
            out = self._f16(tuple(x.shape))
            ops.partial_rope(x, out, self.g.past, a["rotary_width"], a["theta"])
        self.put(op.outputs[0], out)

    def _causal_conv1d(self, op):
        x = self.get(op.inputs[0])
        w = self.w[self.g.values[op.inputs[1]].tensor_id][0]
        history = self.states[op.attrs["state"]]
        C, k = w.shape[0], w.shape[2]
        if self.backend == "oracle":
            out = oracle.causal_conv(x, w.reshape(C, k), history, False)
        else:
            out = self._f16(tuple(x.shape))
            ops.causal_conv(x, w.reshape(C, k), history, out, False)
        self.put(op.outputs[0], out)

    def _delta_gates(self, op):
        a, b, a_log, dt = (self.get(i) for i in op.inputs)
        if self.backend == "oracle":
            beta, decay = oracle.delta_gates(a, b, a_log, dt)
        else:
            beta, decay = self._f32(tuple(a.shape)), self._f32(tuple(a.shape))
            ops.delta_gates(a, b, a_log, dt, beta, decay)
        self.put(op.outputs[0], beta)
        self.put(op.outputs[1], decay)

    def _delta_update(self, op):
        q, k, v, beta, decay = (self.get(i) for i in op.inputs)
        state = self.states[op.attrs["state"]]
        if self.backend == "oracle":
            out, st = oracle.delta_recurrent_f64(q, k, v, beta, decay, state)
            state[...] = st.astype(np.float32)
            out = oracle.f32_to_f16(out.astype(np.float32))
        else:
            out = ops.delta_update(q, k, v, beta, decay, state)
        self.put(op.outputs[0], out)

    def _kv_append(self, op):
        k, v = self.get(op.inputs[0]), self.get(op.inputs[1])
        kc, vc = self.states[op.attrs["keys"]], self.states[op.attrs["values"]]
        T, past = k.shape[0], self.g.past
        if self.backend == "oracle":
            kc[past:past + T] = k
            vc[past:past + T] = v
        else:
            ops.kv_append(k, v, kc, vc, past)

    def _causal_gqa(self, op):
        q = self.get(op.inputs[0])
        kc, vc = self.states[op.attrs["keys"]], self.states[op.attrs["values"]]
        if self.backend == "oracle":
            out = oracle.f32_to_f16(oracle.gqa_dense_f64(q, kc, vc, self.g.past).astype(
                np.float32))
        else:
            out = ops.causal_gqa(q, kc, vc, self.g.past)
        self.put(op.outputs[0], out)
