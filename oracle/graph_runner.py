"""Executes a graph (llminfer_amd.graph) op by op on the CPU oracle: every
op through its oracle.c function, attention and DeltaUpdate in float64 then
rounded to fp16. TEST INFRASTRUCTURE ONLY: the checker of the whole-graph
plan (tests/) and the timed CPU baseline of the whole-model bench legs; no
product path imports it.

Values are held dense per root (fp16 as uint16 bits); views are strided
windows of their root, copied before use. tests/graph_runner.py derives the
op-by-op GPU executor from this class."""
from __future__ import annotations

import time

import numpy as np

import oracle
from llminfer_amd.graph import Graph, OpKind, ValueKind


class GraphRunner:
    def __init__(self, g: Graph, weights: dict, states: list):
        """weights: tensor id -> (data, scales or None); states: one array
        per graph state, updated in place."""
        self.g, self.w, self.states = g, weights, states
        self.roots: dict[int, object] = {}
        self.op_hook = None   # called as op_hook(index, op, seconds) after each op

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
        return self.window(root, v.shape, v.strides, self._offset(vid))

    def window(self, root, shape, strides, offset):
        flat = root.reshape(-1)
        item = flat.itemsize
        return np.ascontiguousarray(np.lib.stride_tricks.as_strided(
            flat[offset:], shape, [s * item for s in strides]))

    def put(self, vid, array):
        self.roots[vid] = array

    # --------------------------------------------------------------- run
    def run(self, ids):
        """Outputs of the graph for token IDs `ids`."""
        g = self.g
        for vid, v in enumerate(g.values):
            if v.kind == ValueKind.INPUT:
                self.put(vid, ids)
        for i, op in enumerate(g.ops):
            t0 = time.perf_counter()
            getattr(self, "_" + OpKind(op.kind).name.lower())(op)
            if self.op_hook is not None:
                self.op_hook(i, op, time.perf_counter() - t0)
        return [self.get(o) for o in g.outputs]

    def _embedding_gather(self, op):
        ids, wv = self.get(op.inputs[0]), self.g.values[op.inputs[1]]
        data, scales = self.w[wv.tensor_id]
        out = (oracle.embedding_w8(ids, data, scales, wv.shape[1]) if scales is not None
               else oracle.embedding(ids, data))
        self.put(op.outputs[0], out)

    def _quantize_activation(self, op):
        q, s, _ = oracle.quantize_activation(self.get(op.inputs[0]))
        self.put(op.outputs[0], q)
        self.put(op.outputs[1], s)

    def _linear_w8a8(self, op):
        q = self.roots[self._root(op.inputs[0])]
        data, scales = self.w[self.g.values[op.inputs[2]].tensor_id]
        self.put(op.outputs[0], oracle.linear_w8a8(q, self.get(op.inputs[1]), data, scales))

    def _linear_f16(self, op):
        w = self.w[self.g.values[op.inputs[1]].tensor_id][0]
        self.put(op.outputs[0], oracle.linear_f16(self.get(op.inputs[0]), w))

    def _rms_norm(self, op):
        x, w = self.get(op.inputs[0]), self.get(op.inputs[1])
        self.put(op.outputs[0], oracle.rms_norm(x, w, op.attrs["epsilon"]))

    def _gated_rms_norm(self, op):
        x, gate, w = (self.get(i) for i in op.inputs)
        width = w.shape[0]
        self.put(op.outputs[0], oracle.gated_rms_norm(
            x.reshape(-1, width), gate.reshape(-1, width), w,
            op.attrs["epsilon"]).reshape(x.shape))

    def _l2_norm(self, op):
        a = op.attrs
        self.put(op.outputs[0], oracle.l2norm_f32(self.get(op.inputs[0]), a["group_width"],
                                                  a["epsilon"], a["scale"]))

    def _binary(self, op, kind):
        a, b = self.get(op.inputs[0]), self.get(op.inputs[1])
        self.put(op.outputs[0], oracle.sigmoid_mul(a, b) if kind == "sigmoid"
                 else oracle.elementwise(kind, a, b))

    def _add(self, op):
        self._binary(op, "add")

    def _silu_mul(self, op):
        self._binary(op, "swiglu")

    def _sigmoid_mul(self, op):
        self._binary(op, "sigmoid")

    def _silu(self, op):
        self.put(op.outputs[0], oracle.elementwise("silu", self.get(op.inputs[0])))

    def _reshape(self, op):
        pass

    def _slice(self, op):
        pass

    def _partial_rope(self, op):
        a = op.attrs
        self.put(op.outputs[0], oracle.partial_rope(self.get(op.inputs[0]), a["rotary_width"],
                                                    self.g.past, a["theta"]))

    def _causal_conv1d(self, op):
        w = self.w[self.g.values[op.inputs[1]].tensor_id][0]
        C, k = w.shape[0], w.shape[2]
        self.put(op.outputs[0], oracle.causal_conv(self.get(op.inputs[0]), w.reshape(C, k),
                                                   self.states[op.attrs["state"]], False))

    def _delta_gates(self, op):
        beta, decay = oracle.delta_gates(*(self.get(i) for i in op.inputs))
        self.put(op.outputs[0], beta)
        self.put(op.outputs[1], decay)

    def _delta_update(self, op):
        q, k, v, beta, decay = (self.get(i) for i in op.inputs)
        state = self.states[op.attrs["state"]]
        out, st = oracle.delta_recurrent_f64(q, k, v, beta, decay, state)
        state[...] = st.astype(np.float32)
        self.put(op.outputs[0], oracle.f32_to_f16(out.astype(np.float32)))

    def _kv_append(self, op):
        k, v = self.get(op.inputs[0]), self.get(op.inputs[1])
        kc, vc = self.states[op.attrs["keys"]], self.states[op.attrs["values"]]
        past = self.g.past
        kc[past:past + k.shape[0]] = k
        vc[past:past + k.shape[0]] = v

    def _causal_gqa(self, op):
        kc, vc = self.states[op.attrs["keys"]], self.states[op.attrs["values"]]
        self.put(op.outputs[0], oracle.f32_to_f16(
            oracle.gqa_dense_f64(self.get(op.inputs[0]), kc, vc, self.g.past)
            .astype(np.float32)))
