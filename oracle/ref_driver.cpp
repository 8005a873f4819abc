// Test-only harness over the reference's own C++ sources.
//
// Linked (by oracle/Makefile, target `ref`) with the unmodified reference
// files lib/GraphIR/Graph.cpp, lib/GraphIR/Cost.cpp and
// lib/ModelFormat/Quantization.cpp, compiled where they lie under
// /root/reference. The output goes to oracle/_ref/ and is never committed.
// Tests use it to pin the C oracle's fp16 conversion and cost model and the
// HIP backend's host-side op contracts against the reference itself.
#include "llminfer/GraphIR/Cost.h"
#include "llminfer/ModelFormat/Quantization.h"

#include <cstdint>
#include <cstring>

using namespace llminfer;
using namespace llminfer::ir;

namespace {
Shape shapeOf(const uint64_t *dims, int rank) {
  Shape s;
  for (int i = 0; i < rank; ++i)
    s.push_back(dims[i]);
  return s;
}

ElementType elementOf(int code) {
  switch (code) {
  case 0:
    return ElementType::I8;
  case 1:
    return ElementType::U32;
  case 2:
    return ElementType::F16;
  default:
    return ElementType::F32;
  }
}

void copyMessage(const Error &e, char *msg, size_t cap) {
  if (!msg || !cap)
    return;
  std::strncpy(msg, e.getMessage().c_str(), cap - 1);
  msg[cap - 1] = 0;
}
} // namespace

extern "C" {

uint16_t ref_float_to_half(float v) { return floatToHalf(v); }
float ref_half_to_float(uint16_t b) { return halfToFloat(b); }

// Builds a one-layer graph: state slots key/value cache (`cache` dims, F16),
// then KvAppend(k, v) and CausalGqa(q) in the order given by `order`
// (bit 0: append first; bit 1: skip append). Returns a bitmask: bit0 = graph
// created, bit1 = KvAppend accepted, bit2 = CausalGqa accepted. On success of
// both, fills cost[0..5] = {append write bytes, append read bytes, gqa fp
// MACs, gqa read bytes, gqa write bytes, gqa exp count} and
// effects[0..5] = {append begin, append length, append version after,
// gqa begin, gqa length, gqa version before}.
int ref_gqa_graph(uint64_t tokens, uint64_t past, uint64_t capacity,
                  const uint64_t *qdims, const uint64_t *kdims,
                  const uint64_t *vdims, const uint64_t *cachedims,
                  int qelem, int kvelem, int order, uint64_t *cost,
                  uint64_t *effects, char *msg, size_t msgcap) {
  auto graph = Graph::create({tokens, past, capacity});
  if (!graph) {
    copyMessage(graph.getError(), msg, msgcap);
    return 0;
  }
  int mask = 1;
  auto q = graph->addInput({elementOf(qelem), shapeOf(qdims, 3)});
  auto k = graph->addInput({elementOf(kvelem), shapeOf(kdims, 3)});
  auto v = graph->addInput({elementOf(kvelem), shapeOf(vdims, 3)});
  if (!q || !k || !v)
    return mask;
  auto ks = graph->addState(StateKind::KeyCache, 0,
                            {ElementType::F16, shapeOf(cachedims, 3)});
  auto vs = graph->addState(StateKind::ValueCache, 0,
                            {ElementType::F16, shapeOf(cachedims, 3)});
  if (!ks || !vs) {
    copyMessage(!ks ? ks.getError() : vs.getError(), msg, msgcap);
    return mask;
  }
  KvAttr slots{*ks, *vs};
  bool doAppend = !(order & 2);
  if (doAppend) {
    auto r = graph->append(OpKind::KvAppend, {*k, *v}, slots, 0);
    if (r)
      mask |= 2;
    else
      copyMessage(r.getError(), msg, msgcap);
  }
  auto r = graph->append(OpKind::CausalGqa, {*q}, slots, 0);
  if (r)
    mask |= 4;
  else
    copyMessage(r.getError(), msg, msgcap);
  if ((mask & 6) == 6) {
    auto report = estimateCost(*graph);
    if (report) {
      const auto &a = report->perOp[0], &g = report->perOp[1];
      cost[0] = a.logicalWriteBytes;
      cost[1] = a.logicalReadBytes;
      cost[2] = g.fpMacs;
      cost[3] = g.logicalReadBytes;
      cost[4] = g.logicalWriteBytes;
      cost[5] = g.exp;
      const auto &ae = graph->getOps()[0].effects.front();
      const auto &ge = graph->getOps()[1].effects.front();
      effects[0] = ae.begin;
      effects[1] = ae.length;
      effects[2] = ae.versionAfter;
      effects[3] = ge.begin;
      effects[4] = ge.length;
      effects[5] = ge.versionBefore;
    } else {
      copyMessage(report.getError(), msg, msgcap);
      mask |= 8;
    }
  }
  return mask;
}

// One DeltaUpdate op on a recurrent state of `sdims` (element `selem`).
// Operand i has rank ranks[i], dims dims[4*i..], element elems[i].
// Returns 1 if accepted (and fills cost[0..3] = {fp MACs, read bytes,
// write bytes, scalar ops}), 0 if rejected, -1 if the graph itself failed.
int ref_delta_graph(uint64_t tokens, const int *ranks, const uint64_t *dims,
                    const int *elems, const uint64_t *sdims, int selem,
                    uint64_t *cost, char *msg, size_t msgcap) {
  auto graph = Graph::create({tokens, 0, tokens});
  if (!graph) {
    copyMessage(graph.getError(), msg, msgcap);
    return -1;
  }
  ValueId ids[5];
  for (int i = 0; i < 5; ++i) {
    auto v = graph->addInput({elementOf(elems[i]), shapeOf(dims + 4 * i, ranks[i])});
    if (!v) {
      copyMessage(v.getError(), msg, msgcap);
      return -1;
    }
    ids[i] = *v;
  }
  auto s = graph->addState(StateKind::DeltaRecurrent, 0,
                           {elementOf(selem), shapeOf(sdims, 3)});
  if (!s) {
    copyMessage(s.getError(), msg, msgcap);
    return -1;
  }
  auto r = graph->append(OpKind::DeltaUpdate,
                         {ids[0], ids[1], ids[2], ids[3], ids[4]},
                         StateAttr{*s}, 0);
  if (!r) {
    copyMessage(r.getError(), msg, msgcap);
    return 0;
  }
  auto report = estimateCost(*graph);
  if (!report) {
    copyMessage(report.getError(), msg, msgcap);
    return -1;
  }
  const auto &c = report->perOp[0];
  cost[0] = c.fpMacs;
  cost[1] = c.logicalReadBytes;
  cost[2] = c.logicalWriteBytes;
  cost[3] = c.scalarOps;
  return 1;
}
}
