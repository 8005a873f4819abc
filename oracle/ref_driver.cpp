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
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <sstream>
#include <optional>
#include <string>
#include <vector>

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

// Replays a graph program through the reference's Graph::create / addInput /
// addWeight / addState / append and reports what the reference inferred, so
// a builder of the same graph can be compared value by value. The program
// is text, one item a line (floats as C hex floats, ids in order):
//   step T P C
//   input ELEM RANK d...
//   weight ID ELEM GROUP RANK d...
//   state KIND LAYER ELEM RANK d...
//   op KIND LAYER NIN in... ATTR [fields]   (LAYER -1: none)
//      ATTR: none | quant G | norm EPS | l2 W EPS SCALE | reshape RANK d... |
//            slice AXIS BEGIN LENGTH | rope W THETA | state S | kv K V
// The report (into out, at most cap bytes) lists, per value:
//   value KIND ELEM RANK d... s... VIEWOF OFFSET DEFOP GROUP   (-1: none)
// and per op: effects OP N (STATE ACCESS BEGIN LENGTH BEFORE AFTER)...
// A rejected item ends the report with "error INDEX message" (INDEX: the
// op's position, or -1 for a source). Returns 0, or -1 when out is too small.
int ref_graph_replay(const char *program, char *out, size_t cap) {
  std::istringstream in(program);
  std::ostringstream rep;
  std::string line;
  std::optional<Graph> graph;
  auto fail = [&](long index, const Error &e) {
    rep << "error " << index << " " << e.getMessage() << "\n";
  };
  auto readShape = [&](std::istringstream &ls) {
    int rank = 0;
    ls >> rank;
    Shape s;
    for (int i = 0; i < rank; ++i) {
      uint64_t d;
      ls >> d;
      s.push_back(d);
    }
    return s;
  };
  auto readFloat = [&](std::istringstream &ls) {
    std::string t;
    ls >> t;
    return std::strtof(t.c_str(), nullptr);
  };
  long opIndex = 0;
  bool failed = false;
  while (!failed && std::getline(in, line)) {
    std::istringstream ls(line);
    std::string kw;
    if (!(ls >> kw))
      continue;
    if (kw == "step") {
      uint64_t t, p, c;
      ls >> t >> p >> c;
      auto g = Graph::create({t, p, c});
      if (!g) {
        fail(-1, g.getError());
        failed = true;
      } else {
        graph.emplace(std::move(*g));
      }
    } else if (kw == "input") {
      int e;
      ls >> e;
      auto r = graph->addInput({elementOf(e), readShape(ls)});
      if (!r) {
        fail(-1, r.getError());
        failed = true;
      }
    } else if (kw == "weight") {
      std::string id;
      int e;
      uint64_t group;
      ls >> id >> e >> group;
      auto r = graph->addWeight(id, {elementOf(e), readShape(ls)}, group);
      if (!r) {
        fail(-1, r.getError());
        failed = true;
      }
    } else if (kw == "state") {
      int kind, e;
      uint32_t layer;
      ls >> kind >> layer >> e;
      auto r = graph->addState(static_cast<StateKind>(kind), layer,
                               {elementOf(e), readShape(ls)});
      if (!r) {
        fail(-1, r.getError());
        failed = true;
      }
    } else if (kw == "op") {
      int kind, layer, n;
      ls >> kind >> layer >> n;
      std::vector<ValueId> ins;
      for (int i = 0; i < n; ++i) {
        size_t v;
        ls >> v;
        ins.push_back({v});
      }
      std::string attr;
      ls >> attr;
      Attributes a;
      if (attr == "quant") {
        uint64_t g;
        ls >> g;
        a = QuantizeAttr{g};
      } else if (attr == "norm") {
        a = NormAttr{readFloat(ls)};
      } else if (attr == "l2") {
        uint64_t w;
        ls >> w;
        float eps = readFloat(ls), scale = readFloat(ls);
        a = L2NormAttr{w, eps, scale};
      } else if (attr == "reshape") {
        a = ReshapeAttr{readShape(ls)};
      } else if (attr == "slice") {
        size_t axis;
        uint64_t b, l;
        ls >> axis >> b >> l;
        a = SliceAttr{axis, b, l};
      } else if (attr == "rope") {
        uint64_t w;
        ls >> w;
        a = RopeAttr{w, readFloat(ls)};
      } else if (attr == "state") {
        size_t st;
        ls >> st;
        a = StateAttr{{st}};
      } else if (attr == "kv") {
        size_t k, v;
        ls >> k >> v;
        a = KvAttr{{k}, {v}};
      }
      std::optional<uint32_t> lay;
      if (layer >= 0)
        lay = static_cast<uint32_t>(layer);
      Result<Values> r = Error("unsupported operand count");
      switch (n) {
      case 1: r = graph->append(static_cast<OpKind>(kind), {ins[0]}, a, lay); break;
      case 2: r = graph->append(static_cast<OpKind>(kind), {ins[0], ins[1]}, a, lay); break;
      case 3:
        r = graph->append(static_cast<OpKind>(kind), {ins[0], ins[1], ins[2]}, a, lay);
        break;
      case 4:
        r = graph->append(static_cast<OpKind>(kind), {ins[0], ins[1], ins[2], ins[3]}, a, lay);
        break;
      case 5:
        r = graph->append(static_cast<OpKind>(kind), {ins[0], ins[1], ins[2], ins[3], ins[4]},
                          a, lay);
        break;
      default: break;
      }
      if (!r) {
        fail(opIndex, r.getError());
        failed = true;
      }
      ++opIndex;
    }
  }
  if (graph) {
    for (const auto &v : graph->getValues()) {
      rep << "value " << static_cast<int>(v.kind) << " " << static_cast<int>(v.type.element)
          << " " << v.type.shape.size();
      for (auto d : v.type.shape)
        rep << " " << d;
      for (auto d : v.strides)
        rep << " " << d;
      rep << " " << (v.viewOf ? (long)v.viewOf->index : -1L) << " " << v.viewOffset << " "
          << (v.definingOp ? (long)*v.definingOp : -1L) << " " << v.groupSize << "\n";
    }
    size_t i = 0;
    for (const auto &op : graph->getOps()) {
      rep << "effects " << i++ << " " << op.effects.size();
      for (const auto &e : op.effects)
        rep << " " << e.state.index << " " << static_cast<int>(e.access) << " " << e.begin
            << " " << e.length << " " << e.versionBefore << " " << e.versionAfter;
      rep << "\n";
    }
  }
  std::string text = rep.str();
  if (text.size() + 1 > cap)
    return -1;
  std::memcpy(out, text.c_str(), text.size() + 1);
  return 0;
}
}
