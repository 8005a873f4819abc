// The whole-graph plan: one step's GraphIR graph lowered to HIP dispatches
// over the per-op C ABI (capi.cpp), then run on a stream.
//
// Replaces MetalExecutionPlan (lib/Backend/Metal/MetalExecutionPlan.cpp:
// 169-760). What the reference's tooling observes is kept: which projection
// epilogue fuses into which consumer (prepareFusions, :313-403), the order
// of the launches, and one record per launch with op index, kernel,
// epilogue and fused op. The storage is MI355X-side: every result lives in
// one device arena (the reference binds a Metal buffer per scratch slot),
// placed first-fit between its defining op and its last use, offsets fixed
// at lowering so a run is pointer arithmetic and launches; contiguous views
// are addressed in place (the reference copies any view with an offset),
// non-contiguous fp16 views go through copyHalfView.
#include "capi_internal.hpp"
#include "kernels.hpp"
#include "llminfer_hip.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <cstring>
#include <string>
#include <vector>

namespace llmi {
namespace {

constexpr uint64_t kAlign = 256;

enum class Space : uint8_t { None, Scratch, Weight, Scale, State, Input, Output, Invalid };

// A device address resolved at run time: the base of `space` (entry `index`
// of the weight or state table) plus `offset` bytes.
struct Ref {
  Space space = Space::None;
  uint32_t index = 0;
  uint64_t offset = 0;
};

enum class Launch : uint8_t {
  Embedding, EmbeddingW8, Quantize, LinearW8, LinearF16, RmsNorm, GatedRmsNorm,
  GatedRmsNormActivated, L2Norm, Elementwise, SigmoidMul, PartialRope, CausalConv, DeltaGates,
  DeltaUpdate, KvAppend, CausalGqa, CopyView, AddNormQuantize, AddNormLinear, L2DeltaUpdate,
  GatedNormQuantize, KvAppendGqa, GatedAttention, L2DeltaNormQuantize
};

// One plan record of a launch that serves several ops.
struct Rec {
  size_t op;
  const char *epilogue;
  size_t fused;
};

struct Dispatch {
  Launch launch;
  ElementwiseKind elementwise = ElementwiseKind::Add;
  Ref buf[12];
  uint64_t workspaceBytes = 0;
  union {
    EmbedParams embed;
    GroupedEmbedParams embedW8;
    QuantizeParams quantize;
    LinearW8Params linearW8;
    LinearParams linear;
    RowParams row;
    L2Params l2;
    ElementParams element;
    PartialRopeParams rope;
    ConvParams conv;
    GraphDeltaParams delta;
    CacheParams cache;
    GqaParams gqa;
    HalfViewParams view;
    NormLinearParams normLinear;
  } p;
  size_t opIndex = 0, fusedOpIndex = 0;
  const char *epilogue = nullptr;
  std::vector<const char *> kernels;
  std::vector<size_t> ops; // a launch serving several ops: a record for each
  std::vector<Rec> recs;   // ... with their epilogues (replaces ops when set)
  // L2DeltaUpdate: the q / k norms; L2DeltaNormQuantize: also the gated
  // norm's epsilon
  float epsilon = 0.0f, scale = 0.0f, normEpsilon = 0.0f;
  // GatedAttention: the rotation of both normRopes, and whether the gate
  // values are already activated
  unsigned rotary = 0;
  float theta = 0.0f;
  bool activated = false;
  // AddNormLinear: weight, scales, output, aux, bias, and the convolution
  // weight and history of a projection with the convolution epilogue
  Ref proj[kNormLinearMax][7];
};

struct Fusion {
  unsigned kind = LLMI_LINEAR_NONE;
  size_t consumer = 0;
  unsigned block = 0;
  // Run at the consumer: the epilogue needs the consumer's other operands,
  // or the consumer's output is the projection's (MetalExecutionPlan.cpp:
  // 60-68).
  bool deferred() const {
    return kind == LLMI_LINEAR_SILU || kind == LLMI_LINEAR_SILU_MUL ||
           kind == LLMI_LINEAR_DELTA_BETA || kind == LLMI_LINEAR_DELTA_DECAY;
  }
};

const char *epilogue_name(unsigned kind) {
  switch (kind) {
  case LLMI_LINEAR_SILU:
  case LLMI_LINEAR_SILU_F32:
    return "silu";
  case LLMI_LINEAR_SILU_MUL:
    return "swiglu";
  case LLMI_LINEAR_SIGMOID_COLUMNS:
  case LLMI_LINEAR_DELTA_BETA:
    return "sigmoid";
  case LLMI_LINEAR_DELTA_DECAY:
    return "softplus_decay";
  default:
    return nullptr;
  }
}

uint64_t element_bytes(uint32_t e) {
  return e == LLMI_GRAPH_I8 ? 1 : e == LLMI_GRAPH_F16 ? 2 : 4;
}

} // namespace
} // namespace llmi

struct llmi_hip_plan {
  std::vector<llmi::Dispatch> dispatches;
  std::vector<llmi_hip_dispatch> records;
  std::vector<llmi_weight> weights;
  uint64_t scratchBytes = 0;
  uint64_t logitRows = 0, logitElements = 0;
  uint64_t invalidOffset = 0;
  size_t stateCount = 0;
  bool hasOutput = false;
};

namespace llmi {
namespace {

// First-fit ranges of one arena; a range is free again once the op index
// passes its last use.
class Arena {
public:
  uint64_t allocate(uint64_t bytes, size_t lastUse) {
    bytes = (std::max<uint64_t>(bytes, 1) + kAlign - 1) / kAlign * kAlign;
    for (size_t i = 0; i < free_.size(); ++i) {
      auto &f = free_[i];
      if (f.second - f.first >= bytes) {
        uint64_t at = f.first;
        f.first += bytes;
        if (f.first == f.second)
          free_.erase(free_.begin() + i);
        live_.push_back({at, bytes, lastUse});
        return at;
      }
    }
    uint64_t at = end_;
    if (!free_.empty() && free_.back().second == end_) { // grow the trailing gap
      at = free_.back().first;
      free_.pop_back();
    }
    end_ = at + bytes;
    live_.push_back({at, bytes, lastUse});
    return at;
  }

  // Releases every range whose last use is before op `index`.
  void release_before(size_t index) {
    for (size_t i = 0; i < live_.size();) {
      if (live_[i].lastUse < index) {
        insert_free(live_[i].at, live_[i].at + live_[i].bytes);
        live_[i] = live_.back();
        live_.pop_back();
      } else {
        ++i;
      }
    }
  }

  uint64_t size() const { return end_; }

private:
  struct Live {
    uint64_t at, bytes;
    size_t lastUse;
  };
  void insert_free(uint64_t b, uint64_t e) {
    auto it = std::lower_bound(free_.begin(), free_.end(), std::make_pair(b, e));
    it = free_.insert(it, {b, e});
    size_t i = it - free_.begin();
    if (i + 1 < free_.size() && free_[i].second == free_[i + 1].first) {
      free_[i].second = free_[i + 1].second;
      free_.erase(free_.begin() + i + 1);
    }
    if (i > 0 && free_[i - 1].second == free_[i].first) {
      free_[i - 1].second = free_[i].second;
      free_.erase(free_.begin() + i);
    }
  }
  std::vector<std::pair<uint64_t, uint64_t>> free_;
  std::vector<Live> live_;
  uint64_t end_ = 0;
};

class Lowering {
public:
  Lowering(const llmi_graph &g, size_t weightCount, llmi_hip_plan &plan)
      : g_(g), weightCount_(weightCount), plan_(plan) {}

  int run();

private:
  const llmi_graph_value &value(uint32_t id) const { return g_.values[id]; }
  uint64_t count(uint32_t id) const {
    uint64_t n = 1;
    for (uint32_t i = 0; i < value(id).rank; ++i)
      n *= value(id).shape[i];
    return n;
  }
  uint64_t dim(uint32_t id, int axis) const {
    const auto &v = value(id);
    return v.shape[axis < 0 ? v.rank + axis : axis];
  }
  bool contiguous(uint32_t id) const {
    const auto &v = value(id);
    uint64_t stride = 1;
    for (uint32_t i = v.rank; i-- > 0;) {
      if (v.shape[i] > 1 && v.strides[i] != stride)
        return false;
      stride *= v.shape[i];
    }
    return true;
  }
  const llmi_graph_op &op(size_t i) const { return g_.ops[i]; }

  int validate();
  void prepare_values();
  void prepare_fusions();
  void prepare_norm_quantize();
  void merge_norm_linears();
  // A one-row step's DeltaGates projections launch at their own ops.
  bool early_gates(size_t producer) const {
    const unsigned k = fusion_[producer].kind;
    return g_.tokens == 1 && (k == LLMI_LINEAR_DELTA_DECAY || k == LLMI_LINEAR_DELTA_BETA);
  }
  int lower(size_t index);
  int gated_attention(size_t s);
  int dense(uint32_t id, Ref &out);
  int linear(size_t producer, uint32_t result, int64_t aux, int64_t bias);
  Ref temporary(uint64_t bytes) { return {Space::Scratch, 0, arena_.allocate(bytes, index_)}; }
  Dispatch &emit(Launch launch, const char *kernel) {
    plan_.dispatches.push_back({});
    Dispatch &d = plan_.dispatches.back();
    d.launch = launch;
    d.opIndex = index_;
    if (kernel)
      d.kernels.push_back(kernel);
    return d;
  }

  const llmi_graph &g_;
  size_t weightCount_;
  llmi_hip_plan &plan_;
  Arena arena_;
  size_t index_ = 0;
  std::vector<size_t> root_, lastUse_;
  std::vector<uint64_t> offset_; // element offset of a view in its root
  std::vector<Ref> buffer_;      // of roots
  std::vector<Fusion> fusion_;
  std::vector<unsigned> uses_;   // non-view uses of each root
  std::vector<int64_t> normQuantize_, normAdd_; // by RmsNorm op: the fused ops
  std::vector<char> skip_;       // launched by a fused launch at another op
  std::vector<std::pair<int64_t, int64_t>> l2Delta_; // by DeltaUpdate op: its q / k L2Norms
  std::vector<int64_t> convSilu_; // by CausalConv1d op: the SiLU launched with it
  // By SigmoidMul op of a one-row step: the attention block launched with
  // it -- q norm, k norm, q rope, k rope, KvAppend, CausalGqa.
  std::vector<std::array<int64_t, 6>> gated_;
  std::vector<char> inGated_; // launched by a gated block's call; its outputs are never stored
  void prepare_l2_delta();
  bool merge_delta_norm(Dispatch &u, const Dispatch &n) const;
  void prepare_kv_decode();
  void prepare_conv_silu();
  void keep_norm_operands(int64_t projection, size_t until);
  void prepare_gated_attention();
};

int Lowering::validate() {
  if (!g_.values || !g_.ops || (g_.state_count && !g_.states) ||
      (g_.output_count && !g_.outputs))
    return fail(LLMI_HIP_INVALID_ARGUMENT, "plan: null graph array");
  if (!g_.tokens || g_.past > g_.capacity || g_.tokens > g_.capacity - g_.past ||
      g_.capacity > UINT32_MAX)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "plan: invalid step (tokens %llu, past %llu, "
                "capacity %llu)", (unsigned long long)g_.tokens,
                (unsigned long long)g_.past, (unsigned long long)g_.capacity);
  for (size_t i = 0; i < g_.value_count; ++i) {
    const auto &v = g_.values[i];
    if (v.rank == 0 || v.rank > LLMI_GRAPH_MAX_RANK || v.element > LLMI_GRAPH_F32 ||
        v.kind > LLMI_GRAPH_VIEW)
      return fail(LLMI_HIP_INVALID_ARGUMENT, "plan: value %zu is malformed", i);
    if (v.kind == LLMI_GRAPH_VIEW &&
        (v.view_of < 0 || (uint64_t)v.view_of >= i))
      return fail(LLMI_HIP_INVALID_ARGUMENT, "plan: view %zu has no preceding base", i);
    if (v.kind == LLMI_GRAPH_WEIGHT && (v.weight < 0 || (uint64_t)v.weight >= weightCount_))
      return fail(LLMI_HIP_INVALID_ARGUMENT, "plan: weight value %zu has no tensor", i);
    if (v.kind == LLMI_GRAPH_RESULT &&
        (v.defining_op < 0 || (uint64_t)v.defining_op >= g_.op_count))
      return fail(LLMI_HIP_INVALID_ARGUMENT, "plan: result %zu has no defining op", i);
    uint64_t span = 1;
    for (uint32_t d = 0; d < v.rank; ++d) {
      if (v.shape[d] == 0 || v.shape[d] > UINT32_MAX)
        return fail(LLMI_HIP_INVALID_ARGUMENT, "plan: value %zu has an extent out of range", i);
      span += (v.shape[d] - 1) * v.strides[d];
    }
    if (span + v.view_offset > UINT32_MAX)
      return fail(LLMI_HIP_INVALID_ARGUMENT,
                  "plan: value %zu exceeds the 32-bit index range", i);
  }
  for (size_t i = 0; i < g_.op_count; ++i) {
    const auto &o = g_.ops[i];
    if (o.kind > LLMI_GRAPH_CAUSAL_GQA || o.input_count > 5 || o.output_count > 2)
      return fail(LLMI_HIP_INVALID_ARGUMENT, "plan: op %zu is malformed", i);
    for (uint32_t j = 0; j < o.input_count; ++j)
      if (o.inputs[j] >= g_.value_count)
        return fail(LLMI_HIP_INVALID_ARGUMENT, "plan: op %zu reads a missing value", i);
    for (uint32_t j = 0; j < o.output_count; ++j)
      if (o.outputs[j] >= g_.value_count || g_.values[o.outputs[j]].defining_op != (int64_t)i)
        return fail(LLMI_HIP_INVALID_ARGUMENT, "plan: op %zu has a foreign output", i);
    const bool stateful = o.kind == LLMI_GRAPH_CAUSAL_CONV1D ||
                          o.kind == LLMI_GRAPH_DELTA_UPDATE;
    const bool cache = o.kind == LLMI_GRAPH_KV_APPEND || o.kind == LLMI_GRAPH_CAUSAL_GQA;
    if ((stateful && o.state >= g_.state_count) ||
        (cache && (o.keys >= g_.state_count || o.values >= g_.state_count)))
      return fail(LLMI_HIP_INVALID_ARGUMENT, "plan: op %zu names a missing state", i);
  }
  for (size_t i = 0; i < g_.output_count; ++i)
    if (g_.outputs[i] >= g_.value_count)
      return fail(LLMI_HIP_INVALID_ARGUMENT, "plan: output %zu is missing", i);
  return LLMI_HIP_OK;
}

// Roots, view offsets and last uses (MetalExecutionPlan.cpp:255-311).
void Lowering::prepare_values() {
  const size_t n = g_.value_count;
  root_.resize(n);
  offset_.assign(n, 0);
  lastUse_.assign(n, 0);
  buffer_.assign(n, {});
  for (size_t i = 0; i < n; ++i) {
    const auto &v = g_.values[i];
    root_[i] = i;
    if (v.kind == LLMI_GRAPH_VIEW) {
      root_[i] = root_[v.view_of];
      offset_[i] = offset_[v.view_of] + v.view_offset;
    } else if (v.kind == LLMI_GRAPH_WEIGHT) {
      buffer_[i] = {Space::Weight, (uint32_t)v.weight, 0};
    } else if (v.kind == LLMI_GRAPH_INPUT) {
      buffer_[i] = {Space::Input, 0, 0};
    }
  }
  for (size_t i = 0; i < g_.op_count; ++i)
    for (uint32_t j = 0; j < op(i).input_count; ++j)
      lastUse_[root_[op(i).inputs[j]]] = i;
  for (size_t i = 0; i < g_.output_count; ++i)
    lastUse_[root_[g_.outputs[i]]] = g_.op_count;
}

// Projection epilogues fused into their consumer (MetalExecutionPlan.cpp:
// 313-403): a projection whose result has exactly one use by Silu / SiluMul
// (the SiLU and SwiGLU epilogues), by GatedRmsNorm as its gate (the fp32
// SiLU epilogue), the a and b projections of DeltaGates (the decay and beta
// epilogues), and the query / gate projection of SigmoidMul when the gate is
// the second half of every interleaved head (the sigmoid-columns epilogue).
void Lowering::prepare_fusions() {
  const size_t n = g_.value_count;
  std::vector<unsigned> &uses = uses_;
  uses.assign(n, 0);
  std::vector<uint32_t> firstUse(n, 0), secondUse(n, 0);
  auto record = [&](uint32_t id) {
    size_t r = root_[id];
    if (uses[r] == 0)
      firstUse[r] = id;
    else if (uses[r] == 1)
      secondUse[r] = id;
    ++uses[r];
  };
  for (size_t i = 0; i < g_.op_count; ++i)
    if (op(i).kind != LLMI_GRAPH_SLICE && op(i).kind != LLMI_GRAPH_RESHAPE)
      for (uint32_t j = 0; j < op(i).input_count; ++j)
        record(op(i).inputs[j]);
  for (size_t i = 0; i < g_.output_count; ++i)
    record(g_.outputs[i]);

  auto projection = [&](uint32_t id) -> int64_t {
    int64_t p = value(id).defining_op;
    if (p >= 0 && (op(p).kind == LLMI_GRAPH_LINEAR_F16 || op(p).kind == LLMI_GRAPH_LINEAR_W8A8))
      return p;
    return -1;
  };
  auto sole = [&](uint32_t id) -> int64_t { return uses[id] == 1 ? projection(id) : -1; };
  fusion_.assign(g_.op_count, {});
  auto fuse = [&](size_t producer, size_t consumer, unsigned kind, unsigned block) {
    fusion_[producer] = {kind, consumer, block};
    if (fusion_[producer].deferred())
      for (uint32_t j = 0; j < op(producer).input_count; ++j) {
        size_t r = root_[op(producer).inputs[j]];
        lastUse_[r] = std::max(lastUse_[r], consumer);
      }
  };
  for (size_t i = 0; i < g_.op_count; ++i) {
    const auto &o = op(i);
    switch (o.kind) {
    case LLMI_GRAPH_SILU:
    case LLMI_GRAPH_SILU_MUL: {
      int64_t p = sole(o.inputs[0]);
      if (p >= 0)
        fuse(p, i, o.kind == LLMI_GRAPH_SILU ? LLMI_LINEAR_SILU : LLMI_LINEAR_SILU_MUL, 0);
      break;
    }
    case LLMI_GRAPH_GATED_RMS_NORM: {
      int64_t p = sole(o.inputs[1]);
      if (p >= 0)
        fuse(p, i, LLMI_LINEAR_SILU_F32, 0);
      break;
    }
    case LLMI_GRAPH_DELTA_GATES: {
      int64_t a = sole(o.inputs[0]), b = sole(o.inputs[1]);
      if (a >= 0 && b >= 0) {
        fuse(a, i, LLMI_LINEAR_DELTA_DECAY, 0);
        fuse(b, i, LLMI_LINEAR_DELTA_BETA, 0);
      }
      break;
    }
    case LLMI_GRAPH_SIGMOID_MUL: {
      const uint32_t gate = o.inputs[0];
      const size_t root = root_[gate];
      const int64_t p = projection((uint32_t)root);
      const auto &gv = value(gate);
      if (p < 0 || uses[root] != 2 || gv.kind != LLMI_GRAPH_VIEW || gv.defining_op < 0)
        break;
      const uint32_t other = firstUse[root] == gate ? secondUse[root] : firstUse[root];
      const auto &ov = value(other);
      if (other == gate || ov.kind != LLMI_GRAPH_VIEW || ov.view_of != gv.view_of ||
          ov.defining_op < 0)
        break;
      // The packed [tokens, heads, 2 * width] reshape of the projection.
      const uint32_t packed = (uint32_t)gv.view_of;
      const auto &pv = value(packed);
      if (pv.kind != LLMI_GRAPH_VIEW || (size_t)pv.view_of != root || pv.rank != 3 ||
          !contiguous(packed))
        break;
      const auto &gs = op(gv.defining_op), &qs = op(ov.defining_op);
      const uint64_t width = pv.shape[2];
      if (gs.kind == LLMI_GRAPH_SLICE && qs.kind == LLMI_GRAPH_SLICE && gs.axis == 2 &&
          qs.axis == 2 && gs.begin == gs.length && qs.begin == 0 && qs.length == gs.length &&
          width == 2 * gs.length)
        fuse(p, i, LLMI_LINEAR_SIGMOID_COLUMNS, (unsigned)gs.length);
      break;
    }
    default:
      break;
    }
  }
}

// RMSNorm -> QuantizeActivation (the norm's only consumer, the next op),
// with the Add that produced the norm's input when it is the op before:
// one launch (llmi_hip_add_rms_norm_quantize) with the same bits, recorded
// under each op. The Add's operands stay live until the norm's index.
void Lowering::prepare_norm_quantize() {
  const size_t n = g_.op_count;
  normQuantize_.assign(n, -1);
  normAdd_.assign(n, -1);
  skip_.assign(n, 0);
  for (size_t j = 0; j + 1 < n; ++j) {
    const auto &o = op(j), &k = op(j + 1);
    if (o.kind != LLMI_GRAPH_RMS_NORM || k.kind != LLMI_GRAPH_QUANTIZE_ACTIVATION)
      continue;
    const uint32_t normed = o.outputs[0], h = o.inputs[0];
    if (k.inputs[0] != normed || uses_[normed] != 1 || value(normed).kind != LLMI_GRAPH_RESULT ||
        value(k.outputs[0]).group_size != 32 || value(h).element != LLMI_GRAPH_F16 ||
        !contiguous(h) || dim(o.inputs[1], 0) > kAddNormQuantizeMax ||
        dim(h, -1) != dim(o.inputs[1], 0) || fusion_[j].kind != LLMI_LINEAR_NONE)
      continue;
    normQuantize_[j] = (int64_t)j + 1;
    skip_[j + 1] = 1;
    // One row (decode): the projections of the quantized row may join the
    // launch (merge_norm_linears), reading nothing the norm reads is
    // overwritten while they run: its inputs stay live as long as the
    // quantized row.
    const bool oneRow = count(h) == dim(o.inputs[1], 0);
    const size_t until = oneRow ? std::max({j, lastUse_[root_[k.outputs[0]]],
                                            lastUse_[root_[k.outputs[1]]]})
                                : j;
    if (j > 0 && op(j - 1).kind == LLMI_GRAPH_ADD && op(j - 1).outputs[0] == h &&
        value(h).kind == LLMI_GRAPH_RESULT) {
      normAdd_[j] = (int64_t)j - 1;
      skip_[j - 1] = 1;
      for (uint32_t x = 0; x < op(j - 1).input_count; ++x) {
        const size_t r = root_[op(j - 1).inputs[x]];
        lastUse_[r] = std::max(lastUse_[r], until);
      }
    } else {
      lastUse_[root_[h]] = std::max(lastUse_[root_[h]], until);
    }
  }
}

// L2Norm(q) and L2Norm(k) whose only consumer is the DeltaUpdate of a
// one-row step, with nothing launched between them and it, at the shapes
// the fused kernels take (dk 64 or 128, dv a multiple of 16): the update
// normalises the fp16 rows as it loads them (llmi_hip_l2_norm_delta_update,
// the same bits), recorded under each of the three ops.
void Lowering::prepare_l2_delta() {
  // A quantization right after the GatedRmsNorm that produced its input may
  // launch with it (merge_norm_linears): the norm's inputs stay live until
  // the quantization, which writes while the launch reads them.
  for (size_t j = 1; j < g_.op_count; ++j)
    if (op(j).kind == LLMI_GRAPH_QUANTIZE_ACTIVATION && op(j - 1).kind == LLMI_GRAPH_GATED_RMS_NORM &&
        op(j).inputs[0] == op(j - 1).outputs[0])
      for (uint32_t x = 0; x < op(j - 1).input_count; ++x) {
        const size_t r = root_[op(j - 1).inputs[x]];
        lastUse_[r] = std::max(lastUse_[r], j);
      }
  l2Delta_.assign(g_.op_count, {-1, -1});
  if (g_.tokens != 1)
    return;
  for (size_t u = 0; u < g_.op_count; ++u) {
    const auto &o = op(u);
    if (o.kind != LLMI_GRAPH_DELTA_UPDATE)
      continue;
    const int64_t qo = value(o.inputs[0]).defining_op, ko = value(o.inputs[1]).defining_op;
    if (qo < 0 || ko < 0 || op(qo).kind != LLMI_GRAPH_L2_NORM ||
        op(ko).kind != LLMI_GRAPH_L2_NORM || uses_[o.inputs[0]] != 1 ||
        uses_[o.inputs[1]] != 1 || skip_[qo] || skip_[ko])
      continue;
    const auto &qn = op(qo), &kn = op(ko);
    const uint64_t dk = g_.states[o.state].shape[1], dv = g_.states[o.state].shape[2];
    // the shapes the fused update kernels take
    if ((dk != 64 && dk != 128) || dv % 16 != 0)
      continue;
    if (qn.epsilon != kn.epsilon || kn.scale != 1.0f || qn.group_width != dk ||
        kn.group_width != dk || value(qn.inputs[0]).element != LLMI_GRAPH_F16 ||
        value(kn.inputs[0]).element != LLMI_GRAPH_F16 || !contiguous(qn.inputs[0]) ||
        !contiguous(kn.inputs[0]))
      continue;
    bool quiet = true; // nothing launched between the norms and the update
    for (size_t j = (size_t)std::max(qo, ko) + 1; j < u && quiet; ++j) {
      const auto &x = op(j);
      const int64_t a = x.kind == LLMI_GRAPH_DELTA_GATES ? value(x.inputs[0]).defining_op : -1;
      quiet = x.kind == LLMI_GRAPH_RESHAPE || x.kind == LLMI_GRAPH_SLICE ||
              (a >= 0 && early_gates((size_t)a));
    }
    if (!quiet || std::min(qo, ko) + 1 != std::max(qo, ko))
      continue;
    l2Delta_[u] = {qo, ko};
    skip_[qo] = skip_[ko] = 1;
    // With the gated norm of the update's output and its quantization right
    // after, the three may launch as one (merge_delta_norm), which writes
    // the norm's outputs while other workgroups still read the update's
    // operands: those then stay live until the quantization.
    size_t until = u;
    if (u + 2 < g_.op_count && op(u + 1).kind == LLMI_GRAPH_GATED_RMS_NORM &&
        op(u + 1).inputs[0] == o.outputs[0] &&
        op(u + 2).kind == LLMI_GRAPH_QUANTIZE_ACTIVATION &&
        op(u + 2).inputs[0] == op(u + 1).outputs[0])
      until = u + 2;
    for (uint32_t x : {qn.inputs[0], kn.inputs[0], o.inputs[2], o.inputs[3], o.inputs[4]})
      lastUse_[root_[x]] = std::max(lastUse_[root_[x]], until);
  }
}

// A one-row L2DeltaUpdate launch (u) and the activated gated norm +
// quantization launch right after it (n) that reads its output, merged
// into one (llmi_hip_l2_norm_delta_gated_norm_activated_quantize, the same
// bits; the update's output is never stored): taken when nothing else reads
// that output, at the shapes of the one-workgroup-per-head kernel, and when
// no output of the merged launch overlaps what it reads or another output.
// Every op keeps its record.
bool Lowering::merge_delta_norm(Dispatch &u, const Dispatch &n) const {
  if (u.launch != Launch::L2DeltaUpdate || n.launch != Launch::GatedNormQuantize ||
      u.ops.size() != 3 || n.recs.size() != 2)
    return false;
  const GraphDeltaParams &p = u.p.delta;
  const RowParams &r = n.p.row;
  const uint32_t y = op(u.ops[2]).outputs[0];
  if (op(n.recs[0].op).inputs[0] != y || uses_[y] != 1 ||
      value(y).kind != LLMI_GRAPH_RESULT || p.tokens > kRecNormMaxT ||
      (p.keyDim != 64 && p.keyDim != 128) || (p.valueDim != 64 && p.valueDim != 128) ||
      r.rows != p.tokens * p.valueHeads || r.width != p.valueDim)
    return false;
  struct Range {
    Ref r;
    uint64_t bytes;
  };
  auto overlap = [](const Range &a, const Range &b) {
    return a.r.space == b.r.space && a.r.index == b.r.index && a.r.space != Space::None &&
           a.r.offset < b.r.offset + b.bytes && b.r.offset < a.r.offset + a.bytes;
  };
  const uint64_t qk = 2ull * p.tokens * p.keyHeads * p.keyDim,
                 nv = (uint64_t)p.tokens * p.valueHeads * p.valueDim,
                 gates = 4ull * p.tokens * p.valueHeads;
  const Range reads[] = {{u.buf[0], qk},     {u.buf[1], qk},      {u.buf[2], 2 * nv},
                         {u.buf[3], gates},  {u.buf[4], gates},   {n.buf[1], 4 * nv},
                         {n.buf[2], 4ull * p.valueDim}};
  const Range writes[] = {{n.buf[3], 2 * nv}, {n.buf[4], nv}, {n.buf[5], nv / 8},
                          {n.buf[6], 4}};
  for (size_t a = 0; a < 4; ++a) {
    for (const Range &x : reads)
      if (overlap(writes[a], x))
        return false;
    for (size_t b = a + 1; b < 4; ++b)
      if (overlap(writes[a], writes[b]))
        return false;
  }
  u.launch = Launch::L2DeltaNormQuantize;
  // q, k, v, beta, decay and state stay; the update's output gives way to
  // the invalid flag, then the gate, the weight and the norm's outputs.
  u.buf[6] = n.buf[6];
  for (int k = 0; k < 5; ++k)
    u.buf[7 + k] = n.buf[1 + k];
  u.normEpsilon = r.epsilon;
  u.kernels = {"deltaRecurrentNormQuantize"};
  u.recs.clear();
  for (size_t o : u.ops)
    u.recs.push_back({o, nullptr, 0});
  for (const Rec &x : n.recs)
    u.recs.push_back(x);
  u.ops.clear();
  return true;
}

// CausalConv1d -> SiLU (the convolution's only consumer, the next op): the
// convolution kernel applies SiLU to each fp16-rounded output
// (causalConv with applySilu, Reference.metal:137-161), the same bits as
// siluF16 over the stored output, so one launch writes the SiLU's output
// and is recorded under both ops. The convolution's own output is never
// stored.
void Lowering::prepare_conv_silu() {
  convSilu_.assign(g_.op_count, -1);
  for (size_t j = 0; j + 1 < g_.op_count; ++j) {
    const auto &c = op(j), &s = op(j + 1);
    if (c.kind != LLMI_GRAPH_CAUSAL_CONV1D || s.kind != LLMI_GRAPH_SILU || skip_[j] ||
        skip_[j + 1] || fusion_[j + 1].kind != LLMI_LINEAR_NONE)
      continue;
    const uint32_t y = c.outputs[0], z = s.outputs[0];
    if (s.inputs[0] != y || uses_[y] != 1 || value(y).kind != LLMI_GRAPH_RESULT ||
        value(z).kind != LLMI_GRAPH_RESULT || value(y).element != LLMI_GRAPH_F16 ||
        value(z).element != LLMI_GRAPH_F16 || count(y) != count(z))
      continue;
    convSilu_[j] = (int64_t)j + 1;
    skip_[j + 1] = 1;
    // In a one-row step the convolution may run as the epilogue of the
    // projection whose row it reads, inside the norm + projections launch.
    keep_norm_operands(value(c.inputs[0]).defining_op, j);
  }
}

// A launch that the norm + projections call of a one-row step may take
// over (merge_norm_linears: a convolution epilogue) writes at op `until`
// while other workgroups still read the norm's operands and the first one
// writes the norm's quantized row: when projection p reads such a norm's
// quantization, those stay live until `until`, so the arena places nothing
// of that op over them.
void Lowering::keep_norm_operands(int64_t p, size_t until) {
  if (g_.tokens != 1 || p < 0 || op(p).kind != LLMI_GRAPH_LINEAR_W8A8)
    return;
  const int64_t qo = value(op(p).inputs[0]).defining_op;
  if (qo < 1 || normQuantize_[qo - 1] != qo)
    return;
  std::vector<uint32_t> live(op(qo - 1).inputs, op(qo - 1).inputs + op(qo - 1).input_count);
  live.insert(live.end(), op(qo).outputs, op(qo).outputs + op(qo).output_count);
  if (normAdd_[qo - 1] >= 0) {
    const auto &a = op(normAdd_[qo - 1]);
    live.insert(live.end(), a.inputs, a.inputs + a.input_count);
  }
  for (uint32_t x : live)
    lastUse_[root_[x]] = std::max(lastUse_[root_[x]], until);
}

// The attention block of a one-row step (Qwen35ModelBuilder.cpp:175-197) in
// one call (llmi_hip_gated_attention, or its activated form when the q
// projection's epilogue has applied the sigmoid to the gate half): RMSNorm
// and PartialRope of the q half of the projected rows and of the new key,
// KvAppend, CausalGqa and the SigmoidMul with the gate half -- the bits of
// those launches in that order. Each op keeps its record; the
// intermediate values are never stored. Taken only when nothing else is
// launched inside the block, every intermediate has that one consumer, q
// and the gate are the two halves of one [1][Hq][2d] row set, both norms
// share the epsilon and both rotations the width and theta, and the fused
// kernels take the shape. The projected rows stay live until the
// SigmoidMul, where the call is made, so its output never covers them.
void Lowering::prepare_gated_attention() {
  gated_.assign(g_.op_count, {-1, -1, -1, -1, -1, -1});
  inGated_.assign(g_.op_count, 0);
  if (g_.tokens != 1)
    return;
  auto def = [&](uint32_t id) { return value(id).defining_op; };
  auto single = [&](uint32_t id) {
    return value(id).kind == LLMI_GRAPH_RESULT && uses_[id] == 1;
  };
  auto is = [&](int64_t x, uint32_t kind) { return x >= 0 && op((size_t)x).kind == kind; };
  auto f16 = [&](uint32_t id) { return value(id).element == LLMI_GRAPH_F16; };
  for (size_t s = 0; s < g_.op_count; ++s) {
    const auto &sm = op(s);
    if (sm.kind != LLMI_GRAPH_SIGMOID_MUL || skip_[s])
      continue;
    const uint32_t gate = sm.inputs[0], mixed = sm.inputs[1];
    const int64_t j = def(mixed);
    if (!is(j, LLMI_GRAPH_CAUSAL_GQA) || !single(mixed))
      continue;
    const auto &att = op((size_t)j);
    const int64_t rq = def(att.inputs[0]);
    if (!is(rq, LLMI_GRAPH_PARTIAL_ROPE) || !single(att.inputs[0]))
      continue;
    const int64_t nq = def(op((size_t)rq).inputs[0]);
    if (!is(nq, LLMI_GRAPH_RMS_NORM) || !single(op((size_t)rq).inputs[0]))
      continue;
    int64_t a = j - 1;
    while (is(a, LLMI_GRAPH_RESHAPE) || is(a, LLMI_GRAPH_SLICE))
      --a;
    if (!is(a, LLMI_GRAPH_KV_APPEND) || op((size_t)a).keys != att.keys ||
        op((size_t)a).values != att.values)
      continue;
    const auto &app = op((size_t)a);
    const int64_t rk = def(app.inputs[0]);
    if (!is(rk, LLMI_GRAPH_PARTIAL_ROPE) || !single(app.inputs[0]))
      continue;
    const int64_t nk = def(op((size_t)rk).inputs[0]);
    if (!is(nk, LLMI_GRAPH_RMS_NORM) || !single(op((size_t)rk).inputs[0]))
      continue;
    // q and the gate: the halves of one contiguous [1][Hq][2d] row set
    const uint32_t qv = op((size_t)nq).inputs[0];
    const int64_t sq = def(qv), sg = def(gate);
    if (!is(sq, LLMI_GRAPH_SLICE) || !is(sg, LLMI_GRAPH_SLICE))
      continue;
    const auto &slq = op((size_t)sq), &slg = op((size_t)sg);
    const uint32_t qg = slq.inputs[0];
    if (value(qg).rank != 3 || !f16(qg) || !contiguous(qg) || slg.inputs[0] != qg)
      continue;
    const uint64_t D = dim(qg, 2) / 2;
    if (slq.axis != 2 || slg.axis != 2 || slq.begin != 0 || slq.length != D ||
        slg.begin != D || slg.length != D || dim(qg, 2) != 2 * D)
      continue;
    const uint32_t k = op((size_t)nk).inputs[0], v = app.inputs[1];
    if (value(k).rank != 3 || value(v).rank != 3 || !f16(k) || !f16(v) || !contiguous(k) ||
        !contiguous(v) || dim(k, 2) != D || dim(v, 2) != D || dim(v, 1) != dim(k, 1))
      continue;
    const auto &oq = op((size_t)rq), &ok = op((size_t)rk);
    const uint32_t wq = op((size_t)nq).inputs[1], wk = op((size_t)nk).inputs[1];
    if (op((size_t)nq).epsilon != op((size_t)nk).epsilon || oq.rotary_width != ok.rotary_width ||
        oq.theta != ok.theta || oq.rotary_width % 16 != 0 || oq.rotary_width > D ||
        value(wq).element != LLMI_GRAPH_F32 || value(wk).element != LLMI_GRAPH_F32 ||
        count(wq) != D || count(wk) != D)
      continue;
    const auto &cache = g_.states[att.keys].shape;
    GqaParams gp{1, (unsigned)dim(qg, 1), (unsigned)cache[1], (unsigned)cache[2],
                 (unsigned)g_.past};
    if (cache[2] != D || dim(k, 1) != cache[1] ||
        llmi_hip_dispatch_count(LLMI_HIP_OP_GATED_ATTENTION, &gp) == 0)
      continue;
    const std::array<int64_t, 6> blk{nq, nk, rq, rk, a, j};
    bool quiet = true; // nothing else launched inside the block
    for (size_t x = (size_t)std::min(nq, nk); x < s && quiet; ++x)
      quiet = std::find(blk.begin(), blk.end(), (int64_t)x) != blk.end()
                  ? !skip_[x]
                  : op(x).kind == LLMI_GRAPH_RESHAPE || op(x).kind == LLMI_GRAPH_SLICE;
    if (!quiet)
      continue;
    gated_[s] = blk;
    for (int64_t x : blk)
      skip_[(size_t)x] = inGated_[(size_t)x] = 1;
    for (uint32_t x : {qg, k, v})
      lastUse_[root_[x]] = std::max(lastUse_[root_[x]], s);
  }
}

// A one-token KvAppend whose next launched op is the CausalGqa on the same
// caches runs as one fused decode call that reads the new K and V rows while
// the attention writes its output, so the new rows stay live until the
// attention op: its output is then never placed over them.
void Lowering::prepare_kv_decode() {
  if (g_.tokens != 1)
    return;
  for (size_t i = 0; i < g_.op_count; ++i) {
    const auto &a = op(i);
    if (a.kind != LLMI_GRAPH_KV_APPEND)
      continue;
    size_t j = i + 1;
    while (j < g_.op_count &&
           (op(j).kind == LLMI_GRAPH_RESHAPE || op(j).kind == LLMI_GRAPH_SLICE))
      ++j;
    if (j == g_.op_count || op(j).kind != LLMI_GRAPH_CAUSAL_GQA || op(j).keys != a.keys ||
        op(j).values != a.values)
      continue;
    for (uint32_t k = 0; k < 2; ++k)
      lastUse_[root_[a.inputs[k]]] = std::max(lastUse_[root_[a.inputs[k]]], j);
  }
}

// A one-row norm + quantization launch and the W8A8 projections right after
// it that read its quantized row, merged into one launch
// (llmi_hip_add_rms_norm_linear_w8a8) whose weight stream runs under the
// norm's chain: at most kNormLinearMax projections, one round of
// workgroups (one a CU), a SwiGLU projection only right after its
// multiplier's projection (the same lanes compute both), not the logits
// head, and no output overlapping what the launch reads or another output.
// Every op keeps its record.
void Lowering::merge_norm_linears() {
  constexpr unsigned kOneRound = 256;
  auto &ds = plan_.dispatches;
  struct Range {
    Ref r;
    uint64_t bytes;
  };
  auto overlap = [](const Range &a, const Range &b) {
    return a.r.space == b.r.space && a.r.index == b.r.index && a.r.space != Space::None &&
           a.r.offset < b.r.offset + b.bytes && b.r.offset < a.r.offset + a.bytes;
  };
  std::vector<Dispatch> out;
  out.reserve(ds.size());
  for (size_t i = 0; i < ds.size(); ++i) {
    const Dispatch &d = ds[i];
    // A one-token KvAppend and the CausalGqa right after it on the same
    // caches: the fused decode call (llmi_hip_kv_append_causal_gqa), whose
    // attention reads the new rows as it appends them.
    if (d.launch == Launch::KvAppend && i + 1 < ds.size() &&
        ds[i + 1].launch == Launch::CausalGqa) {
      const Dispatch &c = ds[i + 1];
      const GqaParams &gp = c.p.gqa;
      auto same = [](const Ref &a, const Ref &b) {
        return a.space == b.space && a.index == b.index && a.offset == b.offset;
      };
      const uint64_t row = 2ull * d.p.cache.count; // the new K (or V) row, fp16
      const Range ws{c.buf[4], c.workspaceBytes};
      const Range o{c.buf[3], 2ull * gp.queryHeads * gp.headDim};
      const bool clash = overlap(ws, {d.buf[0], row}) || overlap(ws, {d.buf[1], row}) ||
                         overlap(ws, {c.buf[0], 2ull * gp.queryHeads * gp.headDim}) ||
                         overlap(ws, o) || overlap(o, {d.buf[0], row}) ||
                         overlap(o, {d.buf[1], row});
      if (gp.tokens == 1 && same(d.buf[2], c.buf[1]) && same(d.buf[3], c.buf[2]) && !clash &&
          llmi_hip_gqa_workspace_bytes(gp) == c.workspaceBytes &&
          llmi_hip_dispatch_count(LLMI_HIP_OP_KV_APPEND_CAUSAL_GQA, &gp) > 0) {
        Dispatch m = c;
        m.launch = Launch::KvAppendGqa;
        m.opIndex = d.opIndex;
        m.buf[5] = d.buf[0];
        m.buf[6] = d.buf[1];
        m.kernels.clear();
        for (unsigned k = 0; k < llmi_hip_dispatch_count(LLMI_HIP_OP_KV_APPEND_CAUSAL_GQA, &gp);
             ++k)
          m.kernels.push_back(llmi_hip_kernel_name(LLMI_HIP_OP_KV_APPEND_CAUSAL_GQA, &gp, k));
        m.recs = {{d.opIndex, nullptr, 0}, {c.opIndex, nullptr, 0}};
        out.push_back(std::move(m));
        ++i;
        continue;
      }
    }
    // The activated gated norm and the quantization of its output right
    // after it (llmi_hip_gated_rms_norm_activated_quantize).
    if (d.launch == Launch::GatedRmsNormActivated && i + 1 < ds.size() &&
        ds[i + 1].launch == Launch::Quantize) {
      const Dispatch &qd = ds[i + 1];
      const RowParams &nr = d.p.row;
      const QuantizeParams &qp = qd.p.quantize;
      const uint64_t n = (uint64_t)nr.rows * nr.width;
      const Range qr{qd.buf[1], n}, sr{qd.buf[2], n / 8};
      bool clash = false; // with the fp16 input, the fp32 gate, the weight, the fp16 output
      const uint64_t bytes[4] = {2 * n, 4 * n, 4ull * nr.width, 2 * n};
      for (int k = 0; k < 4; ++k)
        clash = clash || overlap(qr, {d.buf[k], bytes[k]}) || overlap(sr, {d.buf[k], bytes[k]});
      if (qd.buf[0].space == d.buf[3].space && qd.buf[0].index == d.buf[3].index &&
          qd.buf[0].offset == d.buf[3].offset && nr.width % 32 == 0 && nr.width <= 256 &&
          (uint64_t)qp.rows * qp.width == n && qp.groups * 32 == qp.width && !clash) {
        Dispatch m = d;
        m.launch = Launch::GatedNormQuantize;
        m.buf[4] = qd.buf[1];
        m.buf[5] = qd.buf[2];
        m.buf[6] = qd.buf[3];
        m.kernels = {"gatedRmsNormQuantize"};
        m.recs = {{d.opIndex, nullptr, 0}, {qd.opIndex, nullptr, 0}};
        if (!out.empty() && merge_delta_norm(out.back(), m)) {
          ++i;
          continue;
        }
        out.push_back(std::move(m));
        ++i;
        continue;
      }
    }
    const RowParams &row = d.p.row;
    if (d.launch != Launch::AddNormQuantize || row.rows != 1 || row.width > kNormLinearMaxWidth) {
      out.push_back(d);
      continue;
    }
    const unsigned groups = (row.width + 31) / 32;
    std::vector<Range> reads = {{d.buf[0], 2ull * row.width}, {d.buf[1], 2ull * row.width},
                                {d.buf[2], 2ull * row.width}, {d.buf[4], 32ull * groups},
                                {d.buf[5], 4ull * groups}};
    NormLinearParams np{};
    np.norm = row;
    unsigned wgs = 0;
    bool lastMate = false;
    size_t j = i + 1;
    for (; j < ds.size() && np.count < kNormLinearMax; ++j) {
      const Dispatch &l = ds[j];
      const LinearW8Params &lp = l.p.linearW8;
      // A SwiGLU projection joins only as the mate of the projection just
      // taken (its multiplier), computed by the same lanes.
      const bool mate = lp.epilogue == LLMI_LINEAR_SILU_MUL && np.count > 0 && !lastMate &&
                        row.width <= kNormLinearPairedWidth &&
                        np.linear[np.count - 1].epilogue == LLMI_LINEAR_NONE &&
                        np.linear[np.count - 1].columns == lp.columns &&
                        l.buf[5].space == ds[j - 1].buf[4].space &&
                        l.buf[5].index == ds[j - 1].buf[4].index &&
                        l.buf[5].offset == ds[j - 1].buf[4].offset;
      const unsigned more = mate ? 0 : norm_linear_workgroups(lp.columns);
      if (l.launch != Launch::LinearW8 || l.buf[0].space != d.buf[4].space ||
          l.buf[0].offset != d.buf[4].offset || l.buf[1].offset != d.buf[5].offset ||
          l.buf[1].space != d.buf[5].space || lp.rows != 1 || lp.groups != groups ||
          (lp.epilogue == LLMI_LINEAR_SILU_MUL && !mate) || l.buf[4].space == Space::Output ||
          wgs + more > kOneRound)
        break; // the logits head keeps its own GEMV launch and record
      const bool f32 = lp.epilogue == LLMI_LINEAR_SILU_F32 ||
                       lp.epilogue == LLMI_LINEAR_DELTA_BETA ||
                       lp.epilogue == LLMI_LINEAR_DELTA_DECAY;
      const Range o{l.buf[4], (uint64_t)lp.outputWidth * (f32 ? 4 : 2)};
      bool clash = false;
      for (const Range &r : reads)
        clash = clash || overlap(o, r);
      if (clash)
        break;
      reads.push_back(o);
      np.linear[np.count] = lp;
      ++np.count;
      wgs += more;
      lastMate = mate;
    }
    if (np.count == 0 || llmi_hip_dispatch_count(LLMI_HIP_OP_ADD_RMS_NORM_LINEAR_W8A8, &np) == 0) {
      out.push_back(d);
      continue;
    }
    Dispatch m;
    m.launch = Launch::AddNormLinear;
    for (int k = 0; k < 7; ++k)
      m.buf[k] = d.buf[k];
    m.p.normLinear = np;
    m.opIndex = d.opIndex;
    m.kernels.push_back(d.buf[1].space != Space::None ? "addRmsNormLinearW8A8"
                                                      : "rmsNormLinearW8A8");
    for (size_t o : d.ops)
      m.recs.push_back({o, nullptr, 0});
    for (unsigned k = 0; k < np.count; ++k) {
      const Dispatch &l = ds[i + 1 + k];
      m.recs.push_back({l.opIndex, l.epilogue, l.fusedOpIndex});
      m.proj[k][0] = l.buf[2];
      m.proj[k][1] = l.buf[3];
      m.proj[k][2] = l.buf[4];
      m.proj[k][3] = l.buf[5];
      m.proj[k][4] = l.buf[6];
    }
    // The one-token convolution with its SiLU right after, over the whole
    // row of a projection that nothing else reads (no epilogue, no SwiGLU
    // multiplier): that projection's convolution epilogue, which stores
    // the convolution's output instead of the row; the convolution's
    // records join.
    size_t taken = np.count;
    if (i + 1 + np.count < ds.size() && ds[i + 1 + np.count].launch == Launch::CausalConv) {
      const Dispatch &c = ds[i + 1 + np.count];
      const ConvParams &cp = c.p.conv;
      for (unsigned k = 0; k < np.count; ++k) {
        const LinearW8Params &lp = np.linear[k];
        const uint32_t y = op(ds[i + 1 + k].opIndex).outputs[0];
        const bool multiplier = k + 1 < np.count &&
                                np.linear[k + 1].epilogue == LLMI_LINEAR_SILU_MUL;
        if (cp.tokens != 1 || cp.kernelSize != 4 || !cp.applySilu ||
            lp.epilogue != LLMI_LINEAR_NONE || lp.firstRow != 0 ||
            lp.columns != lp.outputWidth || cp.channels != lp.columns || multiplier ||
            root_[op(c.opIndex).inputs[0]] != root_[y] || uses_[root_[y]] != 1 ||
            c.buf[0].space != m.proj[k][2].space || c.buf[0].index != m.proj[k][2].index ||
            c.buf[0].offset != m.proj[k][2].offset)
          continue;
        const Range o{c.buf[3], 2ull * lp.columns};
        bool clash = false;
        for (const Range &r : reads)
          clash = clash || overlap(o, r);
        if (clash)
          break;
        m.proj[k][2] = c.buf[3];
        m.proj[k][5] = c.buf[1];
        m.proj[k][6] = c.buf[2];
        if (c.recs.empty())
          m.recs.push_back({c.opIndex, nullptr, 0});
        for (const Rec &x : c.recs)
          m.recs.push_back(x);
        ++taken;
        break;
      }
    }
    out.push_back(std::move(m));
    i += taken;
  }
  ds.swap(out);
}

// The address of a value's elements, materialising a non-contiguous fp16
// view of at most 3 dimensions (MetalExecutionPlan.cpp:405-425).
int Lowering::dense(uint32_t id, Ref &out) {
  const auto &v = value(id);
  Ref base = buffer_[root_[id]];
  if (base.space == Space::None)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "plan: value %u is read before it is written", id);
  if (v.kind != LLMI_GRAPH_VIEW || contiguous(id)) {
    base.offset += offset_[id] * element_bytes(v.element);
    out = base;
    return LLMI_HIP_OK;
  }
  if (v.element != LLMI_GRAPH_F16 || v.rank > 3)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "plan: cannot materialise the view %u", id);
  Dispatch &d = emit(Launch::CopyView, "copyHalfView");
  HalfViewParams &p = d.p.view;
  p.count = (unsigned)count(id);
  p.offset = (unsigned)offset_[id];
  for (int k = 0; k < 3; ++k) {
    p.dims[k] = 1;
    p.strides[k] = 0;
  }
  for (uint32_t k = 0; k < v.rank; ++k) {
    p.dims[3 - v.rank + k] = (unsigned)v.shape[k];
    p.strides[3 - v.rank + k] = (unsigned)v.strides[k];
  }
  d.buf[0] = base;
  out = d.buf[1] = temporary(count(id) * 2);
  return LLMI_HIP_OK;
}

int Lowering::linear(size_t producer, uint32_t result, int64_t aux, int64_t bias) {
  const auto &o = op(producer);
  const Fusion &f = fusion_[producer];
  const bool w8 = o.kind == LLMI_GRAPH_LINEAR_W8A8;
  const uint32_t wid = o.inputs[w8 ? 2 : 1];
  Ref in, scales, weight, outRef, auxRef, biasRef;
  if (int rc = dense(o.inputs[0], in))
    return rc;
  if (w8)
    if (int rc = dense(o.inputs[1], scales))
      return rc;
  if (int rc = dense(wid, weight))
    return rc;
  if (int rc = dense(result, outRef))
    return rc;
  if (aux >= 0)
    if (int rc = dense((uint32_t)aux, auxRef))
      return rc;
  if (bias >= 0)
    if (int rc = dense((uint32_t)bias, biasRef))
      return rc;
  const unsigned rows = (unsigned)dim(result, 0), width = (unsigned)dim(result, 1);
  const unsigned cols = (unsigned)dim(wid, 0);
  Dispatch &d = emit(w8 ? Launch::LinearW8 : Launch::LinearF16, nullptr);
  d.epilogue = epilogue_name(f.kind);
  d.fusedOpIndex = d.epilogue ? (producer == index_ ? f.consumer : producer) : 0;
  d.buf[0] = in;
  d.buf[1] = scales;
  d.buf[2] = weight;
  d.buf[3] = {Space::Scale, weight.index, 0};
  d.buf[4] = outRef;
  d.buf[5] = auxRef;
  d.buf[6] = biasRef;
  if (w8) {
    d.p.linearW8 = {width, 0, (unsigned)dim(o.inputs[1], 1), rows, cols, f.kind, f.block};
    if (llmi_hip_dispatch_count(LLMI_HIP_OP_LINEAR_W8A8, &d.p.linearW8) == 0)
      return fail(LLMI_HIP_INVALID_ARGUMENT, "plan: op %zu: %s", producer, llmi_hip_last_error());
    d.kernels.push_back(llmi_hip_kernel_name(LLMI_HIP_OP_LINEAR_W8A8, &d.p.linearW8, 0));
  } else {
    d.p.linear = {rows, (unsigned)dim(o.inputs[0], 1), width, 0, cols, f.kind, f.block};
    d.kernels.push_back("linearF16");
  }
  return LLMI_HIP_OK;
}

int Lowering::lower(size_t i) {
  const auto &o = op(i);
  const uint32_t *in = o.inputs, *out = o.outputs;
  Ref r[6];
  auto dense_all = [&](std::initializer_list<std::pair<uint32_t, int>> ids) -> int {
    for (auto [id, slot] : ids)
      if (int rc = dense(id, r[slot]))
        return rc;
    return LLMI_HIP_OK;
  };
  auto state = [&](uint32_t s) { return Ref{Space::State, s, 0}; };
  switch (o.kind) {
  case LLMI_GRAPH_RESHAPE:
  case LLMI_GRAPH_SLICE:
    return LLMI_HIP_OK;
  case LLMI_GRAPH_EMBEDDING_GATHER: {
    if (int rc = dense_all({{in[0], 0}, {in[1], 1}, {out[0], 2}}))
      return rc;
    const unsigned tokens = (unsigned)g_.tokens, hidden = (unsigned)dim(out[0], 1);
    const unsigned rows = (unsigned)dim(in[1], 0);
    if (value(in[1]).group_size) {
      Dispatch &d = emit(Launch::EmbeddingW8, "embeddingW8");
      d.p.embedW8 = {tokens, hidden, 0, rows, (hidden + 31) / 32};
      d.buf[0] = r[0], d.buf[1] = r[1], d.buf[2] = {Space::Scale, r[1].index, 0}, d.buf[3] = r[2];
    } else {
      Dispatch &d = emit(Launch::Embedding, "embedding");
      d.p.embed = {tokens, hidden, 0, rows};
      d.buf[0] = r[0], d.buf[1] = r[1], d.buf[2] = r[2];
    }
    return LLMI_HIP_OK;
  }
  case LLMI_GRAPH_LINEAR_F16:
  case LLMI_GRAPH_LINEAR_W8A8:
    return linear(i, out[0], -1, -1);
  case LLMI_GRAPH_QUANTIZE_ACTIVATION: {
    if (value(out[0]).group_size != 32)
      return fail(LLMI_HIP_INVALID_ARGUMENT,
                  "plan: activation quantization requires 32-element groups");
    if (int rc = dense_all({{in[0], 0}, {out[0], 1}, {out[1], 2}}))
      return rc;
    Dispatch &d = emit(Launch::Quantize, "quantizeActivation");
    d.p.quantize = {(unsigned)dim(in[0], 0), (unsigned)dim(in[0], 1), (unsigned)dim(out[1], 1)};
    d.buf[0] = r[0], d.buf[1] = r[1], d.buf[2] = r[2], d.buf[3] = {Space::Invalid, 0, 0};
    return LLMI_HIP_OK;
  }
  case LLMI_GRAPH_RMS_NORM:
  case LLMI_GRAPH_GATED_RMS_NORM: {
    const bool gated = o.kind == LLMI_GRAPH_GATED_RMS_NORM;
    const uint32_t w = in[gated ? 2 : 1];
    const unsigned width = (unsigned)dim(w, 0);
    const RowParams p{(unsigned)(count(in[0]) / width), width, o.epsilon};
    if (!gated && normQuantize_[i] >= 0) {
      const auto &add = normAdd_[i] >= 0 ? op(normAdd_[i]) : o;
      const auto &q = op(normQuantize_[i]);
      if (normAdd_[i] >= 0) {
        if (int rc = dense_all({{add.inputs[0], 0}, {add.inputs[1], 1}, {add.outputs[0], 2}}))
          return rc;
      } else if (int rc = dense(in[0], r[0])) {
        return rc;
      }
      if (int rc = dense_all({{in[1], 3}, {q.outputs[0], 4}, {q.outputs[1], 5}}))
        return rc;
      Dispatch &d = emit(Launch::AddNormQuantize,
                         normAdd_[i] >= 0 ? "addRmsNormQuantize" : "rmsNormQuantize");
      d.p.row = p;
      for (int k = 0; k < 6; ++k)
        d.buf[k] = r[k];
      d.buf[6] = {Space::Invalid, 0, 0};
      if (normAdd_[i] >= 0)
        d.ops.push_back((size_t)normAdd_[i]);
      d.ops.push_back(i);
      d.ops.push_back((size_t)normQuantize_[i]);
      return LLMI_HIP_OK;
    }
    if (!gated) {
      if (int rc = dense_all({{in[0], 0}, {in[1], 1}, {out[0], 2}}))
        return rc;
      Dispatch &d = emit(Launch::RmsNorm, nullptr);
      d.p.row = p;
      d.kernels.push_back(llmi_hip_kernel_name(LLMI_HIP_OP_RMS_NORM, &p, 0));
      d.buf[0] = r[0], d.buf[1] = r[1], d.buf[2] = r[2];
      return LLMI_HIP_OK;
    }
    if (int rc = dense_all({{in[0], 0}, {in[1], 1}, {in[2], 2}, {out[0], 3}}))
      return rc;
    const int64_t gp = value(in[1]).defining_op;
    const bool activated = gp >= 0 && fusion_[gp].kind == LLMI_LINEAR_SILU_F32;
    Dispatch &d = emit(activated ? Launch::GatedRmsNormActivated : Launch::GatedRmsNorm,
                       activated ? "gatedRmsNormActivated" : "gatedRmsNorm");
    d.p.row = p;
    d.buf[0] = r[0], d.buf[1] = r[1], d.buf[2] = r[2], d.buf[3] = r[3];
    return LLMI_HIP_OK;
  }
  case LLMI_GRAPH_L2_NORM: {
    if (int rc = dense_all({{in[0], 0}, {out[0], 1}}))
      return rc;
    Dispatch &d = emit(Launch::L2Norm, "l2NormF32");
    const unsigned width = (unsigned)o.group_width;
    d.p.l2 = {(unsigned)(count(in[0]) / width), width, o.epsilon, o.scale};
    d.buf[0] = r[0], d.buf[1] = r[1];
    return LLMI_HIP_OK;
  }
  case LLMI_GRAPH_SIGMOID_MUL:
    if (gated_[i][0] >= 0)
      return gated_attention(i);
    [[fallthrough]];
  case LLMI_GRAPH_ADD:
  case LLMI_GRAPH_SILU_MUL: {
    const int64_t p = value(in[0]).defining_op;
    if (o.kind == LLMI_GRAPH_SILU_MUL && p >= 0 && fusion_[p].kind == LLMI_LINEAR_SILU_MUL)
      return linear(p, out[0], in[1], -1);
    if (int rc = dense_all({{in[0], 0}, {in[1], 1}, {out[0], 2}}))
      return rc;
    const unsigned n = (unsigned)count(out[0]);
    const int64_t gp = value(in[0]).defining_op >= 0 ? value(root_[in[0]]).defining_op : -1;
    if (o.kind == LLMI_GRAPH_SIGMOID_MUL &&
        !(gp >= 0 && fusion_[gp].kind == LLMI_LINEAR_SIGMOID_COLUMNS)) {
      Dispatch &d = emit(Launch::SigmoidMul, nullptr);
      d.p.element = {n};
      d.kernels.push_back(llmi_hip_kernel_name(LLMI_HIP_OP_SIGMOID_MUL, &d.p.element, 0));
      d.buf[0] = r[0], d.buf[1] = r[1], d.buf[2] = r[2];
      return LLMI_HIP_OK;
    }
    const ElementwiseKind k = o.kind == LLMI_GRAPH_ADD        ? ElementwiseKind::Add
                              : o.kind == LLMI_GRAPH_SILU_MUL ? ElementwiseKind::SwiGlu
                                                              : ElementwiseKind::Multiply;
    Dispatch &d = emit(Launch::Elementwise, k == ElementwiseKind::Add      ? "residualAdd"
                                            : k == ElementwiseKind::SwiGlu ? "swiGlu"
                                                                           : "multiplyF16");
    d.elementwise = k;
    d.p.element = {n};
    d.buf[0] = r[0], d.buf[1] = r[1], d.buf[2] = r[2];
    return LLMI_HIP_OK;
  }
  case LLMI_GRAPH_SILU: {
    const int64_t p = value(in[0]).defining_op;
    if (p >= 0 && fusion_[p].kind == LLMI_LINEAR_SILU)
      return linear(p, out[0], -1, -1);
    if (int rc = dense_all({{in[0], 0}, {out[0], 1}}))
      return rc;
    Dispatch &d = emit(Launch::Elementwise, "siluF16");
    d.elementwise = ElementwiseKind::Silu;
    d.p.element = {(unsigned)count(out[0])};
    d.buf[0] = r[0], d.buf[2] = r[1];
    return LLMI_HIP_OK;
  }
  case LLMI_GRAPH_PARTIAL_ROPE: {
    if (int rc = dense_all({{in[0], 0}, {out[0], 1}}))
      return rc;
    Dispatch &d = emit(Launch::PartialRope, nullptr);
    const unsigned width = (unsigned)dim(in[0], 2);
    d.p.rope = {(unsigned)(count(in[0]) / width), (unsigned)dim(in[0], 1), width,
                (unsigned)o.rotary_width, (unsigned)g_.past, o.theta};
    d.kernels.push_back(llmi_hip_kernel_name(LLMI_HIP_OP_PARTIAL_ROPE, &d.p.rope, 0));
    d.buf[0] = r[0], d.buf[1] = r[1];
    return LLMI_HIP_OK;
  }
  case LLMI_GRAPH_CAUSAL_CONV1D: {
    const int64_t silu = convSilu_[i];
    if (int rc = dense_all({{in[0], 0}, {in[1], 1},
                            {silu >= 0 ? op((size_t)silu).outputs[0] : out[0], 2}}))
      return rc;
    Dispatch &d = emit(Launch::CausalConv, nullptr);
    d.p.conv = {(unsigned)g_.tokens, (unsigned)dim(in[0], 1), (unsigned)dim(in[1], 2),
                silu >= 0 ? 1u : 0u};
    d.kernels.push_back(llmi_hip_kernel_name(LLMI_HIP_OP_CAUSAL_CONV, &d.p.conv, 0));
    d.buf[0] = r[0], d.buf[1] = r[1], d.buf[2] = state(o.state), d.buf[3] = r[2];
    if (silu >= 0)
      d.recs = {{i, nullptr, 0}, {(size_t)silu, nullptr, 0}};
    return LLMI_HIP_OK;
  }
  case LLMI_GRAPH_DELTA_GATES: {
    const int64_t a = value(in[0]).defining_op;
    if (a >= 0 && early_gates((size_t)a))
      return LLMI_HIP_OK; // both projections launched at their own ops
    if (a >= 0 && fusion_[a].kind == LLMI_LINEAR_DELTA_DECAY) {
      if (int rc = linear(a, out[1], in[2], in[3]))
        return rc;
      return linear(value(in[1]).defining_op, out[0], -1, -1);
    }
    if (int rc = dense_all({{in[0], 0}, {in[1], 1}, {in[2], 2}, {in[3], 3}, {out[0], 4},
                            {out[1], 5}}))
      return rc;
    Dispatch &d = emit(Launch::DeltaGates, nullptr);
    d.p.row = {(unsigned)dim(in[0], 0), (unsigned)dim(in[0], 1), 0.0f};
    d.kernels.push_back(llmi_hip_kernel_name(LLMI_HIP_OP_DELTA_GATES, &d.p.row, 0));
    for (int k = 0; k < 6; ++k)
      d.buf[k] = r[k];
    return LLMI_HIP_OK;
  }
  case LLMI_GRAPH_DELTA_UPDATE: {
    const auto &s = g_.states[o.state];
    GraphDeltaParams p{(unsigned)g_.tokens, (unsigned)(dim(in[0], 1) / s.shape[1]),
                       (unsigned)s.shape[1], (unsigned)s.shape[0], (unsigned)s.shape[2]};
    if (l2Delta_[i].first >= 0) {
      const auto &qn = op(l2Delta_[i].first), &kn = op(l2Delta_[i].second);
      if (int rc = dense_all({{qn.inputs[0], 0}, {kn.inputs[0], 1}, {in[2], 2}, {in[3], 3},
                              {in[4], 4}, {out[0], 5}}))
        return rc;
      if (llmi_hip_delta_workspace_bytes(p) != 0)
        return fail(LLMI_HIP_UNSUPPORTED, "plan: op %zu: a one-row update with a workspace", i);
      Dispatch &d = emit(Launch::L2DeltaUpdate, llmi_hip_kernel_name(LLMI_HIP_OP_DELTA_UPDATE,
                                                                     &p, 0));
      d.p.delta = p;
      d.epsilon = qn.epsilon;
      d.scale = qn.scale;
      for (int k = 0; k < 5; ++k)
        d.buf[k] = r[k];
      d.buf[5] = state(o.state);
      d.buf[6] = r[5];
      d.ops = {(size_t)std::min(l2Delta_[i].first, l2Delta_[i].second),
               (size_t)std::max(l2Delta_[i].first, l2Delta_[i].second), i};
      return LLMI_HIP_OK;
    }
    if (int rc = dense_all({{in[0], 0}, {in[1], 1}, {in[2], 2}, {in[3], 3}, {in[4], 4},
                            {out[0], 5}}))
      return rc;
    const unsigned n = llmi_hip_dispatch_count(LLMI_HIP_OP_DELTA_UPDATE, &p);
    if (n == 0)
      return fail(LLMI_HIP_UNSUPPORTED, "plan: op %zu: %s", i, llmi_hip_last_error());
    const uint64_t ws = llmi_hip_delta_workspace_bytes(p);
    Dispatch &d = emit(Launch::DeltaUpdate, nullptr);
    d.p.delta = p;
    for (unsigned k = 0; k < n; ++k)
      d.kernels.push_back(llmi_hip_kernel_name(LLMI_HIP_OP_DELTA_UPDATE, &p, k));
    for (int k = 0; k < 5; ++k)
      d.buf[k] = r[k];
    d.buf[5] = state(o.state);
    d.buf[6] = r[5];
    d.workspaceBytes = ws;
    if (ws)
      d.buf[7] = temporary(ws);
    return LLMI_HIP_OK;
  }
  case LLMI_GRAPH_KV_APPEND: {
    if (int rc = dense_all({{in[0], 0}, {in[1], 1}}))
      return rc;
    const unsigned heads = (unsigned)g_.states[o.keys].shape[1];
    const unsigned hd = (unsigned)g_.states[o.keys].shape[2];
    Dispatch &d = emit(Launch::KvAppend, nullptr);
    d.p.cache = {(unsigned)count(in[0]), (unsigned)(g_.past * heads * hd)};
    d.kernels.push_back(llmi_hip_kernel_name(LLMI_HIP_OP_KV_APPEND, &d.p.cache, 0));
    d.buf[0] = r[0], d.buf[1] = r[1], d.buf[2] = state(o.keys), d.buf[3] = state(o.values);
    return LLMI_HIP_OK;
  }
  case LLMI_GRAPH_CAUSAL_GQA: {
    if (int rc = dense_all({{in[0], 0}, {out[0], 1}}))
      return rc;
    const auto &cache = g_.states[o.keys].shape;
    GqaParams p{(unsigned)g_.tokens, (unsigned)dim(in[0], 1), (unsigned)cache[1],
                (unsigned)cache[2], (unsigned)g_.past};
    const unsigned n = llmi_hip_dispatch_count(LLMI_HIP_OP_CAUSAL_GQA, &p);
    if (n == 0)
      return fail(LLMI_HIP_UNSUPPORTED, "plan: op %zu: %s", i, llmi_hip_last_error());
    const uint64_t ws = llmi_hip_gqa_workspace_bytes(p);
    Dispatch &d = emit(Launch::CausalGqa, nullptr);
    d.p.gqa = p;
    for (unsigned k = 0; k < n; ++k)
      d.kernels.push_back(llmi_hip_kernel_name(LLMI_HIP_OP_CAUSAL_GQA, &p, k));
    d.buf[0] = r[0], d.buf[1] = state(o.keys), d.buf[2] = state(o.values), d.buf[3] = r[1];
    d.workspaceBytes = ws;
    if (ws)
      d.buf[4] = temporary(ws);
    return LLMI_HIP_OK;
  }
  default:
    return fail(LLMI_HIP_INVALID_ARGUMENT, "plan: op %zu has an unknown kind", i);
  }
}

// The attention block closed by SigmoidMul s (prepare_gated_attention), in
// one llmi_hip_gated_attention(_activated) call recorded under each op.
int Lowering::gated_attention(size_t s) {
  const auto &blk = gated_[s];
  const auto &sm = op(s), &nq = op((size_t)blk[0]), &nk = op((size_t)blk[1]);
  const auto &rq = op((size_t)blk[2]), &att = op((size_t)blk[5]);
  const uint32_t gate = sm.inputs[0];
  const uint32_t qg = op((size_t)value(nq.inputs[0]).defining_op).inputs[0];
  Ref r[6];
  for (auto [id, slot] : {std::pair<uint32_t, int>{qg, 0}, {nk.inputs[0], 1},
                          {op((size_t)blk[4]).inputs[1], 2}, {nq.inputs[1], 3},
                          {nk.inputs[1], 4}, {sm.outputs[0], 5}})
    if (int rc = dense(id, r[slot]))
      return rc;
  const auto &cache = g_.states[att.keys].shape;
  const GqaParams p{1, (unsigned)dim(qg, 1), (unsigned)cache[1], (unsigned)cache[2],
                    (unsigned)g_.past};
  const unsigned n = llmi_hip_dispatch_count(LLMI_HIP_OP_GATED_ATTENTION, &p);
  if (n == 0)
    return fail(LLMI_HIP_UNSUPPORTED, "plan: op %zu: %s", s, llmi_hip_last_error());
  const int64_t gp = value(root_[gate]).defining_op;
  Dispatch &d = emit(Launch::GatedAttention, nullptr);
  d.p.gqa = p;
  for (unsigned k = 0; k < n; ++k)
    d.kernels.push_back(llmi_hip_kernel_name(LLMI_HIP_OP_GATED_ATTENTION, &p, k));
  for (int k = 0; k < 5; ++k)
    d.buf[k] = r[k];
  d.buf[5] = {Space::State, att.keys, 0};
  d.buf[6] = {Space::State, att.values, 0};
  d.buf[7] = r[5];
  d.epsilon = nq.epsilon;
  d.rotary = (unsigned)rq.rotary_width;
  d.theta = rq.theta;
  d.activated = gp >= 0 && fusion_[gp].kind == LLMI_LINEAR_SIGMOID_COLUMNS;
  d.workspaceBytes = llmi_hip_gqa_workspace_bytes(p);
  if (d.workspaceBytes)
    d.buf[8] = temporary(d.workspaceBytes);
  // The call reads the projected rows while it writes its output and
  // workspace: the rows are live until this op, so the arena keeps them
  // apart; checked here all the same.
  auto overlap = [](const Ref &a, uint64_t an, const Ref &b, uint64_t bn) {
    return a.space == b.space && a.index == b.index && a.space == Space::Scratch &&
           a.offset < b.offset + bn && b.offset < a.offset + an;
  };
  const uint64_t rowsQ = 2ull * p.queryHeads * 2 * p.headDim, rowKV = 2ull * p.kvHeads * p.headDim;
  const uint64_t outBytes = 2ull * p.queryHeads * p.headDim, ws = d.workspaceBytes;
  const std::pair<Ref, uint64_t> reads[3] = {{r[0], rowsQ}, {r[1], rowKV}, {r[2], rowKV}};
  for (const auto &[ref, n] : reads)
    if (overlap(ref, n, r[5], outBytes) || (ws && overlap(ref, n, d.buf[8], ws)))
      return fail(LLMI_HIP_INVALID_ARGUMENT, "plan: op %zu: the attention block's output "
                  "or workspace overlaps its projected rows", s);
  if (ws && overlap(r[5], outBytes, d.buf[8], ws))
    return fail(LLMI_HIP_INVALID_ARGUMENT, "plan: op %zu: output overlaps the workspace", s);
  for (int64_t x : blk)
    d.recs.push_back({(size_t)x, nullptr, 0});
  d.recs.push_back({s, nullptr, 0});
  std::sort(d.recs.begin(), d.recs.end(), [](const Rec &a, const Rec &b) { return a.op < b.op; });
  return LLMI_HIP_OK;
}

int Lowering::run() {
  if (int rc = validate())
    return rc;
  size_t inputs = 0;
  for (size_t i = 0; i < g_.value_count; ++i)
    if (g_.values[i].kind == LLMI_GRAPH_INPUT) {
      const auto &v = g_.values[i];
      if (++inputs > 1 || v.element != LLMI_GRAPH_U32 || v.rank != 1 || v.shape[0] != g_.tokens)
        return fail(LLMI_HIP_INVALID_ARGUMENT, "plan: expects a single token ID input");
    }
  if (!inputs)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "plan: missing token ID input");
  if (g_.output_count > 1)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "plan: expects one logits output");
  prepare_values();
  prepare_fusions();
  prepare_norm_quantize();
  prepare_l2_delta();
  prepare_kv_decode();
  prepare_conv_silu();
  prepare_gated_attention();
  if (g_.output_count) {
    const uint32_t id = g_.outputs[0];
    const auto &v = value(id);
    if (v.element != LLMI_GRAPH_F16 || v.rank != 2 || v.kind != LLMI_GRAPH_RESULT)
      return fail(LLMI_HIP_INVALID_ARGUMENT, "plan: expects a dense FP16 logits result");
    buffer_[id] = {Space::Output, 0, 0};
    plan_.hasOutput = true;
    plan_.logitRows = v.shape[0];
    plan_.logitElements = count(id);
  }
  plan_.invalidOffset = arena_.allocate(4, g_.op_count);
  for (index_ = 0; index_ < g_.op_count; ++index_) {
    arena_.release_before(index_);
    const Fusion &f = fusion_[index_];
    auto allocate = [&](const llmi_graph_op &of, bool f32) {
      for (uint32_t j = 0; j < of.output_count; ++j) {
        const uint32_t id = of.outputs[j];
        const auto &v = value(id);
        if (v.kind == LLMI_GRAPH_VIEW || buffer_[id].space != Space::None)
          continue;
        const uint64_t bytes = f32 ? 4 : element_bytes(v.element);
        buffer_[id] = {Space::Scratch, 0, arena_.allocate(v.shape[0] * v.strides[0] * bytes,
                                                          lastUse_[id])};
      }
    };
    if (early_gates(index_)) {
      // DeltaGates' a / b projection of a one-row step, launched here into
      // DeltaGates' outputs (its record: this op, fused into DeltaGates), so
      // that it can join the norm launch before it
      const auto &c = op(f.consumer);
      allocate(c, false);
      const int rc = f.kind == LLMI_LINEAR_DELTA_DECAY
                         ? linear(index_, c.outputs[1], c.inputs[2], c.inputs[3])
                         : linear(index_, c.outputs[0], -1, -1);
      if (rc)
        return rc;
      continue;
    }
    if (f.deferred())
      continue; // runs at its consumer, into the consumer's output
    const auto &o = op(index_);
    if (inGated_[index_])
      continue; // launched, and recorded, at the block's SigmoidMul
    if (normQuantize_[index_] >= 0)
      allocate(op(normQuantize_[index_]), false); // the norm itself stores nothing
    else if (convSilu_[index_] >= 0)
      allocate(op(convSilu_[index_]), false); // nor does a convolution with its SiLU
    else
      allocate(o, f.kind == LLMI_LINEAR_SILU_F32);
    if (skip_[index_])
      continue;
    if (int rc = lower(index_))
      return rc;
  }
  plan_.scratchBytes = (arena_.size() + kAlign - 1) / kAlign * kAlign;
  merge_norm_linears();
  for (const auto &d : plan_.dispatches) {
    for (const Rec &r : d.recs) // op by op, so the records stay in op order
      for (const char *k : d.kernels)
        plan_.records.push_back({r.op, k, r.epilogue, r.fused});
    if (!d.recs.empty())
      continue;
    for (const char *k : d.kernels) {
      if (d.ops.empty())
        plan_.records.push_back({d.opIndex, k, d.epilogue, d.fusedOpIndex});
      for (size_t o : d.ops)
        plan_.records.push_back({o, k, nullptr, 0});
    }
  }
  plan_.stateCount = g_.state_count;
  return LLMI_HIP_OK;
}

struct Bases {
  unsigned char *scratch;
  void *const *states;
  const llmi_weight *weights;
  const uint32_t *tokens;
  uint16_t *logits;
  uint32_t *invalid;
};

void *resolve(const Bases &b, const Ref &r) {
  unsigned char *base = nullptr;
  switch (r.space) {
  case Space::None:
    return nullptr;
  case Space::Scratch:
    base = b.scratch;
    break;
  case Space::Weight:
    base = (unsigned char *)b.weights[r.index].data;
    break;
  case Space::Scale:
    base = (unsigned char *)b.weights[r.index].scales;
    break;
  case Space::State:
    base = (unsigned char *)b.states[r.index];
    break;
  case Space::Input:
    base = (unsigned char *)b.tokens;
    break;
  case Space::Output:
    base = (unsigned char *)b.logits;
    break;
  case Space::Invalid:
    return b.invalid;
  }
  return base ? base + r.offset : nullptr;
}

int run_dispatch(const Dispatch &d, const Bases &b, hipStream_t stream) {
  void *x[12];
  for (int i = 0; i < 12; ++i)
    x[i] = resolve(b, d.buf[i]);
  auto u16 = [&](int i) { return static_cast<uint16_t *>(x[i]); };
  auto f32 = [&](int i) { return static_cast<float *>(x[i]); };
  switch (d.launch) {
  case Launch::Embedding:
    return llmi_hip_embedding((const uint32_t *)x[0], u16(1), u16(2), d.p.embed, stream);
  case Launch::EmbeddingW8:
    return llmi_hip_embedding_w8((const uint32_t *)x[0], (const int8_t *)x[1], u16(2), u16(3),
                                 d.p.embedW8, stream);
  case Launch::Quantize:
    return llmi_hip_quantize_activation(u16(0), (int8_t *)x[1], f32(2), (uint32_t *)x[3],
                                        d.p.quantize, stream);
  case Launch::LinearW8:
    return llmi_hip_linear_w8a8((const int8_t *)x[0], f32(1), (const int8_t *)x[2], u16(3),
                                x[4], x[5], f32(6), d.p.linearW8, stream);
  case Launch::LinearF16:
    return llmi_hip_linear_f16(u16(0), u16(2), x[4], x[5], f32(6), d.p.linear, stream);
  case Launch::RmsNorm:
    return llmi_hip_rms_norm(u16(0), f32(1), u16(2), d.p.row, stream);
  case Launch::GatedRmsNorm:
    return llmi_hip_gated_rms_norm(u16(0), u16(1), f32(2), u16(3), d.p.row, stream);
  case Launch::GatedRmsNormActivated:
    return llmi_hip_gated_rms_norm_activated(u16(0), f32(1), f32(2), u16(3), d.p.row, stream);
  case Launch::L2Norm:
    return llmi_hip_l2_norm(u16(0), f32(1), d.p.l2, stream);
  case Launch::Elementwise:
    switch (d.elementwise) {
    case ElementwiseKind::Add:
      return llmi_hip_residual_add(u16(0), u16(1), u16(2), d.p.element, stream);
    case ElementwiseKind::SwiGlu:
      return llmi_hip_swiglu(u16(0), u16(1), u16(2), d.p.element, stream);
    case ElementwiseKind::Silu:
      return llmi_hip_silu(u16(0), u16(2), d.p.element, stream);
    case ElementwiseKind::Multiply:
      return llmi_hip_multiply(u16(0), u16(1), u16(2), d.p.element, stream);
    }
    break;
  case Launch::SigmoidMul:
    return llmi_hip_sigmoid_mul(u16(0), u16(1), u16(2), d.p.element, stream);
  case Launch::PartialRope:
    return llmi_hip_partial_rope(u16(0), u16(1), d.p.rope, stream);
  case Launch::CausalConv:
    return llmi_hip_causal_conv(u16(0), u16(1), u16(2), u16(3), d.p.conv, stream);
  case Launch::DeltaGates:
    return llmi_hip_delta_gates(u16(0), u16(1), f32(2), f32(3), f32(4), f32(5), d.p.row,
                                stream);
  case Launch::DeltaUpdate:
    return llmi_hip_delta_update(f32(0), f32(1), u16(2), f32(3), f32(4), f32(5), u16(6),
                                 d.p.delta, x[7], d.workspaceBytes, stream);
  case Launch::KvAppend:
    return llmi_hip_kv_append(u16(0), u16(1), u16(2), u16(3), d.p.cache, stream);
  case Launch::CausalGqa:
    return llmi_hip_causal_gqa(u16(0), u16(1), u16(2), u16(3), d.p.gqa, x[4],
                               d.workspaceBytes, stream);
  case Launch::KvAppendGqa:
    return llmi_hip_kv_append_causal_gqa(u16(0), u16(5), u16(6), u16(1), u16(2), u16(3),
                                         d.p.gqa, x[4], d.workspaceBytes, stream);
  case Launch::CopyView:
    return llmi_hip_copy_half_view(u16(0), u16(1), d.p.view, stream);
  case Launch::GatedAttention:
    return (d.activated ? llmi_hip_gated_attention_activated : llmi_hip_gated_attention)(
        u16(0), u16(1), u16(2), f32(3), f32(4), u16(5), u16(6), u16(7), d.p.gqa, d.rotary,
        d.epsilon, d.theta, x[8], d.workspaceBytes, stream);
  case Launch::GatedNormQuantize:
    return llmi_hip_gated_rms_norm_activated_quantize(u16(0), f32(1), f32(2), u16(3),
                                                      (int8_t *)x[4], f32(5), (uint32_t *)x[6],
                                                      d.p.row, stream);
  case Launch::L2DeltaUpdate:
    return llmi_hip_l2_norm_delta_update(u16(0), u16(1), u16(2), f32(3), f32(4), f32(5), u16(6),
                                         d.p.delta, d.epsilon, d.scale, nullptr, 0, stream);
  case Launch::L2DeltaNormQuantize:
    return llmi_hip_l2_norm_delta_gated_norm_activated_quantize(
        u16(0), u16(1), u16(2), f32(3), f32(4), f32(5), f32(7), f32(8), u16(9), (int8_t *)x[10],
        f32(11), (uint32_t *)x[6], d.p.delta, d.epsilon, d.scale, d.normEpsilon, stream);
  case Launch::AddNormQuantize:
    return llmi_hip_add_rms_norm_quantize(u16(0), u16(1), u16(2), f32(3), (int8_t *)x[4],
                                          f32(5), (uint32_t *)x[6], d.p.row, stream);
  case Launch::AddNormLinear: {
    llmi_hip_norm_projection proj[kNormLinearMax] = {};
    for (unsigned k = 0; k < d.p.normLinear.count; ++k)
      proj[k] = {static_cast<const int8_t *>(resolve(b, d.proj[k][0])),
                 static_cast<const uint16_t *>(resolve(b, d.proj[k][1])),
                 resolve(b, d.proj[k][2]), resolve(b, d.proj[k][3]),
                 static_cast<const float *>(resolve(b, d.proj[k][4])),
                 static_cast<const uint16_t *>(resolve(b, d.proj[k][5])),
                 static_cast<uint16_t *>(resolve(b, d.proj[k][6]))};
    return llmi_hip_add_rms_norm_linear_w8a8(u16(0), u16(1), u16(2), f32(3), (int8_t *)x[4],
                                             f32(5), (uint32_t *)x[6], proj, d.p.normLinear,
                                             stream);
  }
  }
  return fail(LLMI_HIP_INVALID_ARGUMENT, "plan: unknown dispatch");
}

} // namespace
} // namespace llmi

using namespace llmi;

int llmi_hip_plan_lower(const llmi_graph *graph, const llmi_weight *weights, size_t weight_count,
                        llmi_hip_plan **out) {
  if (!out)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "plan: null output");
  *out = nullptr;
  if (!graph || (weight_count && !weights))
    return fail(LLMI_HIP_INVALID_ARGUMENT, "plan: null graph or weights");
  auto *plan = new llmi_hip_plan();
  plan->weights.assign(weights, weights + weight_count);
  Lowering lowering(*graph, weight_count, *plan);
  if (int rc = lowering.run()) {
    delete plan;
    return rc;
  }
  *out = plan;
  return LLMI_HIP_OK;
}

void llmi_hip_plan_destroy(llmi_hip_plan *plan) { delete plan; }

size_t llmi_hip_plan_scratch_bytes(const llmi_hip_plan *plan) {
  return plan ? plan->scratchBytes : 0;
}

void llmi_hip_plan_logits(const llmi_hip_plan *plan, uint64_t *rows, uint64_t *elements) {
  if (rows)
    *rows = plan ? plan->logitRows : 0;
  if (elements)
    *elements = plan ? plan->logitElements : 0;
}

size_t llmi_hip_plan_dispatches(const llmi_hip_plan *plan, llmi_hip_dispatch *records,
                                size_t cap) {
  if (!plan)
    return 0;
  if (records)
    std::memcpy(records, plan->records.data(),
                sizeof(llmi_hip_dispatch) * std::min(cap, plan->records.size()));
  return plan->records.size();
}

size_t llmi_hip_plan_launches(const llmi_hip_plan *plan) {
  size_t n = 0;
  if (plan)
    for (const auto &d : plan->dispatches)
      n += d.kernels.size();
  return n;
}

int llmi_hip_plan_execute(const llmi_hip_plan *plan, void *scratch, size_t scratch_bytes,
                          void *const *states, size_t state_count, const uint32_t *token_ids,
                          uint16_t *logits, uint32_t *invalid, void *stream) {
  if (!plan)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "plan: null plan");
  if (scratch_bytes < plan->scratchBytes || (plan->scratchBytes && !scratch))
    return fail(LLMI_HIP_WORKSPACE, "plan: needs a %llu-byte scratch arena",
                (unsigned long long)plan->scratchBytes);
  if (state_count != plan->stateCount || (state_count && !states))
    return fail(LLMI_HIP_INVALID_ARGUMENT, "plan: expects %zu state buffers",
                plan->stateCount);
  for (size_t i = 0; i < state_count; ++i)
    if (!states[i])
      return fail(LLMI_HIP_INVALID_ARGUMENT, "plan: state %zu is null", i);
  if (!token_ids || (plan->hasOutput && !logits))
    return fail(LLMI_HIP_INVALID_ARGUMENT, "plan: null token IDs or logits");
  unsigned char *base = static_cast<unsigned char *>(scratch);
  const Bases b{base, states, plan->weights.data(), token_ids, logits,
                invalid ? invalid : reinterpret_cast<uint32_t *>(base + plan->invalidOffset)};
  for (const auto &d : plan->dispatches)
    if (int rc = run_dispatch(d, b, static_cast<hipStream_t>(stream)))
      return rc;
  return LLMI_HIP_OK;
}
