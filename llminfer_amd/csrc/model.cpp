// The Qwen3.5 model session: the whole-model counterpart of MetalSession
// (include/llminfer/Backend/Metal/MetalSession.h:26-50) and its executor
// (lib/Backend/Metal/MetalExecutor.mm:56-118, 212-298), over the whole-graph
// plan (plan.cpp). Declarations: include/llminfer_hip.h.
//
//  * The step graph. Every step builds the graph of its shape (tokens, past,
//    capacity, logits mode), as MetalSession::step calls
//    Qwen35ModelBuilder::build (MetalExecutor.mm:264-266). The op sequence
//    is the builder's (lib/Models/Qwen35/Qwen35ModelBuilder.cpp:127-230):
//    the op indices are the interface the plan records report, so the order
//    of ops, of values (weights enter at their first use) and of states has
//    to be the reference's. The result types follow the contracts of
//    lib/GraphIR/Graph.cpp:140-380 for the shapes this builder produces;
//    tests/test_model.py holds the graph equal, field by field, to the
//    Python builder's, whose graphs are replayed through the reference's own
//    Graph.cpp.
//  * The session. open allocates one device buffer per state slot (KV
//    caches, DeltaNet recurrent states, conv histories) and zeroes them
//    (MetalExecutor.mm:56-94, 115-118); the weights are the caller's device
//    tensors, looked up by tensor id. step validates before any launch
//    (empty chunk, capacity, vocabulary, state layout: MetalExecutor.mm:
//    255-276), lowers, runs with one host synchronisation, reads back the
//    fp16 logits as floats (MetalStepResult, MetalSession.h:18-24) and
//    advances past only on success. A failure after the launches (or a
//    non-finite activation flagged by a quantization, MetalExecutor.mm:
//    180-187) leaves the session invalid until reset (:283-298).
#include "llminfer_hip.h"
#include "capi_internal.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <memory>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

namespace llmi {
namespace {

constexpr uint64_t kGroup = 32; // int8 weight and activation group width

struct ModelConfig {
  llmi_qwen35_config c;
  std::vector<uint8_t> layers; // owned copy of c.layer_kinds
  uint64_t keyWidth() const { return c.key_heads * c.key_dim; }
  uint64_t valueWidth() const { return c.value_heads * c.value_dim; }
  uint64_t qkvWidth() const { return 2 * keyWidth() + valueWidth(); }
  uint64_t queryWidth() const { return c.q_heads * c.head_dim; }
  uint64_t kvWidth() const { return c.kv_heads * c.head_dim; }
};

struct Shape {
  uint32_t rank = 0;
  uint64_t d[LLMI_GRAPH_MAX_RANK] = {};
  Shape() = default;
  Shape(std::initializer_list<uint64_t> dims) {
    for (uint64_t x : dims)
      d[rank++] = x;
  }
};

} // namespace
} // namespace llmi

// One step's graph in the flat form llmi_hip_plan_lower takes; `tensors`
// maps a weight value's `weight` index to its tensor id.
struct llmi_qwen35_graph {
  uint64_t tokens = 0, past = 0, capacity = 0;
  std::vector<llmi_graph_value> values;
  std::vector<llmi_graph_state> states;
  std::vector<llmi_graph_op> ops;
  std::vector<uint32_t> outputs;
  std::vector<std::string> tensors;
  llmi_graph flat;

  void seal() {
    flat = llmi_graph{tokens, past, capacity, values.data(), values.size(),
                      states.data(), states.size(), ops.data(), ops.size(),
                      outputs.data(), outputs.size()};
  }
};

namespace llmi {
namespace {

using Graph = llmi_qwen35_graph;

llmi_graph_value make_value(uint32_t element, uint32_t kind, const Shape &s,
                            uint64_t group = 0) {
  llmi_graph_value v{};
  v.element = element;
  v.kind = kind;
  v.rank = s.rank;
  uint64_t stride = 1;
  for (int i = (int)s.rank - 1; i >= 0; --i) {
    v.shape[i] = s.d[i];
    v.strides[i] = stride;
    stride *= s.d[i];
  }
  if (group) // grouped int8 rows are padded to whole groups
    v.strides[0] = (s.d[1] + group - 1) / group * group;
  v.group_size = group;
  v.view_of = v.defining_op = v.weight = -1;
  return v;
}

Shape shape_of(const llmi_graph_value &v) {
  Shape s;
  s.rank = v.rank;
  for (uint32_t i = 0; i < v.rank; ++i)
    s.d[i] = v.shape[i];
  return s;
}

// Emits the graph of one step. Weights enter the value list at their first
// use; a tensor id used twice (the tied head) resolves to the same value.
class Builder {
public:
  Builder(const ModelConfig &m, Graph &g) : m_(m), g_(g) {}

  int32_t layer = -1;

  uint32_t input(uint32_t element, const Shape &s) {
    g_.values.push_back(make_value(element, LLMI_GRAPH_INPUT, s));
    return (uint32_t)g_.values.size() - 1;
  }

  // A model matrix: int8 with 32-wide groups under W8A8, else fp16.
  uint32_t matrix(const std::string &id, uint64_t rows, uint64_t cols) {
    return m_.c.w8 ? weight(id, LLMI_GRAPH_I8, {rows, cols}, kGroup)
                   : weight(id, LLMI_GRAPH_F16, {rows, cols});
  }
  uint32_t vector(const std::string &id, uint64_t n) {
    return weight(id, LLMI_GRAPH_F32, {n});
  }
  uint32_t weight(const std::string &id, uint32_t element, const Shape &s,
                  uint64_t group = 0) {
    auto it = std::find(g_.tensors.begin(), g_.tensors.end(), id);
    if (it != g_.tensors.end()) {
      const int64_t w = it - g_.tensors.begin();
      for (size_t i = 0; i < g_.values.size(); ++i)
        if (g_.values[i].kind == LLMI_GRAPH_WEIGHT && g_.values[i].weight == w)
          return (uint32_t)i;
    }
    llmi_graph_value v = make_value(element, LLMI_GRAPH_WEIGHT, s, group);
    v.weight = (int64_t)g_.tensors.size();
    g_.tensors.push_back(id);
    g_.values.push_back(v);
    return (uint32_t)g_.values.size() - 1;
  }

  uint32_t state(uint32_t kind, uint32_t element, const Shape &s) {
    llmi_graph_state st{};
    st.kind = kind;
    st.layer = (uint32_t)layer;
    st.element = element;
    st.rank = s.rank;
    for (uint32_t i = 0; i < s.rank; ++i)
      st.shape[i] = s.d[i];
    g_.states.push_back(st);
    return (uint32_t)g_.states.size() - 1;
  }

  // A new op with its inputs; results are added with result() / view().
  llmi_graph_op &op(uint32_t kind, std::initializer_list<uint32_t> inputs) {
    llmi_graph_op o{};
    o.kind = kind;
    o.layer = layer;
    for (uint32_t x : inputs)
      o.inputs[o.input_count++] = x;
    g_.ops.push_back(o);
    return g_.ops.back();
  }
  uint32_t result(uint32_t element, const Shape &s, uint64_t group = 0) {
    llmi_graph_value v = make_value(element, LLMI_GRAPH_RESULT, s, group);
    return add_output(v);
  }
  const llmi_graph_value &value(uint32_t id) const { return g_.values[id]; }

  // The builder's ops (Qwen35ModelBuilder.cpp:127-230).
  uint32_t unary(uint32_t kind, uint32_t x, uint32_t element) {
    op(kind, {x});
    return result(element, shape_of(value(x)));
  }
  uint32_t binary(uint32_t kind, uint32_t a, uint32_t b) {
    op(kind, {a, b});
    return result(LLMI_GRAPH_F16, shape_of(value(a)));
  }
  uint32_t rms_norm(uint32_t x, const std::string &id) {
    const uint32_t w = vector(id, value(x).shape[value(x).rank - 1]);
    op(LLMI_GRAPH_RMS_NORM, {x, w}).epsilon = (float)m_.c.epsilon;
    return result(LLMI_GRAPH_F16, shape_of(value(x)));
  }
  // RESHAPE to a dense shape, or SLICE of one axis: views of x.
  uint32_t reshape(uint32_t x, const Shape &s) {
    op(LLMI_GRAPH_RESHAPE, {x});
    llmi_graph_value v = make_value(value(x).element, LLMI_GRAPH_VIEW, s);
    v.view_of = x;
    return add_output(v);
  }
  uint32_t slice(uint32_t x, uint64_t axis, uint64_t begin, uint64_t length) {
    llmi_graph_op &o = op(LLMI_GRAPH_SLICE, {x});
    o.axis = axis;
    o.begin = begin;
    o.length = length;
    llmi_graph_value v = value(x);
    v.kind = LLMI_GRAPH_VIEW;
    v.shape[axis] = length;
    v.view_of = x;
    v.view_offset = begin * v.strides[axis];
    v.weight = -1;
    v.group_size = 0;
    return add_output(v);
  }

  // (x, its quantization's data and scales) of a projection input.
  struct Prepared {
    uint32_t x, data, scales;
  };
  Prepared prepare(uint32_t x) {
    if (!m_.c.w8)
      return {x, 0, 0};
    const uint64_t rows = value(x).shape[0], width = value(x).shape[1];
    op(LLMI_GRAPH_QUANTIZE_ACTIVATION, {x}).group_size = kGroup;
    const uint32_t data = result(LLMI_GRAPH_I8, {rows, width}, kGroup);
    const uint32_t scales = result(LLMI_GRAPH_F32, {rows, 1 + (width - 1) / kGroup});
    return {x, data, scales};
  }
  uint32_t project(const Prepared &p, const std::string &id, uint64_t rows) {
    const uint64_t cols = value(p.x).shape[1];
    const uint32_t w = matrix(id, rows, cols);
    if (m_.c.w8)
      op(LLMI_GRAPH_LINEAR_W8A8, {p.data, p.scales, w});
    else
      op(LLMI_GRAPH_LINEAR_F16, {p.x, w});
    return result(LLMI_GRAPH_F16, {value(p.x).shape[0], rows});
  }

private:
  uint32_t add_output(llmi_graph_value v) {
    llmi_graph_op &o = g_.ops.back();
    v.defining_op = (int64_t)g_.ops.size() - 1;
    g_.values.push_back(v);
    const uint32_t id = (uint32_t)g_.values.size() - 1;
    o.outputs[o.output_count++] = id;
    return id;
  }

  const ModelConfig &m_;
  Graph &g_;
};

// Gated DeltaNet mixer of one layer (Qwen35ModelBuilder.cpp:141-166).
uint32_t delta_layer(Builder &b, const ModelConfig &m, uint32_t x, const std::string &pre,
                     uint64_t tokens) {
  const auto &c = m.c;
  const uint32_t history =
      b.state(LLMI_GRAPH_CONV_HISTORY, LLMI_GRAPH_F16, {m.qkvWidth(), c.conv_kernel - 1});
  const uint32_t recurrent = b.state(LLMI_GRAPH_DELTA_RECURRENT, LLMI_GRAPH_F32,
                                     {c.value_heads, c.key_dim, c.value_dim});
  const Builder::Prepared p = b.prepare(x);
  uint32_t qkv = b.project(p, pre + "in_proj_qkv.weight", m.qkvWidth());
  const uint32_t z = b.project(p, pre + "in_proj_z.weight", m.valueWidth());
  const uint32_t a = b.project(p, pre + "in_proj_a.weight", c.value_heads);
  const uint32_t beta = b.project(p, pre + "in_proj_b.weight", c.value_heads);
  {
    const uint32_t w = b.weight(pre + "conv1d.weight", LLMI_GRAPH_F16,
                                {m.qkvWidth(), 1, c.conv_kernel});
    b.op(LLMI_GRAPH_CAUSAL_CONV1D, {qkv, w}).state = history;
    qkv = b.result(LLMI_GRAPH_F16, {tokens, m.qkvWidth()});
  }
  qkv = b.unary(LLMI_GRAPH_SILU, qkv, LLMI_GRAPH_F16);
  const uint64_t kw = m.keyWidth();
  uint32_t q = b.slice(qkv, 1, 0, kw);
  uint32_t k = b.slice(qkv, 1, kw, kw);
  const uint32_t v = b.slice(qkv, 1, 2 * kw, m.valueWidth());
  // 1 / sqrt(dk), each step correctly rounded in fp32
  const float scale = 1.0f / std::sqrt((float)c.key_dim);
  for (int i = 0; i < 2; ++i) {
    uint32_t &t = i ? k : q;
    llmi_graph_op &o = b.op(LLMI_GRAPH_L2_NORM, {t});
    o.group_width = c.key_dim;
    o.epsilon = 1e-6f;
    o.scale = i ? 1.0f : scale;
    t = b.result(LLMI_GRAPH_F32, {tokens, kw});
  }
  const uint32_t aLog = b.vector(pre + "A_log", c.value_heads);
  const uint32_t dtBias = b.vector(pre + "dt_bias", c.value_heads);
  b.op(LLMI_GRAPH_DELTA_GATES, {a, beta, aLog, dtBias});
  const uint32_t gBeta = b.result(LLMI_GRAPH_F32, {tokens, c.value_heads});
  const uint32_t gDecay = b.result(LLMI_GRAPH_F32, {tokens, c.value_heads});
  b.op(LLMI_GRAPH_DELTA_UPDATE, {q, k, v, gBeta, gDecay}).state = recurrent;
  const uint32_t mixed = b.result(LLMI_GRAPH_F16, {tokens, m.valueWidth()});
  const uint32_t nw = b.vector(pre + "norm.weight", c.value_dim);
  b.op(LLMI_GRAPH_GATED_RMS_NORM, {mixed, z, nw}).epsilon = (float)c.epsilon;
  const uint32_t gated = b.result(LLMI_GRAPH_F16, {tokens, m.valueWidth()});
  return b.project(b.prepare(gated), pre + "out_proj.weight", c.hidden);
}

// Gated GQA mixer of one layer (Qwen35ModelBuilder.cpp:168-199).
uint32_t gqa_layer(Builder &b, const ModelConfig &m, uint32_t x, const std::string &pre,
                   uint64_t tokens, uint64_t capacity) {
  const auto &c = m.c;
  const uint32_t keys =
      b.state(LLMI_GRAPH_KEY_CACHE, LLMI_GRAPH_F16, {capacity, c.kv_heads, c.head_dim});
  const uint32_t vals =
      b.state(LLMI_GRAPH_VALUE_CACHE, LLMI_GRAPH_F16, {capacity, c.kv_heads, c.head_dim});
  const Builder::Prepared p = b.prepare(x);
  uint32_t qGate = b.project(p, pre + "q_proj.weight", 2 * m.queryWidth());
  uint32_t k = b.project(p, pre + "k_proj.weight", m.kvWidth());
  uint32_t v = b.project(p, pre + "v_proj.weight", m.kvWidth());
  qGate = b.reshape(qGate, {tokens, c.q_heads, 2 * c.head_dim});
  uint32_t q = b.slice(qGate, 2, 0, c.head_dim);
  const uint32_t gate = b.slice(qGate, 2, c.head_dim, c.head_dim);
  k = b.reshape(k, {tokens, c.kv_heads, c.head_dim});
  v = b.reshape(v, {tokens, c.kv_heads, c.head_dim});
  q = b.rms_norm(q, pre + "q_norm.weight");
  k = b.rms_norm(k, pre + "k_norm.weight");
  for (int i = 0; i < 2; ++i) {
    uint32_t &t = i ? k : q;
    llmi_graph_op &o = b.op(LLMI_GRAPH_PARTIAL_ROPE, {t});
    o.rotary_width = c.rotary_width;
    o.theta = (float)c.theta;
    t = b.result(LLMI_GRAPH_F16, shape_of(b.value(t)));
  }
  {
    llmi_graph_op &o = b.op(LLMI_GRAPH_KV_APPEND, {k, v});
    o.keys = keys;
    o.values = vals;
  }
  {
    llmi_graph_op &o = b.op(LLMI_GRAPH_CAUSAL_GQA, {q});
    o.keys = keys;
    o.values = vals;
  }
  uint32_t mixed = b.result(LLMI_GRAPH_F16, {tokens, c.q_heads, c.head_dim});
  mixed = b.binary(LLMI_GRAPH_SIGMOID_MUL, gate, mixed);
  mixed = b.reshape(mixed, {tokens, m.queryWidth()});
  return b.project(b.prepare(mixed), pre + "o_proj.weight", c.hidden);
}

int check_config(const ModelConfig &m) {
  const auto &c = m.c;
  if (!c.hidden || !c.intermediate || !c.vocabulary || !c.head_dim || !c.q_heads ||
      !c.kv_heads || !c.rotary_width || !c.key_heads || !c.value_heads || !c.key_dim ||
      !c.value_dim || c.conv_kernel < 2 || !c.layer_count || !c.max_positions ||
      c.q_heads % c.kv_heads || c.value_heads % c.key_heads ||
      c.rotary_width % 2 || c.rotary_width > c.head_dim ||
      !(c.epsilon > 0) || !std::isfinite(c.epsilon) || !(c.theta > 0) ||
      !std::isfinite(c.theta))
    return fail(LLMI_HIP_INVALID_ARGUMENT, "model: invalid Qwen3.5 text config");
  for (uint8_t k : m.layers)
    if (k > 1)
      return fail(LLMI_HIP_INVALID_ARGUMENT, "model: unknown layer kind %u", (unsigned)k);
  return LLMI_HIP_OK;
}

int copy_config(const llmi_qwen35_config *c, ModelConfig &m) {
  if (!c || (c->layer_count && !c->layer_kinds))
    return fail(LLMI_HIP_INVALID_ARGUMENT, "model: null config");
  m.c = *c;
  m.layers.assign(c->layer_kinds, c->layer_kinds + c->layer_count);
  m.c.layer_kinds = m.layers.data();
  return check_config(m);
}

// The graph of one step (Qwen35ModelBuilder::build, Qwen35ModelBuilder.cpp:
// 100-235): capacity 0 means past + tokens.
int build(const ModelConfig &m, uint64_t tokens, uint64_t past, uint64_t capacity, int mode,
          Graph &g) {
  const auto &c = m.c;
  if (!capacity)
    capacity = past + tokens;
  if (capacity > c.max_positions)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "Graph capacity exceeds the model context limit");
  if (!tokens || past > capacity || tokens > capacity - past)
    return fail(LLMI_HIP_INVALID_ARGUMENT,
                "Invalid graph step: expected 0 < tokens <= capacity - past");
  if (mode < LLMI_LOGITS_NONE || mode > LLMI_LOGITS_ALL)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "model: unknown logits mode %d", mode);
  g = Graph{};
  g.tokens = tokens;
  g.past = past;
  g.capacity = capacity;
  Builder b(m, g);
  const uint32_t ids = b.input(LLMI_GRAPH_U32, {tokens});
  uint32_t hidden;
  {
    const uint32_t table = b.matrix("embed_tokens.weight", c.vocabulary, c.hidden);
    b.op(LLMI_GRAPH_EMBEDDING_GATHER, {ids, table});
    hidden = b.result(LLMI_GRAPH_F16, {tokens, c.hidden});
  }
  for (uint32_t i = 0; i < c.layer_count; ++i) {
    b.layer = (int32_t)i;
    const std::string pre = "layers." + std::to_string(i) + ".";
    const uint32_t x = b.rms_norm(hidden, pre + "input_layernorm.weight");
    const uint32_t mixed = m.layers[i] == LLMI_QWEN35_GQA
                               ? gqa_layer(b, m, x, pre + "self_attn.", tokens, capacity)
                               : delta_layer(b, m, x, pre + "linear_attn.", tokens);
    const uint32_t residual = b.binary(LLMI_GRAPH_ADD, hidden, mixed);
    const uint32_t y = b.rms_norm(residual, pre + "post_attention_layernorm.weight");
    const Builder::Prepared p = b.prepare(y);
    const uint32_t gate = b.project(p, pre + "mlp.gate_proj.weight", c.intermediate);
    const uint32_t up = b.project(p, pre + "mlp.up_proj.weight", c.intermediate);
    const uint32_t act = b.binary(LLMI_GRAPH_SILU_MUL, gate, up);
    const uint32_t down = b.project(b.prepare(act), pre + "mlp.down_proj.weight", c.hidden);
    hidden = b.binary(LLMI_GRAPH_ADD, residual, down);
  }
  b.layer = -1;
  if (mode != LLMI_LOGITS_NONE) {
    if (mode == LLMI_LOGITS_LAST && tokens > 1)
      hidden = b.slice(hidden, 0, tokens - 1, 1);
    hidden = b.rms_norm(hidden, "norm.weight");
    // the tied head: lm_head.weight resolves to the embedding
    g.outputs.push_back(b.project(b.prepare(hidden), "embed_tokens.weight", c.vocabulary));
  }
  g.seal();
  return LLMI_HIP_OK;
}

bool same_state(const llmi_graph_state &a, const llmi_graph_state &b) {
  if (a.kind != b.kind || a.layer != b.layer || a.element != b.element || a.rank != b.rank)
    return false;
  for (uint32_t i = 0; i < a.rank; ++i)
    if (a.shape[i] != b.shape[i])
      return false;
  return true;
}

size_t state_bytes(const llmi_graph_state &s) {
  size_t n = s.element == LLMI_GRAPH_F32 ? 4 : 2;
  for (uint32_t i = 0; i < s.rank; ++i)
    n *= s.shape[i];
  return n;
}

float half_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1F, f = h & 0x3FF;
  uint32_t bits;
  if (e == 0x1F)
    bits = sign | 0x7F800000u | (f << 13);
  else if (e)
    bits = sign | ((e + 112) << 23) | (f << 13);
  else if (f) { // subnormal: f * 2^-24, exact in fp32
    const float x = (float)f * 0x1p-24f;
    std::memcpy(&bits, &x, 4);
    bits |= sign;
  } else
    bits = sign;
  float x;
  std::memcpy(&x, &bits, 4);
  return x;
}

} // namespace
} // namespace llmi

using namespace llmi;

struct llmi_hip_model {
  ModelConfig cfg;
  std::unordered_map<std::string, llmi_weight> weights;
  uint64_t capacity = 0, past = 0;
  bool invalid = false;
  hipStream_t stream = nullptr;
  std::vector<llmi_graph_state> layout;
  std::vector<void *> states;
  void *scratch = nullptr;
  size_t scratchBytes = 0;
  uint32_t *ids = nullptr;   // device: one step's token IDs (capacity rows)
  uint32_t *flag = nullptr;  // device: the quantizations' non-finite flag
  uint16_t *logits = nullptr;
  size_t logitBytes = 0;
  std::vector<llmi_hip_dispatch> records; // the last step's plan records
};

namespace llmi {
namespace {

void release(llmi_hip_model *s) {
  for (void *p : s->states)
    if (p)
      (void)hipFree(p);
  s->states.clear();
  for (void *p : {(void *)s->scratch, (void *)s->ids, (void *)s->flag, (void *)s->logits})
    if (p)
      (void)hipFree(p);
  s->scratch = s->ids = nullptr;
  s->flag = nullptr;
  s->logits = nullptr;
  s->scratchBytes = s->logitBytes = 0;
}

hipError_t zero_states(llmi_hip_model *s) {
  for (size_t i = 0; i < s->states.size(); ++i)
    if (hipError_t e = hipMemsetAsync(s->states[i], 0, state_bytes(s->layout[i]), s->stream))
      return e;
  return hipStreamSynchronize(s->stream);
}

// Grows a device buffer between steps (the stream is idle then).
int grow(void **buf, size_t &have, size_t need, hipStream_t stream, const char *what) {
  if (need <= have)
    return LLMI_HIP_OK;
  (void)hipStreamSynchronize(stream);
  void *p = nullptr;
  if (hipMalloc(&p, need) != hipSuccess)
    return fail(LLMI_HIP_WORKSPACE, "model: cannot allocate %zu bytes of %s", need, what);
  if (*buf)
    (void)hipFree(*buf);
  *buf = p;
  have = need;
  return LLMI_HIP_OK;
}

// The plan of a step graph over the model's weights.
int lower(const llmi_hip_model *s, const Graph &g, llmi_hip_plan **out) {
  std::vector<llmi_weight> table(g.tensors.size());
  for (size_t i = 0; i < g.tensors.size(); ++i) {
    auto it = s->weights.find(g.tensors[i]);
    if (it == s->weights.end())
      return fail(LLMI_HIP_INVALID_ARGUMENT, "model: missing tensor %s", g.tensors[i].c_str());
    table[i] = it->second;
  }
  return llmi_hip_plan_lower(&g.flat, table.data(), table.size(), out);
}

struct PlanOwner {
  llmi_hip_plan *p = nullptr;
  ~PlanOwner() { llmi_hip_plan_destroy(p); }
};

} // namespace
} // namespace llmi

extern "C" {

int llmi_qwen35_build(const llmi_qwen35_config *config, uint64_t tokens, uint64_t past,
                      uint64_t capacity, int logits_mode, llmi_qwen35_graph **out) {
  if (!out)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "model: null output");
  *out = nullptr;
  ModelConfig m;
  if (int st = copy_config(config, m))
    return st;
  auto *g = new (std::nothrow) llmi_qwen35_graph;
  if (!g)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "model: out of host memory");
  if (int st = build(m, tokens, past, capacity, logits_mode, *g)) {
    delete g;
    return st;
  }
  *out = g;
  return LLMI_HIP_OK;
}

const llmi_graph *llmi_qwen35_graph_view(const llmi_qwen35_graph *g) {
  return g ? &g->flat : nullptr;
}

size_t llmi_qwen35_graph_tensor_count(const llmi_qwen35_graph *g) {
  return g ? g->tensors.size() : 0;
}

const char *llmi_qwen35_graph_tensor(const llmi_qwen35_graph *g, size_t index) {
  return g && index < g->tensors.size() ? g->tensors[index].c_str() : nullptr;
}

void llmi_qwen35_graph_destroy(llmi_qwen35_graph *g) { delete g; }

int llmi_hip_model_open(const llmi_qwen35_config *config, const llmi_named_weight *weights,
                        size_t weight_count, uint64_t capacity, void *stream,
                        llmi_hip_model **out) {
  if (!out)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "model: null output");
  *out = nullptr;
  std::unique_ptr<llmi_hip_model> s(new (std::nothrow) llmi_hip_model);
  if (!s)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "model: out of host memory");
  if (int st = copy_config(config, s->cfg))
    return st;
  if (!capacity || capacity > std::min<uint64_t>(s->cfg.c.max_positions, UINT32_MAX))
    return fail(LLMI_HIP_INVALID_ARGUMENT, "Invalid session capacity");
  if (weight_count && !weights)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "model: null weight table");
  for (size_t i = 0; i < weight_count; ++i) {
    if (!weights[i].name || !weights[i].data)
      return fail(LLMI_HIP_INVALID_ARGUMENT, "model: weight %zu has no name or data", i);
    s->weights[weights[i].name] = llmi_weight{weights[i].data, weights[i].scales};
  }
  s->capacity = capacity;
  s->stream = static_cast<hipStream_t>(stream);
  // The state layout of every step, and every tensor the model reads
  // (MetalExecutor::initialize, MetalExecutor.mm:56-94).
  Graph g;
  if (int st = build(s->cfg, 1, 0, capacity, LLMI_LOGITS_NONE, g))
    return st;
  for (const llmi_graph_value &v : g.values) {
    if (v.kind != LLMI_GRAPH_WEIGHT)
      continue;
    const std::string &id = g.tensors[(size_t)v.weight];
    auto it = s->weights.find(id);
    if (it == s->weights.end())
      return fail(LLMI_HIP_INVALID_ARGUMENT, "model: missing tensor %s", id.c_str());
    if (v.element == LLMI_GRAPH_I8 && !it->second.scales)
      return fail(LLMI_HIP_INVALID_ARGUMENT, "model: int8 tensor %s has no scales", id.c_str());
  }
  s->layout = g.states;
  s->states.assign(g.states.size(), nullptr);
  for (size_t i = 0; i < g.states.size(); ++i)
    if (hipMalloc(&s->states[i], state_bytes(g.states[i])) != hipSuccess) {
      release(s.get());
      return fail(LLMI_HIP_INVALID_ARGUMENT, "model: cannot allocate state %zu (%zu bytes)",
                  i, state_bytes(g.states[i]));
    }
  if (hipMalloc(reinterpret_cast<void **>(&s->ids), capacity * sizeof(uint32_t)) !=
          hipSuccess ||
      hipMalloc(reinterpret_cast<void **>(&s->flag), sizeof(uint32_t)) != hipSuccess) {
    release(s.get());
    return fail(LLMI_HIP_INVALID_ARGUMENT, "model: cannot allocate step buffers");
  }
  if (hipError_t e = zero_states(s.get())) {
    release(s.get());
    return fail(LLMI_HIP_LAUNCH_FAILED, "model: cannot clear state: %s", hipGetErrorString(e));
  }
  *out = s.release();
  return LLMI_HIP_OK;
}

void llmi_hip_model_close(llmi_hip_model *s) {
  if (!s)
    return;
  (void)hipStreamSynchronize(s->stream);
  release(s);
  delete s;
}

void llmi_hip_model_reset(llmi_hip_model *s) {
  if (!s)
    return;
  if (zero_states(s) != hipSuccess) {
    s->invalid = true; // the state could not be cleared
    return;
  }
  s->past = 0;
  s->invalid = false;
  s->records.clear();
}

uint64_t llmi_hip_model_past(const llmi_hip_model *s) { return s ? s->past : 0; }
int llmi_hip_model_invalid(const llmi_hip_model *s) { return s ? s->invalid : 1; }
uint64_t llmi_hip_model_vocabulary(const llmi_hip_model *s) {
  return s ? s->cfg.c.vocabulary : 0;
}

int llmi_hip_model_step(llmi_hip_model *s, const uint32_t *ids, size_t count, int logits_mode,
                        float *logits, size_t logits_capacity,
                        llmi_hip_model_step_result *result) {
  if (!s)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "model: null session");
  if (s->invalid)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "Session is invalid after a failed GPU step");
  if (!count || count > s->capacity - s->past)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "Token chunk is empty or exceeds session capacity");
  if (!ids)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "model: null token IDs");
  for (size_t i = 0; i < count; ++i)
    if (ids[i] >= s->cfg.c.vocabulary)
      return fail(LLMI_HIP_INVALID_ARGUMENT, "Token ID is outside the vocabulary");
  Graph g;
  if (int st = build(s->cfg, count, s->past, s->capacity, logits_mode, g))
    return st;
  if (g.states.size() != s->layout.size() ||
      !std::equal(g.states.begin(), g.states.end(), s->layout.begin(), same_state))
    return fail(LLMI_HIP_INVALID_ARGUMENT, "Graph state layout changed within the session");
  PlanOwner plan;
  if (int st = lower(s, g, &plan.p))
    return st;
  uint64_t rows = 0, elements = 0;
  llmi_hip_plan_logits(plan.p, &rows, &elements);
  if (elements && (!logits || logits_capacity < elements))
    return fail(LLMI_HIP_INVALID_ARGUMENT, "model: logits need %llu floats",
                (unsigned long long)elements);
  if (int st = grow(&s->scratch, s->scratchBytes, llmi_hip_plan_scratch_bytes(plan.p),
                    s->stream, "scratch"))
    return st;
  if (int st = grow(reinterpret_cast<void **>(&s->logits), s->logitBytes, elements * 2,
                    s->stream, "logits"))
    return st;

  // From here on a failure may leave state written: the session goes invalid.
  std::vector<uint16_t> half(elements);
  uint32_t flag = 0;
  hipError_t e = hipMemcpyAsync(s->ids, ids, count * sizeof(uint32_t), hipMemcpyHostToDevice,
                                s->stream);
  if (e == hipSuccess)
    e = hipMemsetAsync(s->flag, 0, sizeof(uint32_t), s->stream);
  int st = e == hipSuccess ? LLMI_HIP_OK
                           : fail(LLMI_HIP_LAUNCH_FAILED, "model step: %s", hipGetErrorString(e));
  if (st == LLMI_HIP_OK)
    st = llmi_hip_plan_execute(plan.p, s->scratch, s->scratchBytes, s->states.data(),
                               s->states.size(), s->ids, elements ? s->logits : nullptr,
                               s->flag, s->stream);
  if (st == LLMI_HIP_OK && elements)
    e = hipMemcpyAsync(half.data(), s->logits, elements * 2, hipMemcpyDeviceToHost, s->stream);
  if (st == LLMI_HIP_OK && e == hipSuccess)
    e = hipMemcpyAsync(&flag, s->flag, sizeof(uint32_t), hipMemcpyDeviceToHost, s->stream);
  if (st == LLMI_HIP_OK && e == hipSuccess)
    e = hipStreamSynchronize(s->stream);
  if (st == LLMI_HIP_OK && e != hipSuccess)
    st = fail(LLMI_HIP_LAUNCH_FAILED, "model step: %s", hipGetErrorString(e));
  if (st == LLMI_HIP_OK && flag)
    st = fail(LLMI_HIP_LAUNCH_FAILED, "Non-finite activation during W8A8 quantization");
  if (st != LLMI_HIP_OK) {
    s->invalid = true;
    return LLMI_HIP_LAUNCH_FAILED;
  }
  for (uint64_t i = 0; i < elements; ++i)
    logits[i] = half_to_float(half[i]);
  s->past += count;
  const size_t n = llmi_hip_plan_dispatches(plan.p, nullptr, 0);
  s->records.resize(n);
  llmi_hip_plan_dispatches(plan.p, s->records.data(), n);
  if (result)
    *result = llmi_hip_model_step_result{s->past, rows, llmi_hip_plan_scratch_bytes(plan.p), n};
  return LLMI_HIP_OK;
}

size_t llmi_hip_model_dispatches(const llmi_hip_model *s, llmi_hip_dispatch *records,
                                 size_t cap) {
  if (!s)
    return 0;
  if (records)
    std::copy_n(s->records.begin(), std::min(cap, s->records.size()), records);
  return s->records.size();
}

size_t llmi_hip_model_state_count(const llmi_hip_model *s) { return s ? s->states.size() : 0; }

int llmi_hip_model_state(const llmi_hip_model *s, size_t index, llmi_graph_state *desc,
                         void **device, size_t *bytes) {
  if (!s || index >= s->states.size())
    return fail(LLMI_HIP_INVALID_ARGUMENT, "model: no state %zu", index);
  if (desc)
    *desc = s->layout[index];
  if (device)
    *device = s->states[index];
  if (bytes)
    *bytes = state_bytes(s->layout[index]);
  return LLMI_HIP_OK;
}

int llmi_hip_model_read_state(llmi_hip_model *s, size_t index, void *dst, size_t bytes) {
  if (!s || index >= s->states.size() || !dst)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "model: no state %zu or null destination", index);
  if (bytes != state_bytes(s->layout[index]))
    return fail(LLMI_HIP_INVALID_ARGUMENT, "model: state %zu holds %zu bytes", index,
                state_bytes(s->layout[index]));
  hipError_t e = hipMemcpyAsync(dst, s->states[index], bytes, hipMemcpyDefault, s->stream);
  if (e == hipSuccess)
    e = hipStreamSynchronize(s->stream);
  return e == hipSuccess ? LLMI_HIP_OK
                         : fail(LLMI_HIP_LAUNCH_FAILED, "model: %s", hipGetErrorString(e));
}

int llmi_hip_model_plan(const llmi_hip_model *s, uint64_t tokens, uint64_t past,
                        int logits_mode, llmi_hip_plan **out) {
  if (!s || !out)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "model: null argument");
  *out = nullptr;
  Graph g;
  if (int st = build(s->cfg, tokens, past, s->capacity, logits_mode, g))
    return st;
  return lower(s, g, out);
}

int llmi_hip_model_run(llmi_hip_model *s, const llmi_hip_plan *plan, const uint32_t *ids,
                       uint16_t *logits) {
  if (!s || !plan)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "model: null argument");
  if (s->invalid)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "Session is invalid after a failed GPU step");
  if (int st = grow(&s->scratch, s->scratchBytes, llmi_hip_plan_scratch_bytes(plan), s->stream,
                    "scratch"))
    return st;
  return llmi_hip_plan_execute(plan, s->scratch, s->scratchBytes, s->states.data(),
                               s->states.size(), ids, logits, s->flag, s->stream);
}

} // extern "C"
