// C ABI of the HIP backend: validation, kernel selection, workspace sizing
// and status reporting. Declarations and contracts: include/llminfer_hip.h.
#include "llminfer_hip.h"
#include "capi_internal.hpp"
#include "kernels.hpp"
#include "rope_gate.hpp"

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

namespace llmi {

namespace {
thread_local char g_error[512] = "";
} // namespace

int fail(int status, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof g_error, fmt, ap);
  va_end(ap);
  return status;
}

int launched(hipError_t err, const char *what) {
  if (err == hipSuccess)
    return LLMI_HIP_OK;
  return fail(LLMI_HIP_LAUNCH_FAILED, "%s: %s", what, hipGetErrorString(err));
}

// Mirrors the reference lowering's 32-bit element-index limit
// (lib/Backend/Metal/MetalExecutionPlan.cpp:32-40).
static bool fits32(uint64_t a, uint64_t b, uint64_t c) {
  uint64_t ab = a * b;
  if (a && ab / a != b)
    return false;
  uint64_t abc = ab * c;
  if (ab && abc / ab != c)
    return false;
  return abc <= 0xffffffffull;
}

int check_gqa(const GqaParams &p) {
  if (p.tokens == 0 || p.queryHeads == 0 || p.kvHeads == 0 || p.headDim == 0)
    return fail(LLMI_HIP_INVALID_ARGUMENT,
                "CausalGqa: tokens, heads and head_dim must be positive");
  if (p.queryHeads % p.kvHeads)
    return fail(LLMI_HIP_INVALID_ARGUMENT,
                "CausalGqa: query heads %u not a multiple of KV heads %u",
                p.queryHeads, p.kvHeads);
  uint64_t rows = (uint64_t)p.past + p.tokens;
  if (!fits32(p.tokens, p.queryHeads, p.headDim) ||
      !fits32(rows, p.kvHeads, p.headDim))
    return fail(LLMI_HIP_INVALID_ARGUMENT,
                "CausalGqa: tensor exceeds the 32-bit index range");
  return LLMI_HIP_OK;
}

int check_delta(const GraphDeltaParams &p) {
  if (!p.tokens || !p.keyHeads || !p.keyDim || !p.valueHeads || !p.valueDim)
    return fail(LLMI_HIP_INVALID_ARGUMENT,
                "DeltaUpdate: every dimension must be positive");
  if (p.valueHeads % p.keyHeads)
    return fail(LLMI_HIP_INVALID_ARGUMENT,
                "DeltaUpdate: value heads %u not a multiple of key heads %u",
                p.valueHeads, p.keyHeads);
  if (!fits32(p.tokens, p.keyHeads, p.keyDim) ||
      !fits32(p.tokens, p.valueHeads, p.valueDim) ||
      !fits32(p.valueHeads, p.keyDim, p.valueDim))
    return fail(LLMI_HIP_INVALID_ARGUMENT,
                "DeltaUpdate: tensor exceeds the 32-bit index range");
  return LLMI_HIP_OK;
}

GqaKernel select_gqa(const GqaParams &p) {
  GqaShape s{p.tokens, p.queryHeads, p.kvHeads, p.headDim, p.past};
  if (p.tokens == 1 && decode_supported(s))
    return GqaKernel::Decode;
  if (p.tokens > 1 && prefill_supported(s))
    return GqaKernel::Prefill;
  if (generic_supported(s))
    return GqaKernel::Generic;
  return GqaKernel::None;
}

DeltaKernel select_delta(const GraphDeltaParams &p) {
  DeltaShape s{p.tokens, p.keyHeads, p.keyDim, p.valueHeads, p.valueDim};
  if (p.tokens > 1 && delta_chunked_supported(s))
    return DeltaKernel::Chunked;
  if (delta_recurrent_supported(s))
    return DeltaKernel::Recurrent;
  return DeltaKernel::Generic;
}

} // namespace llmi

using namespace llmi;

// normRope / rmsNorm / partialRope as one row shape. Rows per tile (one
// wave each): about 2048 tiles (two waves per SIMD on 256 CUs), but at least
// 8 rows once there are 4096 rows, since the sequential sum costs a tile the
// same whatever its row count, and 2 for a decode step's few rows, where the
// wave's latency is what counts (a sweep of 1..32 on MI355X: q 2048x16 rows
// best at 16, k 2048x4 at 4-8, decode 16 rows at 2).
RopeShape rope_shape(unsigned rows, unsigned heads, unsigned D, unsigned rot,
                     unsigned stride, unsigned past, unsigned out_row0, float eps,
                     float theta, bool norm) {
  unsigned rw = (rows + 2047) / 2048;
  unsigned lo = rows >= 4096 ? 8 : 2;
  rw = rw < lo ? lo : rw > 64 ? 64 : rw;
  return RopeShape{rows, heads, D, rot, stride, past, out_row0, eps, theta, norm, rw};
}

int check_rope(const char *what, uint64_t rows, unsigned heads, unsigned D,
               unsigned rot, uint64_t in_extent, uint64_t out_rows) {
  if (rows && heads == 0)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "%s: heads == 0", what);
  if (rot % 2 || rot > D)
    return fail(LLMI_HIP_INVALID_ARGUMENT,
                "%s: rotary width %u must be even and <= width %u", what, rot, D);
  if (!fits32(rows, in_extent, 1) || !fits32(out_rows, D, 1))
    return fail(LLMI_HIP_INVALID_ARGUMENT, "%s: exceeds the 32-bit index range", what);
  return LLMI_HIP_OK;
}

int rope_kernel_name_index(const RopeShape &s) {
  return norm_rope_tiled(s, nullptr, nullptr) ? 0 : norm_rope_wide_rows(s) ? 2 : 1;
}

static const char *rope_kernel_name(const RopeShape &s, const char *tile, const char *rows,
                                    const char *wide) {
  const int i = rope_kernel_name_index(s);
  return i == 0 ? tile : i == 2 ? wide : rows;
}

extern "C" {

int llmi_hip_norm_rope(const uint16_t *input, const float *weight, uint16_t *output,
                       RopeParams p, void *stream) {
  uint64_t rows = (uint64_t)p.tokens * p.heads;
  if (rows == 0 || p.headDim == 0)
    return LLMI_HIP_OK;
  if (!input || !weight || !output)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "normRope: null buffer");
  if (int st = check_rope("normRope", rows, p.heads, p.headDim, p.rotaryDim,
                          p.headStride > p.headDim ? p.headStride : p.headDim,
                          ((uint64_t)p.outputStart + p.tokens) * p.heads))
    return st;
  if ((uint64_t)p.past + p.tokens > 0xffffffffull)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "normRope: past + tokens overflows");
  RopeShape s = rope_shape((unsigned)rows, p.heads, p.headDim, p.rotaryDim, p.headStride,
                           p.past, p.outputStart * p.heads, p.epsilon, p.theta, true);
  return launched(launch_norm_rope(input, weight, output, s,
                                   static_cast<hipStream_t>(stream)),
                  "normRope");
}

int llmi_hip_rms_norm(const uint16_t *input, const float *weight, uint16_t *output,
                      RowParams p, void *stream) {
  if (p.rows == 0 || p.width == 0)
    return LLMI_HIP_OK;
  if (!input || !weight || !output)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "rmsNorm: null buffer");
  if (int st = check_rope("rmsNorm", p.rows, 1, p.width, 0, p.width, p.rows))
    return st;
  RopeShape s = rope_shape(p.rows, 1, p.width, 0, p.width, 0, 0, p.epsilon, 0.0f, true);
  return launched(launch_norm_rope(input, weight, output, s,
                                   static_cast<hipStream_t>(stream)),
                  "rmsNorm");
}

int llmi_hip_partial_rope(const uint16_t *input, uint16_t *output, PartialRopeParams p,
                          void *stream) {
  if (p.rows == 0 || p.width == 0)
    return LLMI_HIP_OK;
  if (!input || !output)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "partialRope: null buffer");
  if (int st = check_rope("partialRope", p.rows, p.heads, p.width, p.rotaryWidth,
                          p.width, p.rows))
    return st;
  if ((uint64_t)p.past + p.rows / p.heads > 0xffffffffull)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "partialRope: past + tokens overflows");
  RopeShape s = rope_shape(p.rows, p.heads, p.width, p.rotaryWidth, p.width, p.past, 0,
                           0.0f, p.theta, false);
  return launched(launch_norm_rope(input, nullptr, output, s,
                                   static_cast<hipStream_t>(stream)),
                  "partialRope");
}

int llmi_hip_sigmoid_mul(const uint16_t *gate, const uint16_t *input, uint16_t *output,
                         ElementParams p, void *stream) {
  if (p.count == 0)
    return LLMI_HIP_OK;
  if (!gate || !input || !output)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "sigmoidMul: null buffer");
  return launched(launch_sigmoid_mul(gate, input, output, p.count,
                                     static_cast<hipStream_t>(stream)),
                  "sigmoidMul");
}

int llmi_hip_causal_conv(const uint16_t *input, const uint16_t *weight, uint16_t *history,
                         uint16_t *output, ConvParams p, void *stream) {
  if (p.tokens == 0 || p.channels == 0)
    return LLMI_HIP_OK;
  if (!causal_conv_supported(p.kernelSize))
    return fail(LLMI_HIP_UNSUPPORTED, "causalConv: kernel size %u (1..8 supported)",
                p.kernelSize);
  if (!input || !weight || !output || (p.kernelSize > 1 && !history))
    return fail(LLMI_HIP_INVALID_ARGUMENT, "causalConv: null buffer");
  if (!fits32(p.tokens, p.channels, 1) || !fits32(p.channels, p.kernelSize, 1))
    return fail(LLMI_HIP_INVALID_ARGUMENT, "causalConv: exceeds the 32-bit index range");
  return launched(launch_causal_conv(input, weight, history, output, p.tokens, p.channels,
                                     p.kernelSize, p.applySilu ? 1u : 0u,
                                     static_cast<hipStream_t>(stream)),
                  "causalConv");
}

int llmi_hip_l2_norm(const uint16_t *input, float *output, L2Params p, void *stream) {
  if (p.rows == 0 || p.width == 0)
    return LLMI_HIP_OK;
  if (!input || !output)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "l2NormF32: null buffer");
  if (!fits32(p.rows, p.width, 1))
    return fail(LLMI_HIP_INVALID_ARGUMENT, "l2NormF32: exceeds the 32-bit index range");
  return launched(launch_l2_norm(input, output, p.rows, p.width, p.epsilon, p.scale,
                                 static_cast<hipStream_t>(stream)),
                  "l2NormF32");
}

int llmi_hip_delta_gates(const uint16_t *a, const uint16_t *b, const float *a_log,
                         const float *dt_bias, float *beta, float *decay, RowParams p,
                         void *stream) {
  if (p.rows == 0 || p.width == 0)
    return LLMI_HIP_OK;
  if (!a || !b || !a_log || !dt_bias || !beta || !decay)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "deltaGates: null buffer");
  if (!fits32(p.rows, p.width, 1))
    return fail(LLMI_HIP_INVALID_ARGUMENT, "deltaGates: exceeds the 32-bit index range");
  return launched(launch_delta_gates(a, b, a_log, dt_bias, beta, decay, p.rows, p.width,
                                     static_cast<hipStream_t>(stream)),
                  "deltaGates");
}

// ------------------------------------------------------ W8A8 projections

int llmi_hip_quantize_activation(const uint16_t *input, int8_t *quantized, float *scales,
                                 uint32_t *invalid, QuantizeParams p, void *stream) {
  if (p.rows == 0 || p.width == 0)
    return LLMI_HIP_OK;
  if (!input || !quantized || !scales)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "quantizeActivation: null buffer");
  if (p.groups != (p.width + 31) / 32)
    return fail(LLMI_HIP_INVALID_ARGUMENT,
                "quantizeActivation: %u groups for width %u (32-element groups: %u)",
                p.groups, p.width, (p.width + 31) / 32);
  if (!fits32(p.rows, p.groups, 32) || !fits32(p.rows, p.width, 1))
    return fail(LLMI_HIP_INVALID_ARGUMENT,
                "quantizeActivation: exceeds the 32-bit index range");
  if (!aligned16(quantized))
    return fail(LLMI_HIP_UNSUPPORTED, "quantizeActivation: quantized rows not 16-byte aligned");
  return launched(launch_quantize_activation(input, quantized, scales, invalid, p.rows, p.width,
                                             p.groups, static_cast<hipStream_t>(stream)),
                  "quantizeActivation");
}

static int check_linear_w8(const LinearW8Params &p) {
  if (p.epilogue > LLMI_LINEAR_DELTA_DECAY)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "linearW8A8: unknown epilogue %u", p.epilogue);
  if (p.epilogue == LLMI_LINEAR_SIGMOID_COLUMNS && p.epilogueBlock == 0)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "linearW8A8: sigmoid columns need a block width");
  if (p.groups == 0)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "linearW8A8: no groups");
  if ((uint64_t)p.firstRow + p.columns > p.outputWidth)
    return fail(LLMI_HIP_INVALID_ARGUMENT,
                "linearW8A8: columns %u from %u past the output width %u", p.columns,
                p.firstRow, p.outputWidth);
  if (!fits32(p.rows, p.groups, 32) || !fits32(p.columns, p.groups, 32) ||
      !fits32(p.rows, p.outputWidth, 1))
    return fail(LLMI_HIP_INVALID_ARGUMENT, "linearW8A8: exceeds the 32-bit index range");
  return LLMI_HIP_OK;
}

int llmi_hip_linear_w8a8(const int8_t *activation, const float *act_scales,
                         const int8_t *weight, const uint16_t *weight_scales, void *output,
                         const void *aux, const float *bias, LinearW8Params p, void *stream) {
  if (p.rows == 0 || p.columns == 0)
    return LLMI_HIP_OK;
  if (int rc = check_linear_w8(p))
    return rc;
  if (!activation || !act_scales || !weight || !weight_scales || !output)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "linearW8A8: null buffer");
  if (p.epilogue == LLMI_LINEAR_SILU_MUL && !aux)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "linearW8A8: SiluMul needs its multiplier (aux)");
  if (p.epilogue == LLMI_LINEAR_DELTA_DECAY && (!aux || !bias))
    return fail(LLMI_HIP_INVALID_ARGUMENT, "linearW8A8: the decay needs A_log (aux) and bias");
  if (!aligned16(activation) || !aligned16(weight))
    return fail(LLMI_HIP_UNSUPPORTED,
                "linearW8A8: activation and weight rows must be 16-byte aligned");
  const W8Shape s{p.outputWidth, p.firstRow, p.groups, p.rows, p.columns, p.epilogue,
                  p.epilogueBlock};
  return launched(launch_linear_w8a8(activation, act_scales, weight, weight_scales, output, aux,
                                     bias, s, static_cast<hipStream_t>(stream)),
                  linear_w8a8_kernel(p.rows));
}

int llmi_hip_embedding_w8(const uint32_t *ids, const int8_t *weight, const uint16_t *scales,
                          uint16_t *output, GroupedEmbedParams p, void *stream) {
  if (p.tokens == 0 || p.hidden == 0 || p.rowCount == 0)
    return LLMI_HIP_OK;
  if (!ids || !weight || !scales || !output)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "embeddingW8: null buffer");
  if (p.groups < (p.hidden + 31) / 32)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "embeddingW8: %u groups for hidden %u", p.groups,
                p.hidden);
  if (!fits32(p.tokens, p.hidden, 1) || !fits32(p.rowCount, p.groups, 32))
    return fail(LLMI_HIP_INVALID_ARGUMENT, "embeddingW8: exceeds the 32-bit index range");
  return launched(launch_embedding_w8(ids, weight, scales, output, p.tokens, p.hidden,
                                      p.firstRow, p.rowCount, p.groups,
                                      static_cast<hipStream_t>(stream)),
                  "embeddingW8");
}

int llmi_hip_embedding(const uint32_t *ids, const uint16_t *weight, uint16_t *output,
                       EmbedParams p, void *stream) {
  if (p.tokens == 0 || p.hidden == 0 || p.rowCount == 0)
    return LLMI_HIP_OK;
  if (!ids || !weight || !output)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "embedding: null buffer");
  if (!fits32(p.tokens, p.hidden, 1) || !fits32(p.rowCount, p.hidden, 1))
    return fail(LLMI_HIP_INVALID_ARGUMENT, "embedding: exceeds the 32-bit index range");
  return launched(launch_embedding(ids, weight, output, p.tokens, p.hidden, p.firstRow,
                                   p.rowCount, static_cast<hipStream_t>(stream)),
                  "embedding");
}

static int elementwise(ElementwiseKind kind, const char *name, const uint16_t *a,
                       const uint16_t *b, uint16_t *out, ElementParams p, void *stream) {
  if (p.count == 0)
    return LLMI_HIP_OK;
  if (!a || !out || (kind != ElementwiseKind::Silu && !b))
    return fail(LLMI_HIP_INVALID_ARGUMENT, "%s: null buffer", name);
  return launched(launch_elementwise(kind, a, b, out, p.count, static_cast<hipStream_t>(stream)),
                  name);
}

int llmi_hip_residual_add(const uint16_t *a, const uint16_t *b, uint16_t *out, ElementParams p,
                          void *stream) {
  return elementwise(ElementwiseKind::Add, "residualAdd", a, b, out, p, stream);
}

int llmi_hip_swiglu(const uint16_t *gate, const uint16_t *up, uint16_t *out, ElementParams p,
                    void *stream) {
  return elementwise(ElementwiseKind::SwiGlu, "swiGlu", gate, up, out, p, stream);
}

int llmi_hip_silu(const uint16_t *in, uint16_t *out, ElementParams p, void *stream) {
  return elementwise(ElementwiseKind::Silu, "siluF16", in, nullptr, out, p, stream);
}

int llmi_hip_multiply(const uint16_t *a, const uint16_t *b, uint16_t *out, ElementParams p,
                      void *stream) {
  return elementwise(ElementwiseKind::Multiply, "multiplyF16", a, b, out, p, stream);
}

static int check_add_norm_quantize(const RowParams &p) {
  if (p.width > kAddNormQuantizeMax)
    return fail(LLMI_HIP_UNSUPPORTED, "addRmsNormQuantize: width %u (at most %u)", p.width,
                kAddNormQuantizeMax);
  if (!fits32(p.rows, (p.width + 31) / 32 * 32, 1))
    return fail(LLMI_HIP_INVALID_ARGUMENT, "addRmsNormQuantize: exceeds the 32-bit index range");
  return LLMI_HIP_OK;
}

int llmi_hip_add_rms_norm_quantize(const uint16_t *a, const uint16_t *b, uint16_t *sum_out,
                                   const float *weight, int8_t *q, float *scales,
                                   uint32_t *invalid, RowParams p, void *stream) {
  if (p.rows == 0 || p.width == 0)
    return LLMI_HIP_OK;
  if (int rc = check_add_norm_quantize(p))
    return rc;
  if (!a || !weight || !q || !scales || (b && !sum_out))
    return fail(LLMI_HIP_INVALID_ARGUMENT, "addRmsNormQuantize: null buffer");
  if (!aligned16(q))
    return fail(LLMI_HIP_UNSUPPORTED, "addRmsNormQuantize: quantized rows not 16-byte aligned");
  return launched(launch_add_norm_quantize(a, b, sum_out, weight, q, scales, invalid, p.rows,
                                           p.width, p.epsilon, static_cast<hipStream_t>(stream)),
                  b ? "addRmsNormQuantize" : "rmsNormQuantize");
}

static int check_norm_linear(const NormLinearParams &p) {
  const RowParams &n = p.norm;
  if (n.rows != 1 || n.width == 0 || n.width > kNormLinearMaxWidth)
    return fail(LLMI_HIP_UNSUPPORTED, "addRmsNormLinearW8A8: one row of at most %u (%u x %u)",
                kNormLinearMaxWidth, n.rows, n.width);
  if (p.count == 0 || p.count > kNormLinearMax)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "addRmsNormLinearW8A8: %u projections (1 to %u)",
                p.count, kNormLinearMax);
  const unsigned groups = (n.width + 31) / 32;
  unsigned wgs = 0;
  for (unsigned k = 0; k < p.count; ++k) {
    const LinearW8Params &l = p.linear[k];
    if (int rc = check_linear_w8(l))
      return rc;
    if (l.rows != 1 || l.groups != groups || l.columns == 0)
      return fail(LLMI_HIP_INVALID_ARGUMENT,
                  "addRmsNormLinearW8A8: projection %u takes %u rows of %u groups and %u "
                  "columns (one row of %u groups, at least one column)",
                  k, l.rows, l.groups, l.columns, groups);
    wgs += norm_linear_workgroups(l.columns);
  }
  if (wgs > kNormLinearMaxWgs)
    return fail(LLMI_HIP_UNSUPPORTED, "addRmsNormLinearW8A8: %u workgroups (at most %u)", wgs,
                kNormLinearMaxWgs);
  return LLMI_HIP_OK;
}

int llmi_hip_add_rms_norm_linear_w8a8(const uint16_t *a, const uint16_t *b, uint16_t *sum_out,
                                      const float *weight, int8_t *q, float *scales,
                                      uint32_t *invalid,
                                      const llmi_hip_norm_projection *projections,
                                      NormLinearParams p, void *stream) {
  if (int rc = check_norm_linear(p))
    return rc;
  if (!a || !weight || !projections || (b && !sum_out))
    return fail(LLMI_HIP_INVALID_ARGUMENT, "addRmsNormLinearW8A8: null buffer");
  if (q && !aligned16(q))
    return fail(LLMI_HIP_UNSUPPORTED, "addRmsNormLinearW8A8: quantized row not 16-byte aligned");
  NormLinearProj proj[kNormLinearMax];
  for (unsigned k = 0; k < p.count; ++k) {
    const llmi_hip_norm_projection &x = projections[k];
    const LinearW8Params &l = p.linear[k];
    if (!x.weight || !x.weight_scales || !x.output)
      return fail(LLMI_HIP_INVALID_ARGUMENT, "addRmsNormLinearW8A8: projection %u: null buffer",
                  k);
    if (!aligned16(x.weight))
      return fail(LLMI_HIP_UNSUPPORTED,
                  "addRmsNormLinearW8A8: projection %u: weight rows not 16-byte aligned", k);
    bool mate = false; // computed by the lanes of projection k - 1
    if (l.epilogue == LLMI_LINEAR_SILU_MUL) {
      if (!x.aux)
        return fail(LLMI_HIP_INVALID_ARGUMENT,
                    "addRmsNormLinearW8A8: projection %u: SiluMul needs its multiplier (aux)", k);
      mate = k > 0 && x.aux == projections[k - 1].output;
      // (projection k - 1 has no epilogue, so it is nobody's mate itself)
      if (mate && (p.norm.width > kNormLinearPairedWidth ||
                   p.linear[k - 1].epilogue != LLMI_LINEAR_NONE ||
                   p.linear[k - 1].columns != l.columns))
        return fail(LLMI_HIP_UNSUPPORTED,
                    "addRmsNormLinearW8A8: projection %u: a SwiGLU multiplier computed in the "
                    "call must be the previous projection's output, with no epilogue, the same "
                    "columns and width <= %u",
                    k, kNormLinearPairedWidth);
      for (unsigned j = 0; j < p.count; ++j)
        if (j + 1 != k && projections[j].output == x.aux)
          return fail(LLMI_HIP_UNSUPPORTED,
                      "addRmsNormLinearW8A8: projection %u: its SwiGLU multiplier is another "
                      "projection's output",
                      k);
    }
    if (l.epilogue == LLMI_LINEAR_DELTA_DECAY && (!x.aux || !x.bias))
      return fail(LLMI_HIP_INVALID_ARGUMENT,
                  "addRmsNormLinearW8A8: projection %u: the decay needs A_log (aux) and bias", k);
    if (!x.conv_weight != !x.conv_history)
      return fail(LLMI_HIP_INVALID_ARGUMENT,
                  "addRmsNormLinearW8A8: projection %u: a convolution needs its weight and its "
                  "history",
                  k);
    if (x.conv_weight && (l.epilogue != LLMI_LINEAR_NONE || l.firstRow != 0 ||
                          l.columns != l.outputWidth))
      return fail(LLMI_HIP_UNSUPPORTED,
                  "addRmsNormLinearW8A8: projection %u: a convolution takes the whole row of a "
                  "projection with no epilogue",
                  k);
    proj[k] = {x.weight, x.weight_scales, x.output, x.aux, x.bias,
               W8Shape{l.outputWidth, l.firstRow, l.groups, l.rows, l.columns, l.epilogue,
                       l.epilogueBlock},
               false, x.conv_weight, x.conv_history};
    if (mate) {
      if (proj[k - 1].cw)
        return fail(LLMI_HIP_UNSUPPORTED,
                    "addRmsNormLinearW8A8: projection %u: a SwiGLU multiplier has no "
                    "convolution",
                    k);
      proj[k - 1].paired = true;
    }
  }
  return launched(launch_add_norm_linear(a, b, sum_out, weight, q, scales, invalid, p.norm.width,
                                         p.norm.epsilon, proj, p.count,
                                         static_cast<hipStream_t>(stream)),
                  b ? "addRmsNormLinearW8A8" : "rmsNormLinearW8A8");
}

int llmi_hip_gated_rms_norm_activated_quantize(const uint16_t *x, const float *gate,
                                               const float *weight, uint16_t *out, int8_t *q,
                                               float *scales, uint32_t *invalid, RowParams p,
                                               void *stream) {
  if (p.rows == 0 || p.width == 0)
    return LLMI_HIP_OK;
  if (!x || !gate || !weight || !out || !q || !scales)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "gatedRmsNormQuantize: null buffer");
  if (!fits32(p.rows, p.width, 1))
    return fail(LLMI_HIP_INVALID_ARGUMENT, "gatedRmsNormQuantize: exceeds the 32-bit index range");
  if (!gated_rms_norm_quantize_supported(p.width, x, gate, out, q))
    return fail(LLMI_HIP_UNSUPPORTED,
                "gatedRmsNormQuantize: width %u (a multiple of 32, at most 256) or an unaligned "
                "buffer",
                p.width);
  return launched(launch_gated_rms_norm_quantize(x, gate, weight, out, q, scales, invalid, p.rows,
                                                 p.width, p.epsilon,
                                                 static_cast<hipStream_t>(stream)),
                  "gatedRmsNormQuantize");
}

static int check_view(const HalfViewParams &p) {
  uint64_t last = p.offset;
  for (int d = 0; d < 3; ++d) {
    if (p.dims[d] == 0)
      return fail(LLMI_HIP_INVALID_ARGUMENT, "copyHalfView: zero extent on axis %d", d);
    last += (uint64_t)(p.dims[d] - 1) * p.strides[d];
  }
  if ((uint64_t)p.dims[0] * p.dims[1] * p.dims[2] != p.count)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "copyHalfView: count %u is not the view's extent",
                p.count);
  if (last > UINT32_MAX)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "copyHalfView: exceeds the 32-bit index range");
  return LLMI_HIP_OK;
}

int llmi_hip_copy_half_view(const uint16_t *src, uint16_t *out, HalfViewParams p, void *stream) {
  if (p.count == 0)
    return LLMI_HIP_OK;
  if (int rc = check_view(p))
    return rc;
  if (!src || !out)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "copyHalfView: null buffer");
  return launched(launch_copy_half_view(src, out, p, static_cast<hipStream_t>(stream)),
                  "copyHalfView");
}

static int check_linear_f16(const LinearParams &p) {
  if (p.epilogue > LLMI_LINEAR_DELTA_DECAY)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "linearF16: unknown epilogue %u", p.epilogue);
  if (p.epilogue == LLMI_LINEAR_SIGMOID_COLUMNS && p.epilogueBlock == 0)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "linearF16: sigmoid columns need a block width");
  if (p.inputWidth == 0)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "linearF16: zero input width");
  if ((uint64_t)p.firstRow + p.rowCount > p.outputWidth)
    return fail(LLMI_HIP_INVALID_ARGUMENT,
                "linearF16: columns %u from %u past the output width %u", p.rowCount,
                p.firstRow, p.outputWidth);
  if (!fits32(p.tokens, p.inputWidth, 1) || !fits32(p.rowCount, p.inputWidth, 1) ||
      !fits32(p.tokens, p.outputWidth, 1))
    return fail(LLMI_HIP_INVALID_ARGUMENT, "linearF16: exceeds the 32-bit index range");
  return LLMI_HIP_OK;
}

int llmi_hip_linear_f16(const uint16_t *input, const uint16_t *weight, void *output,
                        const void *aux, const float *bias, LinearParams p, void *stream) {
  if (p.tokens == 0 || p.rowCount == 0)
    return LLMI_HIP_OK;
  if (int rc = check_linear_f16(p))
    return rc;
  if (!input || !weight || !output)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "linearF16: null buffer");
  if (p.epilogue == LLMI_LINEAR_SILU_MUL && !aux)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "linearF16: SiluMul needs its multiplier (aux)");
  if (p.epilogue == LLMI_LINEAR_DELTA_DECAY && (!aux || !bias))
    return fail(LLMI_HIP_INVALID_ARGUMENT, "linearF16: the decay needs A_log (aux) and bias");
  return launched(launch_linear_f16(input, weight, output, aux, bias, p,
                                    static_cast<hipStream_t>(stream)),
                  "linearF16");
}

static int gated_norm(const uint16_t *input, const void *gate, bool activated,
                      const float *weight, uint16_t *output, RowParams p, void *stream) {
  if (p.rows == 0 || p.width == 0)
    return LLMI_HIP_OK;
  if (!input || !gate || !weight || !output)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "gatedRmsNorm: null buffer");
  if (!fits32(p.rows, p.width, 1))
    return fail(LLMI_HIP_INVALID_ARGUMENT, "gatedRmsNorm: exceeds the 32-bit index range");
  return launched(launch_gated_rms_norm(input, gate, activated, weight, output, p.rows,
                                        p.width, p.epsilon, static_cast<hipStream_t>(stream)),
                  "gatedRmsNorm");
}

int llmi_hip_gated_rms_norm(const uint16_t *input, const uint16_t *gate, const float *weight,
                            uint16_t *output, RowParams p, void *stream) {
  return gated_norm(input, gate, false, weight, output, p, stream);
}

int llmi_hip_gated_rms_norm_activated(const uint16_t *input, const float *gate,
                                      const float *weight, uint16_t *output, RowParams p,
                                      void *stream) {
  return gated_norm(input, gate, true, weight, output, p, stream);
}

int llmi_hip_cache_append(const uint16_t *src, uint16_t *cache, CacheParams p,
                          void *stream) {
  if (p.count && (!src || !cache))
    return fail(LLMI_HIP_INVALID_ARGUMENT, "cacheAppend: null buffer");
  if ((uint64_t)p.offset + p.count > 0xffffffffull)
    return fail(LLMI_HIP_INVALID_ARGUMENT,
                "cacheAppend: offset + count exceeds the 32-bit index range");
  return launched(launch_cache_append(src, cache, p.count, p.offset,
                                      static_cast<hipStream_t>(stream)),
                  "cacheAppend");
}

int llmi_hip_kv_append(const uint16_t *k_src, const uint16_t *v_src,
                       uint16_t *k_cache, uint16_t *v_cache, CacheParams p,
                       void *stream) {
  if (p.count && (!k_src || !v_src || !k_cache || !v_cache))
    return fail(LLMI_HIP_INVALID_ARGUMENT, "KvAppend: null buffer");
  if ((uint64_t)p.offset + p.count > 0xffffffffull)
    return fail(LLMI_HIP_INVALID_ARGUMENT,
                "KvAppend: offset + count exceeds the 32-bit index range");
  return launched(launch_kv_append(k_src, v_src, k_cache, v_cache, p.count,
                                   p.offset, static_cast<hipStream_t>(stream)),
                  "kvAppend");
}

size_t llmi_hip_gqa_workspace_bytes(GqaParams p) {
  if (check_gqa(p) != LLMI_HIP_OK)
    return 0;
  if (select_gqa(p) == GqaKernel::Decode)
    return decode_workspace_bytes(
        {p.tokens, p.queryHeads, p.kvHeads, p.headDim, p.past});
  return 0;
}

} // extern "C"

namespace llmi {

// CausalGqa with an optional fused KvAppend (k_new/v_new non-null).
int run_gqa(const uint16_t *q, const uint16_t *k_new, const uint16_t *v_new,
            uint16_t *k_cache, uint16_t *v_cache, uint16_t *out,
            const GqaParams &p, void *workspace, size_t workspace_bytes,
            void *stream) {
  if (int st = check_gqa(p))
    return st;
  if (!q || !k_cache || !v_cache || !out)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "CausalGqa: null buffer");
  const bool fused = k_new || v_new;
  if (fused && (!k_new || !v_new))
    return fail(LLMI_HIP_INVALID_ARGUMENT, "KvAppend: null buffer");
  GqaShape s{p.tokens, p.queryHeads, p.kvHeads, p.headDim, p.past};
  hipStream_t st = static_cast<hipStream_t>(stream);
  GqaKernel kind = select_gqa(p);
  if (kind == GqaKernel::None)
    return fail(LLMI_HIP_UNSUPPORTED, "CausalGqa: head_dim %u is not supported",
                p.headDim);
  if (kind == GqaKernel::Decode) {
    size_t need = decode_workspace_bytes(s);
    if (need && (!workspace || workspace_bytes < need))
      return fail(LLMI_HIP_WORKSPACE,
                  "CausalGqa: decode needs a %zu-byte workspace, got %zu",
                  need, workspace ? workspace_bytes : (size_t)0);
    return launched(launch_gqa_decode(q, k_cache, v_cache, k_new, v_new, out,
                                      workspace, s, st),
                    "gqaDecodeSplitK");
  }
  if (fused) {
    unsigned row = p.kvHeads * p.headDim;
    int r = launched(launch_kv_append(k_new, v_new, k_cache, v_cache,
                                      p.tokens * row, p.past * row, st),
                     "kvAppend");
    if (r != LLMI_HIP_OK)
      return r;
  }
  if (kind == GqaKernel::Prefill)
    return launched(launch_gqa_prefill(q, k_cache, v_cache, out, s, st),
                    "gqaPrefillMfma");
  return launched(launch_gqa_generic(q, k_cache, v_cache, out, s, st),
                  "gqaGeneric");
}

} // namespace llmi

extern "C" {

int llmi_hip_causal_gqa(const uint16_t *q, const uint16_t *k_cache,
                        const uint16_t *v_cache, uint16_t *out, GqaParams p,
                        void *workspace, size_t workspace_bytes, void *stream) {
  // The caches are only read on this path; the kernels take them non-const
  // because the fused variant writes the new rows.
  return run_gqa(q, nullptr, nullptr, const_cast<uint16_t *>(k_cache),
                 const_cast<uint16_t *>(v_cache), out, p, workspace,
                 workspace_bytes, stream);
}

int llmi_hip_kv_append_causal_gqa(const uint16_t *q, const uint16_t *k_new,
                                  const uint16_t *v_new, uint16_t *k_cache,
                                  uint16_t *v_cache, uint16_t *out, GqaParams p,
                                  void *workspace, size_t workspace_bytes,
                                  void *stream) {
  if (!k_new || !v_new)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "KvAppend: null buffer");
  return run_gqa(q, k_new, v_new, k_cache, v_cache, out, p, workspace,
                 workspace_bytes, stream);
}

static int gated_attention(const uint16_t *q_proj, const uint16_t *k_proj,
                           const uint16_t *v_new, const float *q_weight, const float *k_weight,
                           uint16_t *k_cache, uint16_t *v_cache, uint16_t *out, GqaParams p,
                           unsigned rotary_dim, float epsilon, float theta, void *workspace,
                           size_t workspace_bytes, bool activated, void *stream) {
  if (int st = check_gqa(p))
    return st;
  if (!q_proj || !k_proj || !v_new || !q_weight || !k_weight || !k_cache || !v_cache || !out)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "gated attention: null buffer");
  if (rotary_dim % 2 || rotary_dim > p.headDim)
    return fail(LLMI_HIP_INVALID_ARGUMENT,
                "gated attention: rotary width %u must be even and <= head_dim %u",
                rotary_dim, p.headDim);
  if (!fits32((uint64_t)p.tokens * p.queryHeads, 2 * p.headDim, 1))
    return fail(LLMI_HIP_INVALID_ARGUMENT, "gated attention: exceeds the 32-bit index range");
  GqaShape s{p.tokens, p.queryHeads, p.kvHeads, p.headDim, p.past};
  hipStream_t st = static_cast<hipStream_t>(stream);
  GatedRows ga;
  ga.qproj = reinterpret_cast<const _Float16 *>(q_proj);
  ga.kproj = reinterpret_cast<const _Float16 *>(k_proj);
  ga.vnew = reinterpret_cast<const _Float16 *>(v_new);
  ga.qw = q_weight;
  ga.kw = k_weight;
  ga.rot = rotary_dim;
  ga.eps = epsilon;
  ga.activated = activated ? 1u : 0u;
  const unsigned half = rotary_dim / 2;
  if (half > 256)
    return fail(LLMI_HIP_UNSUPPORTED, "gated attention: rotary width %u", rotary_dim);
  memcpy(ga.freqs, host_freqs(theta, rotary_dim).v, sizeof(float) * half);
  if (decode_gated_supported(s, rotary_dim)) {
    size_t need = decode_workspace_bytes(s);
    if (need && (!workspace || workspace_bytes < need))
      return fail(LLMI_HIP_WORKSPACE,
                  "gated attention: decode needs a %zu-byte workspace, got %zu", need,
                  workspace ? workspace_bytes : (size_t)0);
    return launched(launch_gqa_decode_gated(k_cache, v_cache, out, workspace, s, ga, st),
                    "gqaDecodeGated");
  }
  if (p.tokens > 1 && prefill_gated_supported(s, rotary_dim)) {
    const unsigned row = p.kvHeads * p.headDim;
    RopeShape ks = rope_shape(p.tokens * p.kvHeads, p.kvHeads, p.headDim, rotary_dim,
                              p.headDim, p.past, p.past * p.kvHeads, epsilon, theta, true);
    int r = launched(launch_norm_rope(k_proj, k_weight, k_cache, ks, st), "normRope");
    if (r == LLMI_HIP_OK)
      r = launched(launch_cache_append(v_new, v_cache, p.tokens * row, p.past * row, st),
                   "cacheAppend");
    if (r == LLMI_HIP_OK)
      r = launched(launch_gqa_prefill_gated(k_cache, v_cache, out, s, ga, st),
                   "gqaPrefillGated");
    return r;
  }
  return fail(LLMI_HIP_UNSUPPORTED,
              "gated attention: no fused kernel for T %u, heads %u/%u, head_dim %u, rotary %u",
              p.tokens, p.queryHeads, p.kvHeads, p.headDim, rotary_dim);
}

int llmi_hip_gated_attention(const uint16_t *q_proj, const uint16_t *k_proj,
                             const uint16_t *v_new, const float *q_weight,
                             const float *k_weight, uint16_t *k_cache, uint16_t *v_cache,
                             uint16_t *out, GqaParams p, unsigned rotary_dim, float epsilon,
                             float theta, void *workspace, size_t workspace_bytes,
                             void *stream) {
  return gated_attention(q_proj, k_proj, v_new, q_weight, k_weight, k_cache, v_cache, out, p,
                         rotary_dim, epsilon, theta, workspace, workspace_bytes, false, stream);
}

int llmi_hip_gated_attention_activated(const uint16_t *q_proj, const uint16_t *k_proj,
                                       const uint16_t *v_new, const float *q_weight,
                                       const float *k_weight, uint16_t *k_cache,
                                       uint16_t *v_cache, uint16_t *out, GqaParams p,
                                       unsigned rotary_dim, float epsilon, float theta,
                                       void *workspace, size_t workspace_bytes, void *stream) {
  return gated_attention(q_proj, k_proj, v_new, q_weight, k_weight, k_cache, v_cache, out, p,
                         rotary_dim, epsilon, theta, workspace, workspace_bytes, true, stream);
}

size_t llmi_hip_delta_workspace_bytes(GraphDeltaParams p) {
  if (check_delta(p) != LLMI_HIP_OK)
    return 0;
  if (select_delta(p) == DeltaKernel::Chunked)
    return delta_chunked_workspace_bytes(
        {p.tokens, p.keyHeads, p.keyDim, p.valueHeads, p.valueDim});
  return 0;
}

int llmi_hip_delta_update(const float *q, const float *k, const uint16_t *v,
                          const float *beta, const float *decay, float *state,
                          uint16_t *out, GraphDeltaParams p, void *workspace,
                          size_t workspace_bytes, void *stream) {
  if (int st = check_delta(p))
    return st;
  if (!q || !k || !v || !beta || !decay || !state || !out)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "DeltaUpdate: null buffer");
  DeltaShape s{p.tokens, p.keyHeads, p.keyDim, p.valueHeads, p.valueDim};
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (select_delta(p)) {
  case DeltaKernel::Chunked: {
    size_t need = delta_chunked_workspace_bytes(s);
    if (need && (!workspace || workspace_bytes < need))
      return fail(LLMI_HIP_WORKSPACE,
                  "DeltaUpdate: chunked form needs a %zu-byte workspace", need);
    return launched(launch_delta_chunked(q, k, v, beta, decay, state, out,
                                         workspace, s, st),
                    "deltaChunkedWy");
  }
  case DeltaKernel::Recurrent:
    return launched(
        launch_delta_recurrent(q, k, v, beta, decay, state, out, s, st),
        "deltaRecurrent");
  case DeltaKernel::Generic:
    return launched(launch_delta_generic(q, k, v, beta, decay, state, out, s, st),
                    "deltaGeneric");
  }
  return fail(LLMI_HIP_UNSUPPORTED, "DeltaUpdate: unsupported shape");
}

int llmi_hip_l2_norm_delta_update(const uint16_t *q, const uint16_t *k, const uint16_t *v,
                                  const float *beta, const float *decay, float *state,
                                  uint16_t *out, GraphDeltaParams p, float epsilon,
                                  float q_scale, void *workspace, size_t workspace_bytes,
                                  void *stream) {
  if (int st = check_delta(p))
    return st;
  if (!q || !k || !v || !beta || !decay || !state || !out)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "L2Norm+DeltaUpdate: null buffer");
  DeltaShape s{p.tokens, p.keyHeads, p.keyDim, p.valueHeads, p.valueDim};
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (select_delta(p)) {
  case DeltaKernel::Chunked: {
    size_t need = delta_chunked_workspace_bytes(s);
    if (need && (!workspace || workspace_bytes < need))
      return fail(LLMI_HIP_WORKSPACE,
                  "L2Norm+DeltaUpdate: chunked form needs a %zu-byte workspace", need);
    return launched(launch_delta_chunked_qk16(q, k, v, beta, decay, state, out, workspace,
                                              epsilon, q_scale, s, st),
                    "deltaChunkedWy");
  }
  case DeltaKernel::Recurrent:
    return launched(launch_delta_recurrent_qk16(q, k, v, beta, decay, state, out, epsilon,
                                                q_scale, s, st),
                    "deltaRecurrent");
  case DeltaKernel::Generic:
    break;
  }
  return fail(LLMI_HIP_UNSUPPORTED,
              "L2Norm+DeltaUpdate: dk %u, dv %u have no fused kernel (dk 64 or 128, dv a "
              "multiple of 16)",
              p.keyDim, p.valueDim);
}

int llmi_hip_l2_norm_delta_gated_norm(const uint16_t *q, const uint16_t *k, const uint16_t *v,
                                      const float *beta, const float *decay, float *state,
                                      const uint16_t *gate, const float *norm_weight,
                                      uint16_t *out, GraphDeltaParams p, float qk_epsilon,
                                      float q_scale, float norm_epsilon, void *workspace,
                                      size_t workspace_bytes, void *stream) {
  if (int st = check_delta(p))
    return st;
  if (!q || !k || !v || !beta || !decay || !state || !gate || !norm_weight || !out)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "L2Norm+DeltaUpdate+GatedRmsNorm: null buffer");
  DeltaShape s{p.tokens, p.keyHeads, p.keyDim, p.valueHeads, p.valueDim};
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (select_delta(p) == DeltaKernel::Chunked) {
    // The scan's norm reads and writes 16-byte row pieces of out and gate.
    if ((reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(gate)) & 15u)
      return fail(LLMI_HIP_UNSUPPORTED,
                  "L2Norm+DeltaUpdate+GatedRmsNorm: out and gate must be 16-byte aligned");
    size_t need = delta_chunked_workspace_bytes(s);
    if (!workspace || workspace_bytes < need)
      return fail(LLMI_HIP_WORKSPACE,
                  "L2Norm+DeltaUpdate+GatedRmsNorm: chunked form needs a %zu-byte workspace",
                  need);
    if (!delta_chunked_norm_resident(s))
      return fail(LLMI_HIP_UNSUPPORTED,
                  "L2Norm+DeltaUpdate+GatedRmsNorm: %u x %u scan workgroups do not fit on the "
                  "device at once",
                  p.valueHeads, p.valueDim / 16);
    return launched(launch_delta_chunked_gated_norm(q, k, v, beta, decay, state, gate,
                                                    norm_weight, out, workspace, qk_epsilon,
                                                    q_scale, norm_epsilon, s, st),
                    "deltaChunkedWy+gatedRmsNorm");
  }
  if (delta_recurrent_norm_supported(s))
    return launched(launch_delta_recurrent_gated_norm(q, k, v, beta, decay, state, gate,
                                                      norm_weight, out, qk_epsilon, q_scale,
                                                      norm_epsilon, s, st),
                    "deltaRecurrent+gatedRmsNorm");
  return fail(LLMI_HIP_UNSUPPORTED,
              "L2Norm+DeltaUpdate+GatedRmsNorm: T %u, dk %u, dv %u have no fused kernel "
              "(chunked: dk 128, T >= 32; recurrent: dk 64 or 128, dv 64 or 128, T <= %u)",
              p.tokens, p.keyDim, p.valueDim, kRecNormMaxT);
}

int llmi_hip_l2_norm_delta_gated_norm_status(const void *workspace, size_t workspace_bytes,
                                             GraphDeltaParams p, void *stream) {
  if (int st = check_delta(p))
    return st;
  // Only the chunked form waits for other workgroups.
  if (select_delta(p) != DeltaKernel::Chunked)
    return LLMI_HIP_OK;
  DeltaShape s{p.tokens, p.keyHeads, p.keyDim, p.valueHeads, p.valueDim};
  if (!workspace || workspace_bytes < delta_chunked_workspace_bytes(s))
    return fail(LLMI_HIP_WORKSPACE, "GatedRmsNorm status: workspace smaller than the call's");
  bool gave_up = false;
  if (int st = launched(delta_chunked_wait_status(workspace, s, static_cast<hipStream_t>(stream),
                                                  &gave_up),
                        "GatedRmsNorm status"))
    return st;
  if (gave_up)
    return fail(LLMI_HIP_LAUNCH_FAILED,
                "L2Norm+DeltaUpdate+GatedRmsNorm: the scan's arrival wait gave up; the "
                "normalised rows are not trustworthy");
  return LLMI_HIP_OK;
}

int llmi_hip_l2_norm_delta_gated_norm_activated_quantize(
    const uint16_t *q, const uint16_t *k, const uint16_t *v, const float *beta,
    const float *decay, float *state, const float *gate, const float *norm_weight,
    uint16_t *out, int8_t *quantized, float *scales, uint32_t *invalid, GraphDeltaParams p,
    float qk_epsilon, float q_scale, float norm_epsilon, void *stream) {
  if (int st = check_delta(p))
    return st;
  if (!q || !k || !v || !beta || !decay || !state || !gate || !norm_weight || !out ||
      !quantized || !scales)
    return fail(LLMI_HIP_INVALID_ARGUMENT,
                "L2Norm+DeltaUpdate+GatedRmsNormQuantize: null buffer");
  DeltaShape s{p.tokens, p.keyHeads, p.keyDim, p.valueHeads, p.valueDim};
  if (!delta_recurrent_norm_supported(s))
    return fail(LLMI_HIP_UNSUPPORTED,
                "L2Norm+DeltaUpdate+GatedRmsNormQuantize: T %u, dk %u, dv %u have no fused "
                "kernel (dk 64 or 128, dv 64 or 128, T <= %u)",
                p.tokens, p.keyDim, p.valueDim, kRecNormMaxT);
  // The norm writes 16-byte pieces of out and 8-byte pieces of quantized.
  if (!aligned16(out) || !aligned16(quantized))
    return fail(LLMI_HIP_UNSUPPORTED,
                "L2Norm+DeltaUpdate+GatedRmsNormQuantize: out and quantized must be 16-byte "
                "aligned");
  return launched(launch_delta_recurrent_gated_norm_quantize(
                      q, k, v, beta, decay, state, gate, norm_weight, out, quantized, scales,
                      invalid, qk_epsilon, q_scale, norm_epsilon, s,
                      static_cast<hipStream_t>(stream)),
                  "deltaRecurrent+gatedRmsNormQuantize");
}

unsigned llmi_hip_set_arrival_wait_limit(unsigned polls) {
  return delta_chunked_wait_limit(polls);
}

int llmi_hip_workspace_init(void *workspace, size_t bytes, void *stream) {
  if (!bytes)
    return LLMI_HIP_OK;
  if (!workspace)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "workspace_init: null workspace");
  return launched(hipMemsetAsync(workspace, 0, bytes,
                                 static_cast<hipStream_t>(stream)),
                  "workspace_init");
}

unsigned llmi_hip_dispatch_count(int op, const void *params) {
  if (!params)
    return 0;
  switch (op) {
  case LLMI_HIP_OP_KV_APPEND:
    return 1;
  case LLMI_HIP_OP_CAUSAL_GQA: {
    const GqaParams &p = *static_cast<const GqaParams *>(params);
    if (check_gqa(p) || select_gqa(p) == GqaKernel::None)
      return 0;
    if (select_gqa(p) == GqaKernel::Decode)
      return decode_launches({p.tokens, p.queryHeads, p.kvHeads, p.headDim, p.past});
    return 1;
  }
  case LLMI_HIP_OP_KV_APPEND_CAUSAL_GQA: {
    const GqaParams &p = *static_cast<const GqaParams *>(params);
    if (check_gqa(p))
      return 0;
    switch (select_gqa(p)) {
    case GqaKernel::Decode:
      return decode_launches({p.tokens, p.queryHeads, p.kvHeads, p.headDim, p.past});
    case GqaKernel::None:
      return 0;
    default:
      return 2;
    }
  }
  case LLMI_HIP_OP_DELTA_UPDATE: {
    const GraphDeltaParams &p = *static_cast<const GraphDeltaParams *>(params);
    if (check_delta(p))
      return 0;
    return select_delta(p) == DeltaKernel::Chunked ? delta_chunked_dispatches() : 1;
  }
  case LLMI_HIP_OP_NORM_ROPE: {
    const RopeParams &p = *static_cast<const RopeParams *>(params);
    return p.tokens && p.heads && p.headDim ? 1 : 0;
  }
  case LLMI_HIP_OP_RMS_NORM: {
    const RowParams &p = *static_cast<const RowParams *>(params);
    return p.rows && p.width ? 1 : 0;
  }
  case LLMI_HIP_OP_PARTIAL_ROPE: {
    const PartialRopeParams &p = *static_cast<const PartialRopeParams *>(params);
    return p.rows && p.width ? 1 : 0;
  }
  case LLMI_HIP_OP_SIGMOID_MUL:
    return static_cast<const ElementParams *>(params)->count ? 1 : 0;
  case LLMI_HIP_OP_CAUSAL_CONV: {
    const ConvParams &p = *static_cast<const ConvParams *>(params);
    return p.tokens && p.channels && causal_conv_supported(p.kernelSize) ? 1 : 0;
  }
  case LLMI_HIP_OP_L2_NORM: {
    const L2Params &p = *static_cast<const L2Params *>(params);
    return p.rows && p.width ? 1 : 0;
  }
  case LLMI_HIP_OP_QUANTIZE_ACTIVATION: {
    const QuantizeParams &p = *static_cast<const QuantizeParams *>(params);
    return p.rows && p.width && p.groups == (p.width + 31) / 32 ? 1 : 0;
  }
  case LLMI_HIP_OP_LINEAR_W8A8: {
    const LinearW8Params &p = *static_cast<const LinearW8Params *>(params);
    return p.rows && p.columns && check_linear_w8(p) == LLMI_HIP_OK ? 1 : 0;
  }
  case LLMI_HIP_OP_EMBEDDING_W8: {
    const GroupedEmbedParams &p = *static_cast<const GroupedEmbedParams *>(params);
    return p.tokens && p.hidden && p.rowCount && p.groups >= (p.hidden + 31) / 32 ? 1 : 0;
  }
  case LLMI_HIP_OP_EMBEDDING: {
    const EmbedParams &p = *static_cast<const EmbedParams *>(params);
    return p.tokens && p.hidden && p.rowCount ? 1 : 0;
  }
  case LLMI_HIP_OP_RESIDUAL_ADD:
  case LLMI_HIP_OP_SWIGLU:
  case LLMI_HIP_OP_SILU:
  case LLMI_HIP_OP_MULTIPLY:
    return static_cast<const ElementParams *>(params)->count ? 1 : 0;
  case LLMI_HIP_OP_COPY_HALF_VIEW: {
    const HalfViewParams &p = *static_cast<const HalfViewParams *>(params);
    return p.count && check_view(p) == LLMI_HIP_OK ? 1 : 0;
  }
  case LLMI_HIP_OP_ADD_RMS_NORM_QUANTIZE: {
    const RowParams &p = *static_cast<const RowParams *>(params);
    return p.rows && p.width && check_add_norm_quantize(p) == LLMI_HIP_OK ? 1 : 0;
  }
  case LLMI_HIP_OP_ADD_RMS_NORM_LINEAR_W8A8:
    return check_norm_linear(*static_cast<const NormLinearParams *>(params)) == LLMI_HIP_OK ? 1
                                                                                          : 0;
  case LLMI_HIP_OP_LINEAR_F16: {
    const LinearParams &p = *static_cast<const LinearParams *>(params);
    return p.tokens && p.rowCount && check_linear_f16(p) == LLMI_HIP_OK ? 1 : 0;
  }
  case LLMI_HIP_OP_DELTA_GATES: {
    const RowParams &p = *static_cast<const RowParams *>(params);
    return p.rows && p.width ? 1 : 0;
  }
  case LLMI_HIP_OP_GATED_RMS_NORM: {
    const RowParams &p = *static_cast<const RowParams *>(params);
    return p.rows && p.width ? 1 : 0;
  }
  case LLMI_HIP_OP_GATED_ATTENTION: {
    // Launches for a rotary width the kernels take (a multiple of 16).
    const GqaParams &p = *static_cast<const GqaParams *>(params);
    if (check_gqa(p))
      return 0;
    GqaShape s{p.tokens, p.queryHeads, p.kvHeads, p.headDim, p.past};
    if (decode_gated_supported(s, 16))
      return decode_launches(s);
    return p.tokens > 1 && prefill_gated_supported(s, 16) ? 3 : 0;
  }
  }
  return 0;
}

const char *llmi_hip_kernel_name(int op, const void *params, unsigned index) {
  if (index >= llmi_hip_dispatch_count(op, params))
    return nullptr;
  switch (op) {
  case LLMI_HIP_OP_KV_APPEND:
    return "kvAppend";
  case LLMI_HIP_OP_KV_APPEND_CAUSAL_GQA:
    if (select_gqa(*static_cast<const GqaParams *>(params)) != GqaKernel::Decode)
      return index == 0 ? "kvAppend"
                        : llmi_hip_kernel_name(LLMI_HIP_OP_CAUSAL_GQA, params, 0);
    return llmi_hip_kernel_name(LLMI_HIP_OP_CAUSAL_GQA, params, index);
  case LLMI_HIP_OP_CAUSAL_GQA:
    switch (select_gqa(*static_cast<const GqaParams *>(params))) {
    case GqaKernel::Decode:
      return index == 0 ? "gqaDecodeSplitK" : "gqaDecodeMerge";
    case GqaKernel::Prefill:
      return "gqaPrefillMfma";
    case GqaKernel::Generic:
      return "gqaGeneric";
    case GqaKernel::None:
      return nullptr;
    }
    return nullptr;
  case LLMI_HIP_OP_DELTA_UPDATE:
    switch (select_delta(*static_cast<const GraphDeltaParams *>(params))) {
    case DeltaKernel::Chunked:
      return delta_chunked_kernel_name(index);
    case DeltaKernel::Recurrent:
      return "deltaRecurrent";
    case DeltaKernel::Generic:
      return "deltaGeneric";
    }
    return nullptr;
  // The tile kernels need 16-byte aligned buffers as well; these names
  // assume them (torch allocations are).
  case LLMI_HIP_OP_NORM_ROPE: {
    const RopeParams &p = *static_cast<const RopeParams *>(params);
    RopeShape s = rope_shape(p.tokens * p.heads, p.heads, p.headDim, p.rotaryDim,
                             p.headStride, p.past, 0, 0, 0, true);
    return rope_kernel_name(s, "normRopeTile", "normRopeRows", "normRopeWide");
  }
  case LLMI_HIP_OP_RMS_NORM: {
    const RowParams &p = *static_cast<const RowParams *>(params);
    RopeShape s = rope_shape(p.rows, 1, p.width, 0, p.width, 0, 0, 0, 0, true);
    return rope_kernel_name(s, "normRopeTile", "normRopeRows", "normRopeWide");
  }
  case LLMI_HIP_OP_PARTIAL_ROPE: {
    const PartialRopeParams &p = *static_cast<const PartialRopeParams *>(params);
    RopeShape s = rope_shape(p.rows, p.heads, p.width, p.rotaryWidth, p.width, 0, 0, 0,
                             0, false);
    return rope_kernel_name(s, "partialRopeTile", "partialRopeRows", "partialRopeWide");
  }
  case LLMI_HIP_OP_CAUSAL_CONV:
    return "causalConv";
  case LLMI_HIP_OP_L2_NORM:
    return l2_norm_tiled(static_cast<const L2Params *>(params)->width, nullptr, nullptr)
               ? "l2NormTile"
               : "l2NormRows";
  case LLMI_HIP_OP_DELTA_GATES:
    return "deltaGates";
  case LLMI_HIP_OP_QUANTIZE_ACTIVATION:
    return "quantizeActivation";
  case LLMI_HIP_OP_LINEAR_W8A8:
    return linear_w8a8_kernel(static_cast<const LinearW8Params *>(params)->rows);
  case LLMI_HIP_OP_EMBEDDING_W8:
    return "embeddingW8";
  case LLMI_HIP_OP_EMBEDDING:
    return "embedding";
  case LLMI_HIP_OP_RESIDUAL_ADD:
    return "residualAdd";
  case LLMI_HIP_OP_SWIGLU:
    return "swiGlu";
  case LLMI_HIP_OP_SILU:
    return "siluF16";
  case LLMI_HIP_OP_MULTIPLY:
    return "multiplyF16";
  case LLMI_HIP_OP_COPY_HALF_VIEW:
    return "copyHalfView";
  case LLMI_HIP_OP_LINEAR_F16:
    return "linearF16";
  case LLMI_HIP_OP_ADD_RMS_NORM_QUANTIZE:
    return "addRmsNormQuantize";
  case LLMI_HIP_OP_ADD_RMS_NORM_LINEAR_W8A8:
    return "addRmsNormLinearW8A8";
  case LLMI_HIP_OP_GATED_RMS_NORM: {
    const unsigned width = static_cast<const RowParams *>(params)->width;
    return width % 8 == 0 && width <= 256 ? "gatedRmsNormTile" : "gatedRmsNormRows";
  }
  case LLMI_HIP_OP_SIGMOID_MUL:
    return sigmoid_mul_vectorised(static_cast<const ElementParams *>(params)->count,
                                  nullptr, nullptr, nullptr)
               ? "sigmoidMulVec"
               : "sigmoidMulScalar";
  case LLMI_HIP_OP_GATED_ATTENTION:
    if (static_cast<const GqaParams *>(params)->tokens == 1)
      return index == 0 ? "gqaDecodeGated" : "gqaDecodeMergeGated";
    return index == 0 ? "normRopeTile" : index == 1 ? "cacheAppend" : "gqaPrefillGated";
  }
  return nullptr;
}

const char *llmi_hip_status_string(int status) {
  switch (status) {
  case LLMI_HIP_OK:
    return "ok";
  case LLMI_HIP_INVALID_ARGUMENT:
    return "invalid argument";
  case LLMI_HIP_UNSUPPORTED:
    return "unsupported";
  case LLMI_HIP_WORKSPACE:
    return "workspace missing or too small";
  case LLMI_HIP_LAUNCH_FAILED:
    return "launch failed";
  case LLMI_HIP_NO_DEVICE:
    return "no device";
  }
  return "unknown status";
}

const char *llmi_hip_last_error(void) { return g_error; }

const char *llmi_hip_build_info(void) {
  return "llminfer-hip 0.1 gfx950";
}

} // extern "C"
