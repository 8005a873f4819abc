// Launch functions of the gfx950 kernels. Each returns the hipError_t of
// its launch(es); shape checks happen in capi.cpp before any of these runs.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "llminfer_hip.h"

namespace llmi {

// ---------------------------------------------------------------- KvAppend
hipError_t launch_cache_append(const uint16_t *src, uint16_t *cache,
                               unsigned count, unsigned offset,
                               hipStream_t stream);
hipError_t launch_kv_append(const uint16_t *ksrc, const uint16_t *vsrc,
                            uint16_t *kcache, uint16_t *vcache, unsigned count,
                            unsigned offset, hipStream_t stream);

// ----------------------------------------------------------------- GQA
struct GqaShape {
  unsigned T, Hq, Hkv, D, P;
};

// Split-K decode (T <= 64). Workspace layout is owned by gqa_decode.hip;
// decode_workspace_bytes sizes it (0 when the launch needs no split merge).
// With knew/vnew non-null the launch also appends those T rows to the
// caches at row P (fused KvAppend); with them null the rows must already be
// in the caches.
bool decode_supported(const GqaShape &s);
size_t decode_workspace_bytes(const GqaShape &s);
unsigned decode_splits(const GqaShape &s);
unsigned decode_launches(const GqaShape &s); // 1, or 2 with a merge launch
hipError_t launch_gqa_decode(const uint16_t *q, uint16_t *k, uint16_t *v,
                             const uint16_t *knew, const uint16_t *vnew,
                             uint16_t *out, void *ws, const GqaShape &s,
                             hipStream_t stream);

// The attention block's row inputs around CausalGqa for the gated forms
// (normRope of q and k, the V append, the sigmoid output gate): the
// projected q rows [T][Hq][2D] (per head D query values, then D gate
// values), the new keys before their norm and the new values [T][Hkv][D],
// the norm weights [D] (the kernels form 1 + w), the rotary width and the
// norm epsilon, and pow(theta, 2i/rot) for i < rot/2. activated: the gate
// values are already fp16(logistic(.)) (the q projection's sigmoid-columns
// epilogue), so the output is fp16(gate * x) -- multiplyF16's bits.
struct GatedRows {
  const _Float16 *qproj = nullptr;
  const _Float16 *kproj = nullptr;
  const _Float16 *vnew = nullptr;
  const float *qw = nullptr, *kw = nullptr;
  unsigned rot = 0;
  float eps = 0.0f;
  unsigned activated = 0;
  float freqs[256] = {};
};

// The gated decode (T == 1, decode_supported, rot/2 a multiple of 8):
// normRope of q and of the new key (written to cache row P), the new V row
// appended, the split-K decode, and the output through the sigmoid gate --
// the bits of the standalone normRope, cacheAppend, decode and sigmoidMul.
bool decode_gated_supported(const GqaShape &s, unsigned rot);
hipError_t launch_gqa_decode_gated(uint16_t *k, uint16_t *v, uint16_t *out, void *ws,
                                   const GqaShape &s, const GatedRows &ga,
                                   hipStream_t stream);

// MFMA flash prefill.
bool prefill_supported(const GqaShape &s);
// The gated prefill: the query rows through normRope in the kernel, the
// output through the sigmoid gate (the keys must already be normRoped into
// the cache, the values appended).
bool prefill_gated_supported(const GqaShape &s, unsigned rot);
hipError_t launch_gqa_prefill_gated(const uint16_t *k, const uint16_t *v, uint16_t *out,
                                    const GqaShape &s, const GatedRows &ga,
                                    hipStream_t stream);
hipError_t launch_gqa_prefill(const uint16_t *q, const uint16_t *k,
                              const uint16_t *v, uint16_t *out,
                              const GqaShape &s, hipStream_t stream);

// Generic fallback for any head_dim <= 512 and any GQA ratio.
bool generic_supported(const GqaShape &s);
hipError_t launch_gqa_generic(const uint16_t *q, const uint16_t *k,
                              const uint16_t *v, uint16_t *out,
                              const GqaShape &s, hipStream_t stream);

// ------------------------------------------------------------- DeltaNet
struct DeltaShape {
  unsigned T, Hk, Dk, Hv, Dv;
};

bool delta_recurrent_supported(const DeltaShape &s);
// The same with fp16 q and k rows that the kernels L2-normalise themselves,
// bit for bit as l2NormF32 (factor rsqrt(sum + eps) * scale; qscale for q,
// 1 for k) before the update.
hipError_t launch_delta_recurrent_qk16(const uint16_t *q, const uint16_t *k,
                                       const uint16_t *v, const float *beta,
                                       const float *decay, float *state, uint16_t *out,
                                       float eps, float qscale, const DeltaShape &s,
                                       hipStream_t stream);
hipError_t launch_delta_chunked_qk16(const uint16_t *q, const uint16_t *k, const uint16_t *v,
                                     const float *beta, const float *decay, float *state,
                                     uint16_t *out, void *ws, float eps, float qscale,
                                     const DeltaShape &s, hipStream_t stream);
hipError_t launch_delta_recurrent(const float *q, const float *k,
                                  const uint16_t *v, const float *beta,
                                  const float *decay, float *state,
                                  uint16_t *out, const DeltaShape &s,
                                  hipStream_t stream);

// L2Norm -> DeltaUpdate -> gatedRmsNorm in one call (fp16 q/k, fp16 gate,
// fp32 norm weight of dv): the recurrent form with one workgroup per value
// head (T <= kRecNormMaxT, dv 64 or 128), and the chunked
// form whose scan normalises the head's rows at its end.
constexpr unsigned kRecNormMaxT = 32;
bool delta_recurrent_norm_supported(const DeltaShape &s);
hipError_t launch_delta_recurrent_gated_norm(const uint16_t *q, const uint16_t *k,
                                             const uint16_t *v, const float *beta,
                                             const float *decay, float *state,
                                             const uint16_t *gate, const float *nweight,
                                             uint16_t *out, float eps, float qscale,
                                             float neps, const DeltaShape &s,
                                             hipStream_t stream);
// The same with the fp32 activated gate, the normalised rows also quantized
// (32-wide groups of the flattened rows) into qout, scales and *invalid.
hipError_t launch_delta_recurrent_gated_norm_quantize(
    const uint16_t *q, const uint16_t *k, const uint16_t *v, const float *beta,
    const float *decay, float *state, const float *gate, const float *nweight, uint16_t *out,
    int8_t *qout, float *scales, unsigned *invalid, float eps, float qscale, float neps,
    const DeltaShape &s, hipStream_t stream);
// Whether the chunked form's norm scan grid fits on the device at once (its
// per-head arrival wait needs every workgroup resident).
bool delta_chunked_norm_resident(const DeltaShape &s);
hipError_t launch_delta_chunked_gated_norm(const uint16_t *q, const uint16_t *k,
                                           const uint16_t *v, const float *beta,
                                           const float *decay, float *state, const uint16_t *gate,
                                           const float *nweight, uint16_t *out, void *ws,
                                           float eps, float qscale, float neps,
                                           const DeltaShape &s, hipStream_t stream);
// The polls the norm scan's arrival wait makes before it gives up: sets the
// bound for later launches (0: give up at once); returns the previous bound.
unsigned delta_chunked_wait_limit(unsigned limit);
// After a launch_delta_chunked_gated_norm on `ws`: waits for `stream`, then
// reports whether any workgroup's arrival wait gave up.
hipError_t delta_chunked_wait_status(const void *ws, const DeltaShape &s, hipStream_t stream,
                                     bool *gave_up);

// Any-shape fallback, one thread per state column.
hipError_t launch_delta_generic(const float *q, const float *k,
                                const uint16_t *v, const float *beta,
                                const float *decay, float *state,
                                uint16_t *out, const DeltaShape &s,
                                hipStream_t stream);

bool delta_chunked_supported(const DeltaShape &s);
size_t delta_chunked_workspace_bytes(const DeltaShape &s);
hipError_t launch_delta_chunked(const float *q, const float *k,
                                const uint16_t *v, const float *beta,
                                const float *decay, float *state,
                                uint16_t *out, void *ws, const DeltaShape &s,
                                hipStream_t stream);

// ------------------------------------------------ norm, rope and the gate
// Rows r < rows of `D` halves at in + r * stride; output row out_row0 + r
// (dense, D halves); position past + r / heads. norm = false is partialRope
// (no normalisation, weight unused); rot = 0 is rmsNorm.
struct RopeShape {
  unsigned rows, heads, D, rot, stride, past, out_row0;
  float eps, theta;
  bool norm;
  unsigned rows_per_tile; // tile rows per wave (host tuning; 1..64)
};

bool norm_rope_tiled(const RopeShape &s, const void *in, const void *out);
// Rows wider than the tile's limit (a workgroup per row, the row in LDS).
bool norm_rope_wide_rows(const RopeShape &s);
hipError_t launch_norm_rope(const uint16_t *in, const float *w, uint16_t *out,
                            const RopeShape &s, hipStream_t stream);

bool sigmoid_mul_vectorised(unsigned count, const void *g, const void *x, const void *o);
hipError_t launch_sigmoid_mul(const uint16_t *gate, const uint16_t *in, uint16_t *out,
                              unsigned count, hipStream_t stream);

// ------------------------------------------------------ DeltaNet front end
bool causal_conv_supported(unsigned k);
hipError_t launch_causal_conv(const uint16_t *in, const uint16_t *w, uint16_t *hist,
                              uint16_t *out, unsigned T, unsigned C, unsigned k,
                              unsigned silu, hipStream_t stream);
bool l2_norm_tiled(unsigned width, const void *in, const void *out);
hipError_t launch_l2_norm(const uint16_t *in, float *out, unsigned rows, unsigned width,
                          float eps, float scale, hipStream_t stream);
// The LDS-tiled kernel (width a multiple of 8 up to 256, 16-byte aligned
// buffers); other shapes take a thread per row.
bool gated_rms_norm_tiled(unsigned width, const void *in, const void *gate, const void *out);
// The activated gated norm with the quantization of its rows in one launch
// (delta_front.hip): width a multiple of 32 on the tiled path.
bool gated_rms_norm_quantize_supported(unsigned width, const void *in, const void *gate,
                                       const void *out, const void *q);
hipError_t launch_gated_rms_norm_quantize(const uint16_t *in, const float *gate, const float *w,
                                          uint16_t *out, int8_t *q, float *scales,
                                          unsigned *invalid, unsigned rows, unsigned width,
                                          float eps, hipStream_t stream);
hipError_t launch_gated_rms_norm(const uint16_t *in, const void *gate, bool activated,
                                 const float *w, uint16_t *out, unsigned rows, unsigned width,
                                 float eps, hipStream_t stream);
hipError_t launch_delta_gates(const uint16_t *a, const uint16_t *b, const float *a_log,
                              const float *dt_bias, float *beta, float *decay,
                              unsigned rows, unsigned width, hipStream_t stream);

// -------------------------------------------------------- W8A8 projections
hipError_t launch_quantize_activation(const uint16_t *in, int8_t *q, float *scales,
                                      unsigned *invalid, unsigned rows, unsigned width,
                                      unsigned groups, hipStream_t stream);
struct W8Shape {
  unsigned outputWidth, firstRow, groups, rows, columns, epilogue, block;
};
const char *linear_w8a8_kernel(unsigned rows);
hipError_t launch_linear_w8a8(const int8_t *act, const float *as, const int8_t *w,
                              const uint16_t *ws, void *out, const void *aux, const float *bias,
                              const W8Shape &s, hipStream_t stream);
hipError_t launch_embedding_w8(const uint32_t *ids, const int8_t *w, const uint16_t *sc,
                               uint16_t *out, unsigned tokens, unsigned hidden, unsigned first,
                               unsigned count, unsigned groups, hipStream_t stream);
hipError_t launch_embedding(const uint32_t *ids, const uint16_t *w, uint16_t *out,
                            unsigned tokens, unsigned hidden, unsigned first, unsigned count,
                            hipStream_t stream);

// residualAdd -> rmsNorm -> quantizeActivation in one launch, a workgroup
// per row of up to kAddNormQuantizeMax halves (w8a8.hip); b null: no add.
constexpr unsigned kAddNormQuantizeMax = 8192;
// The same row's norm and quantization followed by up to kNormLinearMax
// W8A8 projections of it, rows == 1, width <= kNormLinearMaxWidth, one
// workgroup per 60 columns of a projection (w8a8.hip).
// A SwiGLU projection right after its multiplier's projection is computed
// by the same lanes (paired) up to kNormLinearPairedWidth.
constexpr unsigned kNormLinearMax = LLMI_HIP_NORM_LINEAR_MAX, kNormLinearMaxWidth = 4096;
constexpr unsigned kNormLinearPairedWidth = 2560;
constexpr unsigned kNormLinearCols = 60, kNormLinearMaxWgs = 4096;
inline unsigned norm_linear_workgroups(unsigned columns) {
  return (columns + kNormLinearCols - 1) / kNormLinearCols;
}
struct NormLinearProj {
  const int8_t *w;
  const uint16_t *ws;
  void *out;
  const void *aux;
  const float *bias;
  W8Shape shape;
  bool paired; // the next projection is this one's SwiGLU partner
  // the one-token kernel-4 convolution + SiLU the row passes through
  const uint16_t *cw = nullptr;
  uint16_t *ch = nullptr;
};
hipError_t launch_add_norm_linear(const uint16_t *a, const uint16_t *b, uint16_t *sum_out,
                                  const float *w, int8_t *q, float *scales, unsigned *invalid,
                                  unsigned width, float eps, const NormLinearProj *proj,
                                  unsigned count, hipStream_t stream);
hipError_t launch_add_norm_quantize(const uint16_t *a, const uint16_t *b, uint16_t *sum_out,
                                   const float *w, int8_t *q, float *scales, unsigned *invalid,
                                   unsigned rows, unsigned width, float eps, hipStream_t stream);

// residualAdd / swiGlu / siluF16 / multiplyF16, copyHalfView, linearF16
// (graph_ops.hip).
enum class ElementwiseKind { Add, SwiGlu, Silu, Multiply };
hipError_t launch_elementwise(ElementwiseKind kind, const uint16_t *a, const uint16_t *b,
                              uint16_t *out, unsigned count, hipStream_t stream);
hipError_t launch_copy_half_view(const uint16_t *src, uint16_t *out, const HalfViewParams &p,
                                 hipStream_t stream);
hipError_t launch_linear_f16(const uint16_t *in, const uint16_t *w, void *out, const void *aux,
                             const float *bias, const LinearParams &p, hipStream_t stream);

} // namespace llmi
