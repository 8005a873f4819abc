/*
 * llminfer HIP backend: C ABI of the attention / linear-attention hot path.
 *
 * Drop-in replacement, on AMD Instinct MI355X (gfx950), for the Metal
 * dispatches the reference's lowering emits for three GraphIR ops:
 *
 *   KvAppend    -> cacheAppend x2           lib/Backend/Metal/MetalExecutionPlan.cpp:516-523
 *   CausalGqa   -> gqaFlashAttention (T>1)  lib/Backend/Metal/MetalExecutionPlan.cpp:528-534
 *                  gqaScores/gqaSoftmax/gqaValue (T==1)  :536-548
 *   DeltaUpdate -> graphDeltaUpdate         lib/Backend/Metal/MetalExecutionPlan.cpp:663-676
 *
 * The parameter structs are byte-identical to the reference's kernel
 * parameter structs (all fields 32-bit unsigned), so a lowering that fills
 * them for Metal fills them for this backend unchanged.
 *
 * Conventions (mirroring lib/Backend/Metal/MetalExecutionPlan.h:36-39 and
 * include/llminfer/Support/Result.h:12-59):
 *   - Every pointer is a device pointer owned by the caller and borrowed for
 *     the duration of the call. Work is enqueued on `stream` (a hipStream_t,
 *     NULL = the default stream) in order; nothing synchronises the host.
 *   - Return value 0 (LLMI_HIP_OK) means enqueued. A nonzero status before
 *     any launch (INVALID_ARGUMENT, UNSUPPORTED, WORKSPACE) leaves every
 *     buffer untouched ("submitted = false"); LLMI_HIP_LAUNCH_FAILED means a
 *     launch was attempted, so state buffers may be partially written and a
 *     session must become invalid until reset (MetalExecutor.mm:283-298).
 *   - llmi_hip_last_error() returns a per-thread message for the last
 *     nonzero status.
 *   - Calls that share a workspace must not overlap (same stream is fine).
 */
#ifndef LLMINFER_HIP_H
#define LLMINFER_HIP_H

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__)
#define LLMI_HIP_API __attribute__((visibility("default")))
#else
#define LLMI_HIP_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* lib/Backend/Metal/Kernels/ReferenceParams.h:49-51 */
typedef struct CacheParams {
  unsigned count, offset;
} CacheParams;

/* lib/Backend/Metal/Kernels/ReferenceParams.h:53-55 */
typedef struct GqaParams {
  unsigned tokens, queryHeads, kvHeads, headDim, past;
} GqaParams;

/* lib/Backend/Metal/Kernels/GraphParams.h:50-52 */
typedef struct GraphDeltaParams {
  unsigned tokens, keyHeads, keyDim, valueHeads, valueDim;
} GraphDeltaParams;

/* lib/Backend/Metal/Kernels/ReferenceParams.h:23-26 */
typedef struct RowParams {
  unsigned rows, width;
  float epsilon;
} RowParams;

/* lib/Backend/Metal/Kernels/ReferenceParams.h:28-30 */
typedef struct ElementParams {
  unsigned count;
} ElementParams;

/* lib/Backend/Metal/Kernels/ReferenceParams.h:44-47 */
typedef struct RopeParams {
  unsigned tokens, heads, headDim, rotaryDim, headStride, past, outputStart;
  float epsilon, theta;
} RopeParams;

/* lib/Backend/Metal/Kernels/GraphParams.h:35-38 */
typedef struct PartialRopeParams {
  unsigned rows, heads, width, rotaryWidth, past;
  float theta;
} PartialRopeParams;

/* lib/Backend/Metal/Kernels/ReferenceParams.h:32-34 */
typedef struct ConvParams {
  unsigned tokens, channels, kernelSize, applySilu;
} ConvParams;

/* lib/Backend/Metal/Kernels/GraphParams.h:30-33 */
typedef struct L2Params {
  unsigned rows, width;
  float epsilon, scale;
} L2Params;

/* lib/Backend/Metal/Kernels/GraphParams.h:12-14 */
typedef struct QuantizeParams {
  unsigned rows, width, groups;
} QuantizeParams;

/* lib/Backend/Metal/Kernels/GraphParams.h:25-28 (epilogue: LinearEpilogue
 * below; epilogueBlock: the column block of LLMI_LINEAR_SIGMOID_COLUMNS) */
typedef struct LinearW8Params {
  unsigned outputWidth, firstRow, groups, rows, columns;
  unsigned epilogue, epilogueBlock;
} LinearW8Params;

/* lib/Backend/Metal/Kernels/GraphParams.h:8-10 */
typedef struct GroupedEmbedParams {
  unsigned tokens, hidden, firstRow, rowCount, groups;
} GroupedEmbedParams;

/* lib/Backend/Metal/Kernels/ReferenceParams.h:4-6 */
typedef struct EmbedParams {
  unsigned tokens, hidden, firstRow, rowCount;
} EmbedParams;

/* lib/Backend/Metal/Kernels/GraphParams.h:4-6: a view of at most three
 * dimensions (outermost first), strides and offset in elements */
typedef struct HalfViewParams {
  unsigned count, offset, dims[3], strides[3];
} HalfViewParams;

/* lib/Backend/Metal/Kernels/ReferenceParams.h:18-21 (rowCount: output
 * columns this call computes, from firstRow) */
typedef struct LinearParams {
  unsigned tokens, inputWidth, outputWidth, firstRow, rowCount;
  unsigned epilogue, epilogueBlock;
} LinearParams;

/* LinearEpilogue, lib/Backend/Metal/Kernels/ReferenceParams.h:8-16 */
enum llmi_linear_epilogue {
  LLMI_LINEAR_NONE = 0,
  LLMI_LINEAR_SILU = 1,
  LLMI_LINEAR_SILU_MUL = 2,
  LLMI_LINEAR_SIGMOID_COLUMNS = 3,
  LLMI_LINEAR_SILU_F32 = 4,
  LLMI_LINEAR_DELTA_BETA = 5,
  LLMI_LINEAR_DELTA_DECAY = 6
};

enum llmi_hip_status {
  LLMI_HIP_OK = 0,
  LLMI_HIP_INVALID_ARGUMENT = 1, /* bad shape/pointer; nothing launched */
  LLMI_HIP_UNSUPPORTED = 2,      /* valid op, no kernel for it; nothing launched */
  LLMI_HIP_WORKSPACE = 3,        /* workspace missing or too small; nothing launched */
  LLMI_HIP_LAUNCH_FAILED = 4,    /* a launch failed; buffers may be partially written */
  LLMI_HIP_NO_DEVICE = 5         /* no usable gfx950 device; nothing launched */
};

enum llmi_hip_op {
  LLMI_HIP_OP_KV_APPEND = 0,
  LLMI_HIP_OP_CAUSAL_GQA = 1,
  LLMI_HIP_OP_DELTA_UPDATE = 2,
  LLMI_HIP_OP_KV_APPEND_CAUSAL_GQA = 3, /* the fused pair; params: GqaParams */
  LLMI_HIP_OP_NORM_ROPE = 4,            /* params: RopeParams */
  LLMI_HIP_OP_RMS_NORM = 5,             /* params: RowParams */
  LLMI_HIP_OP_PARTIAL_ROPE = 6,         /* params: PartialRopeParams */
  LLMI_HIP_OP_SIGMOID_MUL = 7,          /* params: ElementParams */
  LLMI_HIP_OP_CAUSAL_CONV = 8,          /* params: ConvParams */
  LLMI_HIP_OP_L2_NORM = 9,              /* params: L2Params */
  LLMI_HIP_OP_DELTA_GATES = 10,         /* params: RowParams (rows = tokens, width = heads) */
  LLMI_HIP_OP_GATED_RMS_NORM = 11,      /* params: RowParams */
  LLMI_HIP_OP_GATED_ATTENTION = 12,     /* params: GqaParams */
  LLMI_HIP_OP_QUANTIZE_ACTIVATION = 13, /* params: QuantizeParams */
  LLMI_HIP_OP_LINEAR_W8A8 = 14,         /* params: LinearW8Params */
  LLMI_HIP_OP_EMBEDDING_W8 = 15,        /* params: GroupedEmbedParams */
  LLMI_HIP_OP_EMBEDDING = 16,           /* params: EmbedParams */
  LLMI_HIP_OP_RESIDUAL_ADD = 17,        /* params: ElementParams */
  LLMI_HIP_OP_SWIGLU = 18,              /* params: ElementParams */
  LLMI_HIP_OP_SILU = 19,                /* params: ElementParams */
  LLMI_HIP_OP_MULTIPLY = 20,            /* params: ElementParams */
  LLMI_HIP_OP_COPY_HALF_VIEW = 21,      /* params: HalfViewParams */
  LLMI_HIP_OP_LINEAR_F16 = 22,          /* params: LinearParams */
  LLMI_HIP_OP_ADD_RMS_NORM_QUANTIZE = 23, /* params: RowParams */
  LLMI_HIP_OP_ADD_RMS_NORM_LINEAR_W8A8 = 24 /* params: NormLinearParams */
};

/* ---------------------------------------------------------------- KvAppend
 * cacheAppend (lib/Backend/Metal/Kernels/Reference.metal:295-301):
 * cache[p.offset + i] = src[i] for i < p.count, fp16 elements. The
 * reference issues it once for K and once for V with
 * offset = past * kvHeads * headDim (MetalExecutionPlan.cpp:516-523). */
LLMI_HIP_API int llmi_hip_cache_append(const uint16_t *src, uint16_t *cache, CacheParams p,
                          void *stream);

/* Both halves of KvAppend in one launch: k_src -> k_cache and
 * v_src -> v_cache with the same CacheParams. Same result as two
 * llmi_hip_cache_append calls. */
LLMI_HIP_API int llmi_hip_kv_append(const uint16_t *k_src, const uint16_t *v_src,
                       uint16_t *k_cache, uint16_t *v_cache, CacheParams p,
                       void *stream);

/* ------------------------------------------------- norms, rope, the gate
 * The row work on either side of CausalGqa in the attention block
 * (Qwen35ModelBuilder.cpp:175-197; MetalReferenceGraph.mm:307-330). Results
 * equal the reference kernels' expressions evaluated in IEEE fp32 in their
 * order (sequential fma sum of squares; 1/sqrt for rsqrt; pow, cos, sin and
 * exp correctly rounded to fp32), bit for bit. fp16 buffers; weights fp32.
 *
 * normRope (Reference.metal:271-293, dispatched by
 * MetalReferenceGraph.mm:315-326): for row r < tokens * heads, the headDim
 * halves at input + r * headStride are RMS-normalised with (1 + weight),
 * rounded to fp16, and pairs (i, i + rotaryDim/2), i < rotaryDim/2, are
 * rotated by (past + r / heads) / theta^(2i / rotaryDim); the row is
 * written at output + (outputStart * heads + r) * headDim. With
 * outputStart = past and output = the key cache this is the K path with its
 * cache append. output may equal input when headStride == headDim and
 * outputStart == 0 (each row is read before it is written); other overlaps
 * are undefined. rotaryDim must be even and <= headDim. */
LLMI_HIP_API int llmi_hip_norm_rope(const uint16_t *input, const float *weight,
                                    uint16_t *output, RopeParams p, void *stream);

/* rmsNorm (Reference.metal:105-117; MetalExecutionPlan.cpp:579-596):
 * output[r][i] = fp16(input[r][i] * rsqrt(mean(input[r]^2) + eps) *
 * (1 + weight[i])), rows x width, dense. In place allowed. */
LLMI_HIP_API int llmi_hip_rms_norm(const uint16_t *input, const float *weight,
                                   uint16_t *output, RowParams p, void *stream);

/* partialRope (Graph.metal:111-129; MetalExecutionPlan.cpp:628-637): rows of
 * width halves, dense; the first rotaryWidth dims rotated as in normRope at
 * position past + row / heads, the rest copied. In place allowed. */
LLMI_HIP_API int llmi_hip_partial_rope(const uint16_t *input, uint16_t *output,
                                       PartialRopeParams p, void *stream);

/* sigmoidMul (Graph.metal:78-85; MetalExecutionPlan.cpp:609-620):
 * output[i] = fp16(fp16(1 / (1 + exp(-gate[i]))) * input[i]), i < count. */
LLMI_HIP_API int llmi_hip_sigmoid_mul(const uint16_t *gate, const uint16_t *input,
                                      uint16_t *output, ElementParams p, void *stream);

/* ------------------------------------------------------ DeltaNet front end
 * The DeltaNet layer's ops ahead of DeltaUpdate (Qwen35ModelBuilder.cpp:
 * 146-160; lowered at MetalExecutionPlan.cpp:597-603, 639-662). Results equal
 * the reference kernels' fp32 expressions bit for bit, with exp and log
 * correctly rounded to fp32.
 *
 * causalConv (Reference.metal:137-161): input, output [tokens][channels]
 * fp16; weight [channels][kernelSize] fp16; history [channels][kernelSize-1]
 * fp16, read and updated in place (the last kernelSize-1 inputs of the
 * sequence). applySilu != 0 applies fp16(silu(fp16(acc))). kernelSize 1..8;
 * history may be null when kernelSize == 1. */
LLMI_HIP_API int llmi_hip_causal_conv(const uint16_t *input, const uint16_t *weight,
                                      uint16_t *history, uint16_t *output, ConvParams p,
                                      void *stream);

/* l2NormF32 (Graph.metal:96-109): output[r][i] = input[r][i] *
 * (rsqrt(sum_i input[r][i]^2 + epsilon) * scale), fp16 in, fp32 out, rows x
 * width dense. */
LLMI_HIP_API int llmi_hip_l2_norm(const uint16_t *input, float *output, L2Params p,
                                  void *stream);

/* deltaGates (Graph.metal:131-144): for i < rows * width, head = i % width:
 * beta[i] = fp16(logistic(b[i])) (as fp32), decay[i] = exp(-exp(a_log[head])
 * * stableSoftplus(a[i] + dt_bias[head])). a, b fp16; a_log, dt_bias,
 * beta, decay fp32. */
LLMI_HIP_API int llmi_hip_delta_gates(const uint16_t *a, const uint16_t *b, const float *a_log,
                                      const float *dt_bias, float *beta, float *decay,
                                      RowParams p, void *stream);

/* gatedRmsNorm (Reference.metal:228-259, dispatched at
 * MetalReferenceGraph.mm:298-303 and MetalExecutionPlan.cpp:586-594): the
 * DeltaNet output's norm, out[r][i] = fp16(fp16(x[r][i] * rmsScale(x[r])) *
 * weight[i] * silu(gate[r][i])), rows x width, fp16 x, gate and out, fp32
 * weight. width a multiple of 8 up to 256 and 16-byte aligned buffers
 * (DeltaNet's valueDim 128); other shapes return LLMI_HIP_UNSUPPORTED. */
LLMI_HIP_API int llmi_hip_gated_rms_norm(const uint16_t *input, const uint16_t *gate,
                                         const float *weight, uint16_t *output, RowParams p,
                                         void *stream);

/* gatedRmsNormActivated (Reference.metal:252-259): the same with an fp32
 * gate already activated by the projection's epilogue (no SiLU here). */
LLMI_HIP_API int llmi_hip_gated_rms_norm_activated(const uint16_t *input, const float *gate,
                                                   const float *weight, uint16_t *output,
                                                   RowParams p, void *stream);

/* --------------------------------------------------------------- CausalGqa
 * Replaces gqaFlashAttention (FlashAttention.metal:1-83) for T > 1 and the
 * 3-pass gqaScores/gqaSoftmax/gqaValue (Reference.metal:303-323,
 * Graph.metal:172-230) for T == 1. Semantics of the op contract
 * (lib/GraphIR/Graph.cpp:248-279):
 *   q        [T][Hq][d] fp16, dense
 *   k_cache  [cap][Hkv][d] fp16, rows [0, P+T) already appended
 *   v_cache  same layout
 *   out      [T][Hq][d] fp16
 *   O[t,h] = softmax_j(q[t,h] . k[j,h/(Hq/Hkv)] / sqrt(d)) v[j,...], j <= P+t
 * Softmax and accumulation are fp32; the output is rounded to fp16 once.
 * `workspace` must hold llmi_hip_gqa_workspace_bytes(p) bytes (0 = none
 * needed): the split-K decode's per-split partials, written and read
 * within the call, so its contents between calls do not matter. */
LLMI_HIP_API int llmi_hip_causal_gqa(const uint16_t *q, const uint16_t *k_cache,
                        const uint16_t *v_cache, uint16_t *out, GqaParams p,
                        void *workspace, size_t workspace_bytes, void *stream);

LLMI_HIP_API size_t llmi_hip_gqa_workspace_bytes(GqaParams p);

/* KvAppend followed by CausalGqa on the same step, in one call: the T new
 * rows k_new/v_new [T][Hkv][d] are written to cache rows [P, P+T) exactly as
 * llmi_hip_kv_append would, and the attention sees them -- the effect of the
 * two ops in graph order (lib/GraphIR/Graph.cpp:248-279; the reference
 * lowers them as two dispatch groups, MetalExecutionPlan.cpp:516-548). For
 * T == 1 it is one launch (the decode kernel reads the new row from
 * k_new/v_new and stores it while it attends); for T > 1 it is the append
 * launch followed by the prefill launch. Workspace as for
 * llmi_hip_causal_gqa (llmi_hip_gqa_workspace_bytes of the same params). */
LLMI_HIP_API int llmi_hip_kv_append_causal_gqa(const uint16_t *q, const uint16_t *k_new,
                                  const uint16_t *v_new, uint16_t *k_cache,
                                  uint16_t *v_cache, uint16_t *out, GqaParams p,
                                  void *workspace, size_t workspace_bytes,
                                  void *stream);

/* The same as llmi_hip_kv_append_causal_gqa, allocating nothing and taking
 * no workspace. It has no counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). The split-K decode's
 * partials go to a static device array of LLMI_HIP_NOALLOC_SCRATCH_BYTES
 * that each device the library runs on holds until the process ends; a
 * shape whose partials need more returns LLMI_HIP_WORKSPACE before any
 * launch (the north-star shapes need at most 2.1 MB). Calls that overlap on
 * one device share that array and race; calls on one stream are ordered. */
#define LLMI_HIP_NOALLOC_SCRATCH_BYTES (8u << 20)
LLMI_HIP_API int llmi_hip_kv_append_causal_gqa_noalloc(const uint16_t *q,
                                                       const uint16_t *k_new,
                                                       const uint16_t *v_new,
                                                       uint16_t *k_cache, uint16_t *v_cache,
                                                       uint16_t *out, GqaParams p,
                                                       void *stream);

/* The attention block of a Qwen3.5 GQA layer around CausalGqa in one call
 * (Qwen35ModelBuilder.cpp:175-197; the reference graph's dispatches,
 * MetalReferenceGraph.mm:307-337): q_proj [T][Hq][2d] holds per head the d
 * query values followed by the d gate values (headStride 2d), k_proj and
 * v_new [T][Hkv][d] the step's new keys (before their norm) and values. In
 * order, as the reference does them:
 *   q   = normRope(q_proj rows, q_weight)        (Reference.metal:271-293)
 *   k_cache rows [P, P+T) = normRope(k_proj, k_weight) at positions P + t
 *   v_cache rows [P, P+T) = v_new                (cacheAppend)
 *   a   = CausalGqa(q, caches)                   (as llmi_hip_causal_gqa)
 *   out = fp16(fp16(logistic(gate)) * a)         (sigmoidMul; the gate of
 *                                                 applyGqa, Reference.metal:350-353)
 * with rotary_dim, epsilon and theta the normRope parameters of both norms.
 * out, k_cache and v_cache are bit-identical to llmi_hip_norm_rope (q and
 * k), llmi_hip_cache_append, llmi_hip_causal_gqa and llmi_hip_sigmoid_mul
 * run in that order. T == 1 is one decode launch (plus its merge) that does
 * all of it; T > 1 normRopes K into the cache and appends V (two launches),
 * then runs the MFMA prefill with the q normRope in its query load and the
 * gate in its output store. Workspace: llmi_hip_gqa_workspace_bytes(p).
 * Supported: d 128 or 256, Hq/Hkv 2 or 4 (decode) or <= 4 (prefill),
 * rotary_dim a multiple of 16 up to d; other shapes return UNSUPPORTED. */
LLMI_HIP_API int llmi_hip_gated_attention(const uint16_t *q_proj, const uint16_t *k_proj,
                                          const uint16_t *v_new, const float *q_weight,
                                          const float *k_weight, uint16_t *k_cache,
                                          uint16_t *v_cache, uint16_t *out, GqaParams p,
                                          unsigned rotary_dim, float epsilon, float theta,
                                          void *workspace, size_t workspace_bytes,
                                          void *stream);

/* The same block when the q projection has already activated its gate
 * half: the execution plan fuses Sigmoid into that projection's epilogue
 * (the sigmoid-columns epilogue of the interleaved query / gate halves,
 * MetalExecutionPlan.cpp:376-404), and SigmoidMul then lowers to
 * multiplyF16 of the stored gate and the attention output
 * (MetalExecutionPlan.cpp:606-614). Here the gate values in q_proj are
 * those fp16(logistic(.)) values and
 *   out = fp16(gate * a)                         (multiplyF16, Graph.metal:87-94)
 * Everything else, the launches, the workspace and the supported shapes are
 * llmi_hip_gated_attention's. */
LLMI_HIP_API int llmi_hip_gated_attention_activated(
    const uint16_t *q_proj, const uint16_t *k_proj, const uint16_t *v_new,
    const float *q_weight, const float *k_weight, uint16_t *k_cache, uint16_t *v_cache,
    uint16_t *out, GqaParams p, unsigned rotary_dim, float epsilon, float theta,
    void *workspace, size_t workspace_bytes, void *stream);

/* ------------------------------------------------------------- DeltaUpdate
 * Replaces graphDeltaUpdate (Graph.metal:146-170 with updateDeltaColumn,
 * Reference.metal:182-197): the gated delta rule over T tokens, per value
 * head h (key head h / (Hv/Hk)) and state column j:
 *   S <- decay_t * S ; delta = beta_t (v_tj - k_t . S[:,j])
 *   S[:,j] += k_t delta ; out_tj = fp16(q_t . S[:,j])
 * Operand contract (lib/GraphIR/Graph.cpp:226-246):
 *   q, k   [T][Hk*dk] fp32 (q already L2-normalised and scaled, k normalised)
 *   v      [T][Hv*dv] fp16
 *   beta   [T][Hv] fp32      decay [T][Hv] fp32, LINEAR decay in [0, 1]
 *   state  [Hv][dk][dv] fp32, read and written in place
 *   out    [T][Hv*dv] fp16
 * T == 1 runs the recurrent decode step; T > 1 runs the chunk-wise form. */
LLMI_HIP_API int llmi_hip_delta_update(const float *q, const float *k, const uint16_t *v,
                          const float *beta, const float *decay, float *state,
                          uint16_t *out, GraphDeltaParams p, void *workspace,
                          size_t workspace_bytes, void *stream);

LLMI_HIP_API size_t llmi_hip_delta_workspace_bytes(GraphDeltaParams p);

/* The L2Norm -> DeltaUpdate pair of a DeltaNet layer in one call
 * (Qwen35ModelBuilder.cpp:155-156 emits L2Norm(q, eps, 1/sqrt(dk)) and
 * L2Norm(k, eps, 1) ahead of DeltaUpdate; l2NormF32, Graph.metal:96-109):
 * q and k are the fp16 rows [T][Hk*dk] the convolution produced, and the
 * update kernels normalise them as they load them. Each fp32 operand
 * element is the bits l2NormF32 would write (factor = rsqrt(sum of squares
 * in index order + epsilon) * scale, q_scale for q and 1 for k; element =
 * x * factor), so state and output equal llmi_hip_l2_norm on q and k
 * followed by llmi_hip_delta_update, without the fp32 q/k round trip. Other
 * operands, the workspace (llmi_hip_delta_workspace_bytes of the same
 * params) and the T == 1 / T > 1 kernel choice as llmi_hip_delta_update;
 * dk must be 64 or 128 and dv a multiple of 16 (else UNSUPPORTED). */
LLMI_HIP_API int llmi_hip_l2_norm_delta_update(const uint16_t *q, const uint16_t *k,
                                               const uint16_t *v, const float *beta,
                                               const float *decay, float *state,
                                               uint16_t *out, GraphDeltaParams p,
                                               float epsilon, float q_scale, void *workspace,
                                               size_t workspace_bytes, void *stream);

/* The L2Norm -> DeltaUpdate -> GatedRmsNorm chain of a DeltaNet layer in
 * one call (Qwen35ModelBuilder.cpp:155-166: the two L2Norms, DeltaUpdate,
 * then GatedRmsNorm(mixed, z, norm.weight, epsilon); gatedRmsNorm,
 * Reference.metal:228-259, dispatched at MetalReferenceGraph.mm:298-303).
 * q, k, v, beta, decay, state and the workspace as
 * llmi_hip_l2_norm_delta_update; gate is z, fp16 [T][Hv*dv]; norm_weight is
 * fp32 [dv]; out receives the normalised rows, fp16 [T][Hv*dv], bit for
 * bit what llmi_hip_l2_norm_delta_update followed by
 * llmi_hip_gated_rms_norm(out, gate, norm_weight, rows T*Hv, width dv,
 * norm_epsilon) leave there, without the round trip of the un-normalised
 * rows. Shapes: dk 128 and T >= 32 (the chunked form, whose scan
 * normalises the rows at its end once all Hv * dv / 16 of its workgroups
 * have arrived: out and gate 16-byte aligned, and the grid must fit on the
 * device at once -- 512 workgroups on MI355X), or dk 64 / 128, dv 64 / 128
 * and T <= 32 (one workgroup per value head); others return
 * LLMI_HIP_UNSUPPORTED. */
LLMI_HIP_API int llmi_hip_l2_norm_delta_gated_norm(
    const uint16_t *q, const uint16_t *k, const uint16_t *v, const float *beta,
    const float *decay, float *state, const uint16_t *gate, const float *norm_weight,
    uint16_t *out, GraphDeltaParams p, float qk_epsilon, float q_scale, float norm_epsilon,
    void *workspace, size_t workspace_bytes, void *stream);

/* After llmi_hip_l2_norm_delta_gated_norm with the same params and
 * workspace (no counterpart in the reference, whose Metal dispatches do not
 * wait for each other inside a launch): the chunked form's scan normalises
 * a value head's rows only after a bounded wait for all of the head's
 * workgroups. This call waits for `stream` and returns LLMI_HIP_OK, or
 * LLMI_HIP_LAUNCH_FAILED if any workgroup's wait gave up (the normalised
 * rows are then not trustworthy and a session using them must become
 * invalid, MetalExecutor.mm:283-298). Shapes that take the recurrent form
 * return LLMI_HIP_OK at once without waiting. */
LLMI_HIP_API int llmi_hip_l2_norm_delta_gated_norm_status(const void *workspace,
                                                          size_t workspace_bytes,
                                                          GraphDeltaParams p, void *stream);

/* The same chain with the W8A8 model's tail (Qwen35ModelBuilder.cpp:
 * 155-166, then project(prepare(gated)): the out projection's
 * QuantizeActivation of the normalised rows), for a one-workgroup-per-head
 * step: gate is z as the fp32 SiLU epilogue of its projection left it
 * (llmi_hip_gated_rms_norm_activated), fp32 [T][Hv*dv]; out, quantized,
 * scales and *invalid receive, bit for bit, what
 * llmi_hip_l2_norm_delta_update followed by
 * llmi_hip_gated_rms_norm_activated_quantize(rows T*Hv, width dv,
 * norm_epsilon) leave there (its quantization: the flattened rows in
 * 32-wide groups). No counterpart in the reference, which launches them
 * one by one; the plan uses it for a decode step's DeltaNet tail. q, k, v,
 * beta, decay and state as llmi_hip_l2_norm_delta_update. dk 64 or 128, dv
 * 64 or 128, T <= 32, out and quantized 16-byte aligned (else
 * LLMI_HIP_UNSUPPORTED); no workspace. No output may overlap an input:
 * each workgroup writes its head's rows while others still read. */
LLMI_HIP_API int llmi_hip_l2_norm_delta_gated_norm_activated_quantize(
    const uint16_t *q, const uint16_t *k, const uint16_t *v, const float *beta,
    const float *decay, float *state, const float *gate, const float *norm_weight,
    uint16_t *out, int8_t *quantized, float *scales, uint32_t *invalid, GraphDeltaParams p,
    float qk_epsilon, float q_scale, float norm_epsilon, void *stream);

/* Bound, in polls, of that arrival wait for later launches (0: every
 * workgroup gives up at once); returns the previous bound (default 2^22,
 * ~0.3 s). Process-wide, not thread-safe against concurrent launches. No
 * counterpart in the reference: for tests that force the give-up from the
 * host, so that every workgroup still exits normally. */
LLMI_HIP_API unsigned llmi_hip_set_arrival_wait_limit(unsigned polls);

/* ------------------------------------------------------- W8A8 projections
 * The quantized projection path of the whole-graph plan (lowered at
 * MetalExecutionPlan.cpp:464-510 for LinearW8A8, :566-580 for
 * QuantizeActivation, :435-462 for EmbeddingGather). Integer parts are exact; the fp32 arithmetic and every fp16
 * rounding follow the reference kernels' expressions, with exp and log
 * correctly rounded to fp32.
 *
 * quantizeActivation (Graph.metal:33-68): input [rows][width] fp16 ->
 * quantized [rows][groups * 32] int8 (groups = ceil(width / 32), the tail of
 * the last group zero), scales [rows][groups] fp32 (max |x| / 127 of the
 * group; 1 for an all-zero group); a group holding a non-finite value is
 * quantized to zeros with scale 1 and ORs 1 into *invalid (may be NULL). */
LLMI_HIP_API int llmi_hip_quantize_activation(const uint16_t *input, int8_t *quantized,
                                              float *scales, uint32_t *invalid,
                                              QuantizeParams p, void *stream);

/* linearW8A8Gemv (rows == 1) / linearW8A8Gemm (W8A8.metal:28-113; launch
 * shape LinearW8Launch.h:14-21) with storeLinear (Reference.metal:14-47):
 * activation [rows][groups * 32] int8 and act_scales [rows][groups] fp32 (a
 * quantizeActivation result); weight [columns][groups * 32] int8 and
 * weight_scales [columns][groups] fp16 (one shard of the projection: output
 * columns firstRow .. firstRow + columns - 1). For each (row, column): the
 * exact int32 dot of each 32-wide group, times the activation scale, times
 * the weight scale, summed in fp32 by 16 (one row) or 8 interleaved group
 * lanes combined by an xor butterfly -- the reference's order -- then
 * rounded to fp16 and passed through the epilogue into
 * output[row * outputWidth + firstRow + column]: fp16, or fp32 for
 * LLMI_LINEAR_SILU_F32 / DELTA_BETA / DELTA_DECAY. aux is the fp16
 * multiplier of SILU_MUL (same index as the output) or the fp32 A_log of
 * DELTA_DECAY (by column), bias the fp32 dt bias of DELTA_DECAY; otherwise
 * both may be NULL. */
LLMI_HIP_API int llmi_hip_linear_w8a8(const int8_t *activation, const float *act_scales,
                                      const int8_t *weight, const uint16_t *weight_scales,
                                      void *output, const void *aux, const float *bias,
                                      LinearW8Params p, void *stream);

/* embeddingW8 (Graph.metal:16-31): for token t with id in [firstRow,
 * firstRow + rowCount), output[t][c] = fp16(weight[id - firstRow][c] *
 * scales[id - firstRow][c / 32]), weight rows groups * 32 int8 wide, scales
 * fp16; rows of other ids are left as they are (another shard writes them).
 * ids uint32. */
LLMI_HIP_API int llmi_hip_embedding_w8(const uint32_t *ids, const int8_t *weight,
                                       const uint16_t *scales, uint16_t *output,
                                       GroupedEmbedParams p, void *stream);

/* embedding (Reference.metal:49-58): fp16 rows [rowCount][hidden], copied
 * for ids in [firstRow, firstRow + rowCount). */
LLMI_HIP_API int llmi_hip_embedding(const uint32_t *ids, const uint16_t *weight,
                                    uint16_t *output, EmbedParams p, void *stream);

/* -------------------------------------------- elementwise, views, linearF16
 * The whole-graph plan's remaining ops (lowered at MetalExecutionPlan.cpp:
 * 469-477, 604-626). Elementwise ops take count fp16 elements, dense. */

/* residualAdd (Reference.metal:119-126): out[i] = fp16(a[i] + b[i]). */
LLMI_HIP_API int llmi_hip_residual_add(const uint16_t *a, const uint16_t *b, uint16_t *out,
                                       ElementParams p, void *stream);

/* swiGlu (Reference.metal:128-135): out[i] = fp16(fp16(silu(gate[i])) * up[i]). */
LLMI_HIP_API int llmi_hip_swiglu(const uint16_t *gate, const uint16_t *up, uint16_t *out,
                                 ElementParams p, void *stream);

/* siluF16 (Graph.metal:70-76): out[i] = fp16(silu(in[i])). In place allowed. */
LLMI_HIP_API int llmi_hip_silu(const uint16_t *in, uint16_t *out, ElementParams p, void *stream);

/* multiplyF16 (Graph.metal:87-94): out[i] = fp16(a[i] * b[i]). */
LLMI_HIP_API int llmi_hip_multiply(const uint16_t *a, const uint16_t *b, uint16_t *out,
                                   ElementParams p, void *stream);

/* copyHalfView (Graph.metal:1-14): out[i] = src[offset + sum_d index_d(i) *
 * strides[d]], i < count, the index taken over dims (outermost first). */
LLMI_HIP_API int llmi_hip_copy_half_view(const uint16_t *src, uint16_t *out, HalfViewParams p,
                                         void *stream);

/* linearF16 (Reference.metal:61-103): for row < tokens, col < rowCount,
 * acc = fma chain over k = 0 .. inputWidth-1 of input[row][k] *
 * weight[col][k] in fp32, then storeLinear at output[row * outputWidth +
 * firstRow + col] with the given epilogue (aux, bias as for linearW8A8). */
LLMI_HIP_API int llmi_hip_linear_f16(const uint16_t *input, const uint16_t *weight, void *output,
                                     const void *aux, const float *bias, LinearParams p,
                                     void *stream);

/* residualAdd -> rmsNorm -> quantizeActivation of rows x width in one launch
 * (no counterpart in the reference, which launches the three; the plan uses
 * it where a norm's only consumer is the quantization): sum = fp16(a + b)
 * written to sum_out, then exactly llmi_hip_rms_norm of sum and
 * llmi_hip_quantize_activation of that into q [rows][groups * 32] (16-byte
 * aligned), scales [rows][groups] and *invalid (may be NULL). b == NULL
 * normalises a itself (sum_out unused). width <= 8192. */
LLMI_HIP_API int llmi_hip_add_rms_norm_quantize(const uint16_t *a, const uint16_t *b,
                                                uint16_t *sum_out, const float *weight,
                                                int8_t *q, float *scales, uint32_t *invalid,
                                                RowParams p, void *stream);

/* The buffers of one projection of llmi_hip_add_rms_norm_linear_w8a8: those
 * of an llmi_hip_linear_w8a8 call on the norm's quantized row. With
 * conv_weight set, the projection's fp16 row (no epilogue) is not stored:
 * it passes through the one-token causalConv of a kernel-4 convolution
 * with SiLU (causalConv with applySilu, Reference.metal:137-161, T = 1):
 * output receives, bit for bit, what llmi_hip_causal_conv (silu on) of the
 * projected row leaves there, and conv_history [columns][3] fp16 is
 * updated in place as it updates it. */
typedef struct llmi_hip_norm_projection {
  const int8_t *weight;          /* [columns][groups * 32], 16-byte aligned */
  const uint16_t *weight_scales; /* [columns][groups] fp16 */
  void *output;
  const void *aux;
  const float *bias;
  const uint16_t *conv_weight;   /* NULL, or [columns][4] fp16 */
  uint16_t *conv_history;        /* with conv_weight: [columns][3] fp16 */
} llmi_hip_norm_projection;

#define LLMI_HIP_NORM_LINEAR_MAX 4

typedef struct NormLinearParams {
  RowParams norm;   /* rows == 1, width <= 4096 */
  unsigned count;   /* projections, 1 .. LLMI_HIP_NORM_LINEAR_MAX */
  LinearW8Params linear[LLMI_HIP_NORM_LINEAR_MAX]; /* rows == 1, groups = ceil(width / 32) */
} NormLinearParams;

/* llmi_hip_add_rms_norm_quantize of one row followed by llmi_hip_linear_w8a8
 * of each projection on the quantized row, in one launch (no counterpart in
 * the reference, which launches them one by one; the plan uses it for a
 * decode step's input norm and the projections that read its quantization).
 * The outputs are the separate calls' bits. q and scales may be NULL (not
 * written) when nothing else reads them. Epilogues as for
 * llmi_hip_linear_w8a8; a LLMI_LINEAR_SILU_MUL multiplier (aux) computed
 * in the same call must be the previous projection's output, that
 * projection with no epilogue and the same columns, width <= 2560 (the two
 * are computed by the same lanes). A projection with a convolution
 * (conv_weight) has no epilogue, computes all of its output row (first row
 * 0, columns == output width) and is no SwiGLU multiplier. At most 4096
 * workgroups of 60 columns in all (one per CU runs best: 256 on MI355X).
 * No output may overlap a, b, sum_out, q, scales or another output: the
 * projections run concurrently with the norm of other workgroups. */
LLMI_HIP_API int llmi_hip_add_rms_norm_linear_w8a8(const uint16_t *a, const uint16_t *b,
                                                   uint16_t *sum_out, const float *weight,
                                                   int8_t *q, float *scales, uint32_t *invalid,
                                                   const llmi_hip_norm_projection *projections,
                                                   NormLinearParams p, void *stream);

/* llmi_hip_gated_rms_norm_activated of rows x width followed by
 * llmi_hip_quantize_activation of its output (the flattened rows, 32-wide
 * groups), in one launch (no counterpart in the reference, which launches
 * the two; the plan uses it where the quantization reads the norm's output
 * right after it). out, q, scales and *invalid receive the two launches'
 * bits. width a multiple of 32 and at most 256; x, gate, out and q 16-byte
 * aligned (else LLMI_HIP_UNSUPPORTED). */
LLMI_HIP_API int llmi_hip_gated_rms_norm_activated_quantize(const uint16_t *x, const float *gate,
                                                            const float *weight, uint16_t *out,
                                                            int8_t *q, float *scales,
                                                            uint32_t *invalid, RowParams p,
                                                            void *stream);

/* ----------------------------------------------------------------- helpers */

/* Zero a workspace (enqueued on `stream`). No kernel of this library needs
 * a zeroed workspace; provided for callers that want deterministic
 * contents. */
LLMI_HIP_API int llmi_hip_workspace_init(void *workspace, size_t bytes, void *stream);

/* Plan-record support (MetalSession.h:11-16, tools/run/Main.cpp:244-255):
 * the number of kernel launches an op lowers to and the name of launch
 * `index`. `params` points to the op's parameter struct. NULL / 0 on a
 * parameter set the backend rejects. */
LLMI_HIP_API unsigned llmi_hip_dispatch_count(int op, const void *params);
LLMI_HIP_API const char *llmi_hip_kernel_name(int op, const void *params, unsigned index);

LLMI_HIP_API const char *llmi_hip_status_string(int status);
LLMI_HIP_API const char *llmi_hip_last_error(void);

/* Library version and the gfx target its kernels were built for. */
LLMI_HIP_API const char *llmi_hip_build_info(void);

/* -------------------------------------------------------------- session
 * A host-side mirror of MetalSession's state ownership and step contract
 * (include/llminfer/Backend/Metal/MetalSession.h:28-50,
 * lib/Backend/Metal/MetalExecutor.mm:56-118, 255-298) for one hybrid layer
 * pair: one GQA layer (its K/V caches) and one DeltaNet layer (its fp32
 * recurrent state). The session allocates and owns the device state,
 * validates before launching, advances `past` only on success, becomes
 * invalid after a failure that happened after a launch, and zeroes state on
 * reset. Calls on one session must be serialised. */
typedef struct llmi_hip_session llmi_hip_session;

typedef struct llmi_hip_session_config {
  unsigned capacity;   /* KV cache rows */
  unsigned queryHeads, kvHeads, headDim;
  unsigned keyHeads, keyDim, valueHeads, valueDim;
} llmi_hip_session_config;

/* A plan record, laid out as MetalDispatchInfo{opIndex, kernel, epilogue,
 * fusedOpIndex} (MetalSession.h:11-16). As in the reference, `epilogue`
 * names a projection epilogue fused into the launch and `fused_op_index` is
 * meaningful only when `epilogue` is non-empty (tools/run/Main.cpp:244-255
 * prints it only then); this path has no projection epilogues, so every
 * record carries epilogue "" and fused_op_index 0 (the reference's
 * defaults, MetalExecutionPlan.h:31-32). A launch that performs two ops of
 * the step -- the decode launch that also appends the new K/V row -- is
 * recorded once under each op, in op order, so the records' op indices
 * alone cover every op of the step (MetalReferenceTest.py:346-351). */
typedef struct llmi_hip_dispatch {
  size_t op_index;
  const char *kernel;
  const char *epilogue;
  size_t fused_op_index;
} llmi_hip_dispatch;

LLMI_HIP_API int llmi_hip_session_open(const llmi_hip_session_config *config,
                          void *stream, llmi_hip_session **out);
LLMI_HIP_API void llmi_hip_session_close(llmi_hip_session *s);
LLMI_HIP_API void llmi_hip_session_reset(llmi_hip_session *s);
LLMI_HIP_API unsigned llmi_hip_session_past(const llmi_hip_session *s);
LLMI_HIP_API int llmi_hip_session_invalid(const llmi_hip_session *s);

/* Device pointers of the session-owned state (for inspection and tests). */
LLMI_HIP_API uint16_t *llmi_hip_session_key_cache(llmi_hip_session *s);
LLMI_HIP_API uint16_t *llmi_hip_session_value_cache(llmi_hip_session *s);
LLMI_HIP_API float *llmi_hip_session_recurrent_state(llmi_hip_session *s);

/* Declare rows [0, past) of the caches and the recurrent state as written:
 * for a caller that filled the session-owned buffers itself through the
 * pointers above (a restored checkpoint, or a test seeding a long context).
 * past <= capacity; a session left invalid by a failed step must be reset
 * first. Host only: nothing is launched. */
LLMI_HIP_API int llmi_hip_session_restore(llmi_hip_session *s, unsigned past);

/* The checks llmi_hip_session_open and llmi_hip_session_step make before
 * any allocation or launch, for a step of `tokens` tokens at `past` in a
 * session of `config` -- the op contracts of KvAppend, CausalGqa and
 * DeltaUpdate (lib/GraphIR/Graph.cpp:226-279) on the shapes the session
 * derives from its config, the step shape (0 < tokens <= capacity - past,
 * Graph.cpp:382-387), the lowering's 32-bit element-index limit
 * (MetalExecutionPlan.cpp:32-40) and kernel availability. Host only: needs
 * no device. */
LLMI_HIP_API int llmi_hip_session_check(const llmi_hip_session_config *config,
                                        unsigned past, unsigned tokens);

/* One step of T tokens through both layers, in graph order: DeltaUpdate
 * (op 0), KvAppend (op 1), CausalGqa (op 2) -- the order the builder emits
 * them for a DeltaNet layer followed by a GQA layer. All operands are
 * device pointers with the op contracts above; outputs are written to
 * delta_out [T][Hv*dv] and gqa_out [T][Hq][d]. Validation failures return
 * nonzero before any launch. If `records` is non-NULL, up to `cap` plan
 * records are written and *count receives the total; for T == 1 KvAppend
 * runs inside the attention launch, which is recorded under op 1 and again
 * under op 2. The step waits for the GPU once at the end (one host sync per
 * step, MetalContext.mm:141-151). */
LLMI_HIP_API int llmi_hip_session_step(llmi_hip_session *s, unsigned tokens,
                          const float *dq, const float *dk, const uint16_t *dv,
                          const float *beta, const float *decay,
                          uint16_t *delta_out, const uint16_t *q,
                          const uint16_t *k, const uint16_t *v,
                          uint16_t *gqa_out, llmi_hip_dispatch *records,
                          size_t cap, size_t *count);

/* ------------------------------------------------------ whole-graph plan
 * Replaces MetalExecutionPlan::lower (lib/Backend/Metal/
 * MetalExecutionPlan.cpp:169-760) and the executor that encodes it
 * (MetalExecutor.mm:120-200): one step's GraphIR graph lowered to HIP
 * dispatches over the calls above. The graph is passed flat; its enums are
 * GraphIR's in declaration order (include/llminfer/GraphIR/Graph.h:22-88),
 * so a reference-side adapter copies ir::Graph field by field.
 *
 * Lowering keeps the reference's decisions that its tooling observes:
 * projection epilogues fused into their sole consumer (Silu, SiluMul,
 * GatedRmsNorm's gate, DeltaGates' a and b, and the interleaved query /
 * gate halves of SigmoidMul; MetalExecutionPlan.cpp:313-403), one record per
 * launched kernel with its op, epilogue and fused op, non-contiguous fp16
 * views materialised by copyHalfView. Results live in one scratch arena:
 * each value takes the first free range that fits from its defining op to
 * its last use. Contiguous views are addressed in place. */

enum llmi_graph_element { LLMI_GRAPH_I8 = 0, LLMI_GRAPH_U32, LLMI_GRAPH_F16, LLMI_GRAPH_F32 };
enum llmi_graph_value_kind {
  LLMI_GRAPH_INPUT = 0, LLMI_GRAPH_WEIGHT, LLMI_GRAPH_RESULT, LLMI_GRAPH_VIEW
};
enum llmi_graph_state_kind {
  LLMI_GRAPH_CONV_HISTORY = 0, LLMI_GRAPH_DELTA_RECURRENT, LLMI_GRAPH_KEY_CACHE,
  LLMI_GRAPH_VALUE_CACHE
};
enum llmi_graph_op_kind {
  LLMI_GRAPH_EMBEDDING_GATHER = 0, LLMI_GRAPH_QUANTIZE_ACTIVATION, LLMI_GRAPH_LINEAR_F16,
  LLMI_GRAPH_LINEAR_W8A8, LLMI_GRAPH_RMS_NORM, LLMI_GRAPH_GATED_RMS_NORM, LLMI_GRAPH_L2_NORM,
  LLMI_GRAPH_ADD, LLMI_GRAPH_SILU, LLMI_GRAPH_SILU_MUL, LLMI_GRAPH_SIGMOID_MUL,
  LLMI_GRAPH_RESHAPE, LLMI_GRAPH_SLICE, LLMI_GRAPH_PARTIAL_ROPE, LLMI_GRAPH_CAUSAL_CONV1D,
  LLMI_GRAPH_DELTA_GATES, LLMI_GRAPH_DELTA_UPDATE, LLMI_GRAPH_KV_APPEND, LLMI_GRAPH_CAUSAL_GQA
};

#define LLMI_GRAPH_MAX_RANK 4

/* ir::ValueDesc (Graph.h:35-46): strides and view_offset in elements;
 * view_of and defining_op -1 when absent; weight: the index of a weight
 * value's tensor in the table given to llmi_hip_plan_lower, -1 otherwise. */
typedef struct llmi_graph_value {
  uint32_t element, kind, rank, reserved;
  uint64_t shape[LLMI_GRAPH_MAX_RANK], strides[LLMI_GRAPH_MAX_RANK];
  int64_t view_of, defining_op, weight;
  uint64_t view_offset, group_size;
} llmi_graph_value;

/* ir::StateDesc (Graph.h:48-52). */
typedef struct llmi_graph_state {
  uint32_t kind, layer, element, rank;
  uint64_t shape[LLMI_GRAPH_MAX_RANK];
} llmi_graph_state;

/* ir::Operation (Graph.h:120-126) with its attributes flattened
 * (Graph.h:90-118): group_size (QuantizeAttr), epsilon (NormAttr),
 * group_width / epsilon / scale (L2NormAttr), axis / begin / length
 * (SliceAttr), rotary_width / theta (RopeAttr), state (StateAttr), keys /
 * values (KvAttr). layer -1: none. */
typedef struct llmi_graph_op {
  uint32_t kind;
  int32_t layer;
  uint32_t input_count, output_count;
  uint32_t inputs[5], outputs[2];
  uint32_t state, keys, values;
  uint64_t group_size, group_width, axis, begin, length, rotary_width;
  float epsilon, scale, theta, reserved;
} llmi_graph_op;

/* One step's graph (ir::Graph, Graph.h:133-170). */
typedef struct llmi_graph {
  uint64_t tokens, past, capacity;
  const llmi_graph_value *values;
  size_t value_count;
  const llmi_graph_state *states;
  size_t state_count;
  const llmi_graph_op *ops;
  size_t op_count;
  const uint32_t *outputs;
  size_t output_count;
} llmi_graph;

/* A model tensor in device memory (ModelFile's TensorView): data, and for
 * int8 tensors the fp16 group scales [rows][groups]. Rows of int8 tensors
 * are padded to whole 32-wide groups. */
typedef struct llmi_weight {
  const void *data;
  const uint16_t *scales;
} llmi_weight;

typedef struct llmi_hip_plan llmi_hip_plan;

/* Lowers `graph` (host memory, read during the call only) over `weights`
 * (device pointers, which must stay valid while the plan is used). Host
 * only: launches nothing and needs no device. Fails with
 * LLMI_HIP_INVALID_ARGUMENT for a malformed graph or a graph the plan
 * cannot lower (a message in llmi_hip_last_error), LLMI_HIP_UNSUPPORTED for
 * an op shape no kernel here serves. */
LLMI_HIP_API int llmi_hip_plan_lower(const llmi_graph *graph, const llmi_weight *weights,
                                     size_t weight_count, llmi_hip_plan **out);
LLMI_HIP_API void llmi_hip_plan_destroy(llmi_hip_plan *plan);

/* Bytes of the scratch arena llmi_hip_plan_execute needs (256-aligned). */
LLMI_HIP_API size_t llmi_hip_plan_scratch_bytes(const llmi_hip_plan *plan);

/* The logits output: rows and elements (0 when the graph has no output). */
LLMI_HIP_API void llmi_hip_plan_logits(const llmi_hip_plan *plan, uint64_t *rows,
                                       uint64_t *elements);

/* The plan's records, one per launched kernel in launch order
 * (MetalDispatchInfo, MetalSession.h:11-16): up to `cap` are written to
 * `records` (may be NULL); returns the total. Kernel and epilogue names are
 * static strings; epilogue is NULL for an unfused launch, and
 * fused_op_index is then 0. */
LLMI_HIP_API size_t llmi_hip_plan_dispatches(const llmi_hip_plan *plan,
                                             llmi_hip_dispatch *records, size_t cap);

/* The kernel launches one llmi_hip_plan_execute issues (no counterpart in
 * the reference: a launch that serves several ops has a record for each, so
 * records outnumber launches). */
LLMI_HIP_API size_t llmi_hip_plan_launches(const llmi_hip_plan *plan);

/* Runs the plan on `stream`: scratch (device, llmi_hip_plan_scratch_bytes),
 * states[i] the device buffer of graph state i (its shape, dense),
 * token_ids (device, tokens uint32), logits (device fp16 [rows][vocab], or
 * NULL when the graph has no output), invalid (device uint32 that each
 * quantizeActivation ORs 1 into on a non-finite group; NULL: ignored). The
 * launches are only enqueued: the caller synchronises. */
LLMI_HIP_API int llmi_hip_plan_execute(const llmi_hip_plan *plan, void *scratch,
                                       size_t scratch_bytes, void *const *states,
                                       size_t state_count, const uint32_t *token_ids,
                                       uint16_t *logits, uint32_t *invalid, void *stream);

/* ------------------------------------------------------ Qwen3.5 session
 * The whole-model session: MetalSession (include/llminfer/Backend/Metal/
 * MetalSession.h:26-50) and its executor (lib/Backend/Metal/
 * MetalExecutor.mm:56-118, 212-298) over the plan above. Each step builds
 * the graph of its shape with the op sequence of Qwen35ModelBuilder::build
 * (lib/Models/Qwen35/Qwen35ModelBuilder.cpp:100-235), lowers it, runs it
 * with one host synchronisation and returns the logits as floats. */

/* Qwen35TextConfig's fields (lib/ModelFormat/Qwen35Schema.h:16-23); the
 * derived widths follow from them. layer_kinds: one per layer. */
enum llmi_qwen35_layer { LLMI_QWEN35_DELTANET = 0, LLMI_QWEN35_GQA = 1 };
typedef struct llmi_qwen35_config {
  uint64_t hidden, intermediate, vocabulary, max_positions;
  uint64_t head_dim, q_heads, kv_heads, rotary_width;
  uint64_t key_heads, value_heads, key_dim, value_dim, conv_kernel;
  double epsilon, theta;
  uint32_t w8;            /* 1: int8 matrices and W8A8 projections; 0: fp16 */
  uint32_t layer_count;
  const uint8_t *layer_kinds;
} llmi_qwen35_config;

/* LogitsMode (include/llminfer/Models/Qwen35/Qwen35ModelBuilder.h:10). */
enum llmi_logits_mode { LLMI_LOGITS_NONE = 0, LLMI_LOGITS_LAST = 1, LLMI_LOGITS_ALL = 2 };

/* The graph of one step, host only (Qwen35ModelBuilder::build): tokens new
 * rows after past cached ones in caches of capacity rows (0: past +
 * tokens). Weight values refer by index to llmi_qwen35_graph_tensor's ids
 * ("embed_tokens.weight", "layers.<i>.mlp.up_proj.weight", ...; the tied
 * head reads the embedding). */
typedef struct llmi_qwen35_graph llmi_qwen35_graph;
LLMI_HIP_API int llmi_qwen35_build(const llmi_qwen35_config *config, uint64_t tokens,
                                   uint64_t past, uint64_t capacity, int logits_mode,
                                   llmi_qwen35_graph **out);
LLMI_HIP_API const llmi_graph *llmi_qwen35_graph_view(const llmi_qwen35_graph *graph);
LLMI_HIP_API size_t llmi_qwen35_graph_tensor_count(const llmi_qwen35_graph *graph);
LLMI_HIP_API const char *llmi_qwen35_graph_tensor(const llmi_qwen35_graph *graph, size_t index);
LLMI_HIP_API void llmi_qwen35_graph_destroy(llmi_qwen35_graph *graph);

/* A model tensor by id: device data and, for int8 tensors, fp16 group
 * scales (llmi_weight). */
typedef struct llmi_named_weight {
  const char *name;
  const void *data;
  const uint16_t *scales;
} llmi_named_weight;

/* MetalStepResult (MetalSession.h:18-24) without its vectors: the logits
 * go to the caller's buffer, the records to llmi_hip_model_dispatches. */
typedef struct llmi_hip_model_step_result {
  uint64_t past, logit_rows, scratch_bytes;
  size_t dispatch_count;
} llmi_hip_model_step_result;

typedef struct llmi_hip_model llmi_hip_model;

/* MetalSession::open (MetalExecutor.mm:230-253): the weights are borrowed
 * (device pointers that must outlive the session, looked up by id; every
 * tensor the model reads must be present); the session allocates and
 * zeroes one device buffer per state slot of the model's graph, and runs on
 * `stream`. 0 < capacity <= min(max_positions, 2^32 - 1). */
LLMI_HIP_API int llmi_hip_model_open(const llmi_qwen35_config *config,
                                     const llmi_named_weight *weights, size_t weight_count,
                                     uint64_t capacity, void *stream, llmi_hip_model **out);
LLMI_HIP_API void llmi_hip_model_close(llmi_hip_model *model);
/* MetalSession::reset (MetalExecutor.mm:294-298): zero state, past 0. */
LLMI_HIP_API void llmi_hip_model_reset(llmi_hip_model *model);
LLMI_HIP_API uint64_t llmi_hip_model_past(const llmi_hip_model *model);
LLMI_HIP_API int llmi_hip_model_invalid(const llmi_hip_model *model);
LLMI_HIP_API uint64_t llmi_hip_model_vocabulary(const llmi_hip_model *model);

/* MetalSession::step (MetalExecutor.mm:255-292): `count` host token IDs.
 * Checked before any launch: the session is valid, 0 < count <= capacity -
 * past, every ID is in the vocabulary, the step's state layout equals the
 * session's, the logits buffer holds the step's rows x vocabulary floats.
 * Then one graph run and one host synchronisation; past advances only on
 * success. A failure after the launches, or a non-finite activation found
 * by a quantization (MetalExecutor.mm:180-187), returns
 * LLMI_HIP_LAUNCH_FAILED and leaves the session invalid until reset. */
LLMI_HIP_API int llmi_hip_model_step(llmi_hip_model *model, const uint32_t *ids, size_t count,
                                     int logits_mode, float *logits, size_t logits_capacity,
                                     llmi_hip_model_step_result *result);
/* The plan records of the last successful step (MetalStepResult's
 * dispatches): up to `cap` written, the total returned. */
LLMI_HIP_API size_t llmi_hip_model_dispatches(const llmi_hip_model *model,
                                              llmi_hip_dispatch *records, size_t cap);
/* State slot `index` in graph order: its descriptor, device buffer (dense,
 * session-owned) and size. */
LLMI_HIP_API size_t llmi_hip_model_state_count(const llmi_hip_model *model);
LLMI_HIP_API int llmi_hip_model_state(const llmi_hip_model *model, size_t index,
                                      llmi_graph_state *desc, void **device, size_t *bytes);
/* Copies state slot `index` (all `bytes` of it) to `dst`, host or device
 * memory, after the session's pending work; waits for the copy. */
LLMI_HIP_API int llmi_hip_model_read_state(llmi_hip_model *model, size_t index, void *dst,
                                           size_t bytes);

/* Timing aid (no counterpart in the reference): the plan of a step of
 * `tokens` rows at `past` (destroy with llmi_hip_plan_destroy), and its run
 * on the session's state, scratch and stream without a synchronisation, a
 * check or a change of past. ids: device uint32 [tokens]; logits: device
 * fp16 [rows][vocabulary] or NULL for LLMI_LOGITS_NONE. */
LLMI_HIP_API int llmi_hip_model_plan(const llmi_hip_model *model, uint64_t tokens, uint64_t past,
                                     int logits_mode, llmi_hip_plan **out);
LLMI_HIP_API int llmi_hip_model_run(llmi_hip_model *model, const llmi_hip_plan *plan,
                                    const uint32_t *ids, uint16_t *logits);

#ifdef __cplusplus
}
#endif
#endif
