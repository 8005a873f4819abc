/*
 * CPU oracle for the llminfer attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker and the CPU
 * baseline that bench.py times next to the GPU. Only tests/, the smoke()
 * entry of __graft_entry__.py and bench.py's cpu_baseline leg may load it.
 * The product path (llminfer_amd, libllminfer_hip.so) never links or calls it.
 *
 * Every function restates the reference's arithmetic from its source (cited
 * per function as /root/reference relative path:line). The reference's GPU
 * kernels are Metal shaders that cannot run here, so these are restatements,
 * not builds. The pins that check each function are listed in tests/
 * (test_oracle_*.py); a function without a pin says so below.
 *
 * Layouts (identical to the reference's buffers):
 *   q          [T][Hq][d]        fp16 bits (uint16)
 *   k/v cache  [cap][Hkv][d]     fp16 bits, rows [0, P+T) valid
 *   out        [T][Hq][d]
 *   delta q,k  [T][Hk*dk]        fp32
 *   delta v    [T][Hv*dv]        fp16 bits
 *   beta,decay [T][Hv]           fp32 (decay is LINEAR, not log)
 *   state      [Hv][dk][dv]      fp32, updated in place
 *   delta out  [T][Hv*dv]        fp16 bits
 */
#ifndef LLMI_ORACLE_H
#define LLMI_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* fp16 <-> fp32, round-to-nearest-even with subnormals.
 * Follows lib/ModelFormat/Quantization.cpp:25-55. */
uint16_t orc_f32_to_f16(float value);
float orc_f16_to_f32(uint16_t bits);
void orc_f32_to_f16_n(const float *in, uint16_t *out, size_t n);
void orc_f16_to_f32_n(const uint16_t *in, float *out, size_t n);

/* Seeded synthetic inputs. Counter-based SplitMix64 -> Box-Muller in double,
 * rounded to fp32 then (for the _f16 variant) fp16 RNE. Sample i of
 * (seed, stream) depends only on (seed, stream, i). */
void orc_fill_normal_f32(uint64_t seed, uint64_t stream, size_t n, double mean,
                         double stddev, float *out);
void orc_fill_normal_f16(uint64_t seed, uint64_t stream, size_t n, double mean,
                         double stddev, uint16_t *out);

/* The LCG fixture generator of tests/FlashAttentionTest.mm:28-36:
 * state = state*1664525 + 1013904223; value = (int(state>>24) - 128) / 64.
 * *state carries over between calls, as the reference fills q, k, v in turn. */
void orc_fill_lcg_f16(uint32_t *state, size_t n, uint16_t *out);

/* Dense causal GQA in double precision.
 * Restates tests/FlashAttentionTest.mm:53-86: query row (t, h) sees keys
 * [0, P + t]; KV head = h / (Hq / Hkv); scores scaled by 1/sqrt(d). */
void orc_gqa_dense_f64(const uint16_t *q, const uint16_t *k_cache,
                       const uint16_t *v_cache, double *out, uint32_t T,
                       uint32_t Hq, uint32_t Hkv, uint32_t d, uint32_t P);

/* Eager 3-pass GQA with the fp16 rounding points of the reference decode
 * path: score = fp16(fp16(q.k) * rsqrt(d)) (Reference.metal:303-323),
 * probabilities rounded to fp16 (Graph.metal:172-210), fp32 PV accumulate
 * rounded to fp16 (Graph.metal:212-230). */
void orc_gqa_eager_f16(const uint16_t *q, const uint16_t *k_cache,
                       const uint16_t *v_cache, uint16_t *out, uint32_t T,
                       uint32_t Hq, uint32_t Hkv, uint32_t d, uint32_t P);

/* fp32 causal GQA with a per-row max/sum softmax and fp16 output: the
 * semantics of the fused flash kernel (FlashAttention.metal:14-82: fp32
 * scores, fp32 softmax, fp32 accumulate, one fp16 rounding at the end).
 * Multi-threaded over query rows with `threads` workers (0 = all CPUs in the
 * affinity mask). This is the CPU baseline that bench.py times. */
void orc_gqa_f32(const uint16_t *q, const uint16_t *k_cache,
                 const uint16_t *v_cache, uint16_t *out, uint32_t T,
                 uint32_t Hq, uint32_t Hkv, uint32_t d, uint32_t P,
                 int threads);

/* KvAppend: copy T new rows into cache rows [P, P+T). Reference.metal:295-301
 * with the offset of MetalExecutionPlan.cpp:516-523. */
void orc_kv_append(const uint16_t *src, uint16_t *cache, uint32_t T,
                   uint32_t Hkv, uint32_t d, uint32_t P);

/* Gated delta rule, token recurrence, double accumulation in a double state.
 * Restates Reference.metal:182-197 (updateDeltaColumn) with the layouts and
 * key-head map of Graph.metal:146-170: for value head h and column j,
 *   pred = sum_i decay*S[i][j]*k_i ; delta = beta*(v_j - pred)
 *   S[i][j] = decay*S[i][j] + k_i*delta ; y_j = sum_i S[i][j]*q_i.
 * state_in is read, state_out written (may alias). out may be NULL. */
void orc_delta_recurrent_f64(const float *q, const float *k, const uint16_t *v,
                             const float *beta, const float *decay,
                             const float *state_in, double *state_out,
                             double *out, uint32_t T, uint32_t Hk, uint32_t dk,
                             uint32_t Hv, uint32_t dv);

/* The same recurrence in fp32 with fp16 outputs, operation for operation as
 * updateDeltaColumn (fma order included). Multi-threaded over value columns.
 * This is the DeltaNet CPU baseline. state is updated in place. */
void orc_delta_recurrent_f32(const float *q, const float *k, const uint16_t *v,
                             const float *beta, const float *decay,
                             float *state, uint16_t *out, uint32_t T,
                             uint32_t Hk, uint32_t dk, uint32_t Hv, uint32_t dv,
                             int threads);

/* Chunk-wise (WY / UT-transform) form of the same recurrence, in double.
 * Published method: Yang, Kautz, Hatamizadeh, "Gated Delta Networks"
 * (arXiv:2412.06464) and Yang et al. "Parallelizing Linear Transformers with
 * the Delta Rule over Sequence Length" (arXiv:2406.06484). For each chunk of
 * C tokens with cumulative log decay g:
 *   A[t][s] = beta_t exp(g_t-g_s) k_t.k_s (s<t);  Tm = (I+A)^-1
 *   W = Tm diag(beta exp(g)) K ;  U' = Tm diag(beta) V ;  U = U' - W S
 *   Y = diag(exp(g)) Q S + M U,  M[t][s] = exp(g_t-g_s) q_t.k_s (s<=t)
 *   S <- exp(g_C) S + K^T diag(exp(g_C-g)) U
 * Only differences g_t - g_s with s <= t are exponentiated. */
void orc_delta_chunked_f64(const float *q, const float *k, const uint16_t *v,
                           const float *beta, const float *decay,
                           const float *state_in, double *state_out,
                           double *out, uint32_t T, uint32_t Hk, uint32_t dk,
                           uint32_t Hv, uint32_t dv, uint32_t chunk);

/* DeltaNet gate numerics of Graph.metal:131-144 with Reference.metal:4-12:
 * beta = fp16(logistic(b)) stored as f32; decay = exp(-exp(A_log[h]) *
 * stableSoftplus(a + dt_bias[h])). a, b are fp16 bits [T][Hv]. */
void orc_delta_gates(const uint16_t *a, const uint16_t *b, const float *a_log,
                     const float *dt_bias, float *beta, float *decay,
                     uint32_t T, uint32_t Hv);

/* Grouped L2 norm of Graph.metal:96-109 (l2NormF32): per row of `width`,
 * out = x * rsqrt(sum(x^2) + eps) * scale, fp16 in, fp32 out. */
void orc_l2norm_f32(const uint16_t *in, float *out, uint32_t rows,
                    uint32_t width, float eps, float scale);

/* causalConv (lib/Backend/Metal/Kernels/Reference.metal:137-161): the
 * DeltaNet depthwise causal convolution with its k-1 history rows (updated
 * in place), optionally followed by SiLU (silu(x) = x * logistic(x) in fp32,
 * exp correctly rounded). input/output [tokens][channels], weight
 * [channels][kernel_size], history [channels][kernel_size - 1], fp16. */
void orc_causal_conv(const uint16_t *input, const uint16_t *weight, uint16_t *history,
                     uint16_t *output, uint32_t tokens, uint32_t channels,
                     uint32_t kernel_size, uint32_t apply_silu);

/* Fused q/k RmsNorm + PartialRoPE of the reference graph, normRope
 * (lib/Backend/Metal/Kernels/Reference.metal:271-293 with rmsScale :98-103
 * and rotatePair :262-269; RopeParams, ReferenceParams.h:44-47). Row r of
 * `tokens * heads` reads `headDim` halves at input + r * headStride and
 * writes output + (outputStart * heads + r) * headDim; position =
 * past + r / heads. Same rounding points as the kernel: the normalised
 * value is rounded to fp16 before the rotation, cos/sin are rounded to fp16,
 * each product is rounded to fp16 before the sum. rsqrt is 1/sqrtf (two
 * correctly rounded steps); pow/cos/sin are the correctly rounded fp32
 * functions (evaluated in double, rounded once). */
void orc_norm_rope(const uint16_t *input, const float *weight, uint16_t *output,
                   uint32_t tokens, uint32_t heads, uint32_t head_dim,
                   uint32_t rotary_dim, uint32_t head_stride, uint32_t past,
                   uint32_t output_start, float epsilon, float theta);

/* partialRope (lib/Backend/Metal/Kernels/Graph.metal:111-129): rows of
 * width fp16 values, rotatePair on the first rotary_dim, the rest copied. */
void orc_partial_rope(const uint16_t *input, uint16_t *output, uint32_t rows, uint32_t heads,
                      uint32_t width, uint32_t rotary_dim, uint32_t past, float theta);

/* gatedRmsNorm (gate16, fp16 gate through SiLU) or gatedRmsNormActivated
 * (gate32, already activated), lib/Backend/Metal/Kernels/Reference.metal:
 * 228-259: out = fp16(fp16(x * rmsScale(x)) * weight[i] * g), rows x width. */
void orc_gated_rms_norm(const uint16_t *input, const uint16_t *gate16, const float *gate32,
                        const float *weight, uint16_t *output, uint32_t rows, uint32_t width,
                        float eps);

/* sigmoidMul (lib/Backend/Metal/Kernels/Graph.metal:78-85, logistic
 * Reference.metal:4): out = fp16(fp16(1 / (1 + exp(-gate))) * input), exp
 * correctly rounded to fp32. */
void orc_sigmoid_mul(const uint16_t *gate, const uint16_t *input, uint16_t *output,
                     size_t count);

/* The W8A8 projection path (lib/Backend/Metal/Kernels/W8A8.metal,
 * Graph.metal:16-68, storeLinear Reference.metal:14-47). Epilogue codes are
 * LinearEpilogue of ReferenceParams.h:8-16. */
enum {
  ORC_LINEAR_NONE = 0,
  ORC_LINEAR_SILU = 1,
  ORC_LINEAR_SILU_MUL = 2,
  ORC_LINEAR_SIGMOID_COLUMNS = 3,
  ORC_LINEAR_SILU_F32 = 4,
  ORC_LINEAR_DELTA_BETA = 5,
  ORC_LINEAR_DELTA_DECAY = 6,
};
void orc_quantize_activation(const uint16_t *input, int8_t *quantized, float *scales,
                             uint32_t *invalid, uint32_t rows, uint32_t width,
                             uint32_t groups);
/* output is fp16 (uint16_t) or, for SILU_F32 / DELTA_BETA / DELTA_DECAY,
 * fp32; aux is the fp16 multiplier (SILU_MUL) or the fp32 A_log
 * (DELTA_DECAY). */
void orc_linear_w8a8(const int8_t *act, const float *act_scales, const int8_t *weight,
                     const uint16_t *weight_scales, void *output, const void *aux,
                     const float *bias, uint32_t output_width, uint32_t first_row,
                     uint32_t groups, uint32_t rows, uint32_t columns, uint32_t epilogue,
                     uint32_t epilogue_block);
void orc_embedding_w8(const uint32_t *ids, const int8_t *weight, const uint16_t *scales,
                      uint16_t *output, uint32_t tokens, uint32_t hidden, uint32_t first_row,
                      uint32_t row_count, uint32_t groups);
void orc_embedding(const uint32_t *ids, const uint16_t *weight, uint16_t *output,
                   uint32_t tokens, uint32_t hidden, uint32_t first_row, uint32_t row_count);

/* residualAdd / swiGlu / siluF16 / multiplyF16 (kind 0..3), copyHalfView and
 * linearF16 (Reference.metal:61-135, Graph.metal:1-14, 70-95). */
void orc_elementwise(uint32_t kind, const uint16_t *a, const uint16_t *b, uint16_t *out,
                     size_t count);
void orc_copy_half_view(const uint16_t *src, uint16_t *out, uint32_t count, uint32_t offset,
                        const uint32_t *dims, const uint32_t *strides);
void orc_linear_f16(const uint16_t *input, const uint16_t *weight, void *output,
                    const void *aux, const float *bias, uint32_t tokens, uint32_t input_width,
                    uint32_t output_width, uint32_t first_row, uint32_t columns,
                    uint32_t epilogue, uint32_t epilogue_block);

/* Cost model of lib/GraphIR/Cost.cpp:180-201 (MACs) and :56-94 (bytes) for
 * the three hot ops. Returns 0 on success, -1 on overflow. */
typedef struct {
  uint64_t fp_macs, scalar_ops, exp;
  uint64_t read_bytes, write_bytes;
} orc_cost;
int orc_cost_kv_append(uint64_t T, uint64_t Hkv, uint64_t d, orc_cost *c);
int orc_cost_causal_gqa(uint64_t T, uint64_t P, uint64_t Hq, uint64_t Hkv,
                        uint64_t d, orc_cost *c);
int orc_cost_delta_update(uint64_t T, uint64_t Hk, uint64_t dk, uint64_t Hv,
                          uint64_t dv, orc_cost *c);

/* Number of CPUs in this process's affinity mask. */
int orc_cpu_count(void);

#ifdef __cplusplus
}
#endif
#endif
