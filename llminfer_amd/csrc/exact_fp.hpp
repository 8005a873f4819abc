// Device helpers for kernels whose results must equal a reference's fp32 /
// fp16 expressions bit for bit: every product and every fp16 rounding is
// kept as written. Files using these are compiled with -ffp-contract=off
// (llminfer_amd/build.py), and products and fp16 roundings pass through
// opaque(): without it the gfx950 backend selects v_fma_mixlo_f16 for an fp32
// product converted to fp16 (one rounding instead of two, and +0 for a -0
// product) and v_fma_mix_f32 for an fp16-rounded product added to another,
// whatever the contraction setting.
#pragma once

#include "hip_common.hpp"

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace llmi {

__device__ __forceinline__ float h2f(uint16_t b) {
  return (float)__builtin_bit_cast(_Float16, b);
}
__device__ __forceinline__ uint16_t f2h(float x) {
  return __builtin_bit_cast(uint16_t, (_Float16)x);
}

// The value, hidden from the optimiser, so that the operation producing it
// is selected as written and rounded on its own.
__device__ __forceinline__ float opaque(float x) {
  asm volatile("" : "+v"(x));
  return x;
}
__device__ __forceinline__ float mul32(float a, float b) { return opaque(a * b); }

// fp16 of the fp32 value x, with x itself rounded to fp32 first -- the two
// roundings of the reference's half(float expression). Without opaque() the
// backend may fold the product or fma producing x into v_fma_mix*_f16 and
// round once, and it decides that per instantiation.
__device__ __forceinline__ _Float16 f16_of(float x) { return (_Float16)opaque(x); }
__device__ __forceinline__ float round16(float x) { return opaque((float)f16_of(x)); }

// Correctly rounded float square root: taken in double and rounded once,
// which is exact rounding for a float argument (HIP's __fsqrt_rn is the
// native instruction, not always rounded to nearest).
__device__ __forceinline__ float sqrt_cr(float x) { return (float)__builtin_sqrt((double)x); }

// l2NormF32's row factor rsqrt(sum + eps) * scale (Graph.metal:96-109), with
// rsqrt as 1/sqrt, every step correctly rounded; each output element is then
// the single fp32 product x * factor. Explicit _rn operations, so that the
// result does not depend on the file's contraction setting.
__device__ __forceinline__ float l2_row_factor(float sum, float eps, float scale) {
  return __fmul_rn(__fdiv_rn(1.0f, sqrt_cr(__fadd_rn(sum, eps))), scale);
}

// The sum of squares of 8 fp16 values (as one 16-byte word) continued in
// index order by fma, the reference's loop.
__device__ __forceinline__ float sumsq8(uint4_t x, float sum) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float lo = h2f((uint16_t)(x[e] & 0xFFFFu)), hi = h2f((uint16_t)(x[e] >> 16));
    sum = __builtin_fmaf(lo, lo, sum);
    sum = __builtin_fmaf(hi, hi, sum);
  }
  return sum;
}

// True when every float within 2^-kLog2Margin (relative) of v has the same
// fp16 rounding as v (fp16 rounding is monotonic, so the two ends decide).
// A fast estimate whose error is inside the margin then has the fp16
// rounding of the exact value.
template <int kLog2Margin = 19>
__device__ __forceinline__ bool f16_settled(float v) {
  constexpr float m = 1.0f / (float)(1u << kLog2Margin);
  _Float16 a = (_Float16)__fmul_rn(v, 1.0f - m);
  _Float16 b = (_Float16)__fmul_rn(v, 1.0f + m);
  return __builtin_bit_cast(uint16_t, a) == __builtin_bit_cast(uint16_t, b);
}

// logistic(g) = 1 / (1 + exp(-g)) with exp(-g) as 2^(-g log2 e) on the
// hardware exp2 and the hardware reciprocal. Relative error: |g| 2^-24 from
// the rounded argument plus about 2^-22 from the three instructions, at most
// 1.3 * 2^-20 while the result can still round to a nonzero fp16
// (g > -17.4), inside f16_settled's default 2^-19 margin. Below that the
// estimate and the exact value both round to 0, above g = 16 both to 1.
__device__ __forceinline__ float logistic_estimate(float g) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-g * 1.4426950408889634f));
}

// logistic with the correctly rounded fp32 exp (double, rounded once).
__device__ __forceinline__ float logistic_exact(float g) {
  return __fdiv_rn(1.0f, __fadd_rn(1.0f, (float)exp(-(double)g)));
}

// fp16(silu(h)) for an fp16 value h: silu(h) = h * logistic(h) in fp32.
__device__ __forceinline__ uint16_t silu16(float h) {
  float y = mul32(h, logistic_estimate(h));
  if (!f16_settled(y))
    y = mul32(h, logistic_exact(h));
  return f2h(y);
}

__device__ __forceinline__ float exp_cr(float x) { return (float)exp((double)x); }
__device__ __forceinline__ float log_cr(float x) { return (float)log((double)x); }

// stableSoftplus (Reference.metal:8-12) with correctly rounded exp and log.
__device__ __forceinline__ float stable_softplus(float x) {
  float e = exp_cr(-fabsf(x));
  float tail = e < 1e-4f ? mul32(e, __fsub_rn(1.0f, mul32(0.5f, e))) : log_cr(__fadd_rn(1.0f, e));
  return __fadd_rn(fmaxf(x, 0.0f), tail);
}

} // namespace llmi
