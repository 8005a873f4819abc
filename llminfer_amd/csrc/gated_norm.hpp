// gatedRmsNorm's arithmetic (Reference.metal:228-259) -- out =
// fp16(fp16(x * rmsScale(x)) * weight * silu(gate)) -- shared by the
// standalone tile kernel and the kernels that fuse it behind DeltaUpdate, so
// that they agree bit for bit. Every step is an explicit rounded operation
// (exact_fp.hpp), independent of the including file's contraction setting.
#pragma once

#include "exact_fp.hpp"

namespace llmi {

// The sum of squares of a row continues in index order by fma (the
// reference's loop); its factor is 1 / sqrt(sum / width + eps), each step
// correctly rounded.
__device__ __forceinline__ float gated_norm_factor(float sum, unsigned width, float eps) {
  return __fdiv_rn(1.0f, sqrt_cr(__fadd_rn(__fdiv_rn(sum, (float)width), eps)));
}

// fp16(x * f) * w, in fp32.
__device__ __forceinline__ float gated_norm_scaled(float x, float f, float w) {
  return mul32(round16(mul32(x, f)), w);
}

// norm * silu(g) with the fast logistic; f16_settled() tells whether its
// fp16 rounding is that of the exact value.
__device__ __forceinline__ float gated_norm_silu_estimate(float norm, float g) {
  return mul32(norm, mul32(g, logistic_estimate(g)));
}
__device__ __forceinline__ float gated_norm_silu_exact(float norm, float g) {
  return mul32(norm, mul32(g, logistic_exact(g)));
}

// One output element, the estimate re-evaluated exactly when its rounding
// is not settled.
__device__ __forceinline__ _Float16 gated_norm_out(float x, float f, float w, float g) {
  const float norm = gated_norm_scaled(x, f, w);
  float y = gated_norm_silu_estimate(norm, g);
  if (!f16_settled(y))
    y = gated_norm_silu_exact(norm, g);
  return (_Float16)y;
}

// Eight elements of one row (8 fp16 values x and gate g packed in 16 bytes,
// weights w[0..8)), packed the same way: the estimates first, then the few
// whose rounding is not settled redone exactly, one pass per element
// position that some lane needs (lanes rarely need any, so a wave runs ~1
// exact pass per 8 elements instead of up to 8).
__device__ __forceinline__ uint4_t gated_norm_out8(uint4_t x, uint4_t gv, float f,
                                                   const float *w) {
  float norm[8], g[8], y[8];
  unsigned need = 0;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    norm[e] = gated_norm_scaled(h2f((uint16_t)(x[e / 2] >> (16 * (e & 1)))), f, w[e]);
    g[e] = h2f((uint16_t)(gv[e / 2] >> (16 * (e & 1))));
    y[e] = gated_norm_silu_estimate(norm[e], g[e]);
    need |= f16_settled(y[e]) ? 0u : 1u << e;
  }
  while (need) {
    const unsigned k = __builtin_ctz(need);
    need &= need - 1;
    float gk = g[0], nk = norm[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) {
      gk = k == (unsigned)e ? g[e] : gk;
      nk = k == (unsigned)e ? norm[e] : nk;
    }
    const float yk = gated_norm_silu_exact(nk, gk);
#pragma unroll
    for (int e = 0; e < 8; ++e)
      y[e] = k == (unsigned)e ? yk : y[e];
  }
  uint4_t o;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    o[e] = (uint32_t)f2h(y[2 * e]) | ((uint32_t)f2h(y[2 * e + 1]) << 16);
  return o;
}

// quantizeActivation's expressions for the fp16 rounding of eight fp32
// values y, chunk (lane & 3) of a 32-wide group held by four consecutive
// lanes, all four active: scale = max|x| / 127 over the group (1 for an
// all-zero or non-finite group), q = rint(clamp(x / scale, +-127)) (zeros
// for a non-finite group), written as 8 bytes at q; the group's first lane
// (first) writes *scale and raises *invalid for a non-finite group.
__device__ __forceinline__ void quantize_chunk8(const float *y, int8_t *q, float *scale,
                                                unsigned *invalid, bool first) {
  float x[8], max_abs = 0.0f;
  bool finite = true;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    x[e] = h2f(f2h(y[e]));
    finite = finite && __builtin_isfinite(x[e]);
    max_abs = fmaxf(max_abs, fabsf(x[e]));
  }
#pragma unroll
  for (int m = 1; m < 4; m *= 2) {
    max_abs = fmaxf(max_abs, __shfl_xor(max_abs, m, 4));
    finite = __shfl_xor((int)finite, m, 4) && finite;
  }
  const float qs = finite && max_abs > 0.0f ? __fdiv_rn(max_abs, 127.0f) : 1.0f;
  uint32_t words[2] = {0u, 0u};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    int r = 0;
    if (finite) {
      const float v = fminf(fmaxf(__fdiv_rn(x[e], qs), -127.0f), 127.0f);
      r = (int)__builtin_rintf(v);
    }
    words[e / 4] |= ((uint32_t)r & 0xFFu) << (8 * (e % 4));
  }
  reinterpret_cast<uint32_t *>(q)[0] = words[0];
  reinterpret_cast<uint32_t *>(q)[1] = words[1];
  if (first) {
    *scale = qs;
    if (!finite && invalid)
      atomicOr(invalid, 1u);
  }
}

} // namespace llmi
