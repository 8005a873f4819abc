// Row arithmetic of the attention block shared by the standalone row
// kernels (norm_rope.hip) and the attention kernels that fuse it: normRope
// (Reference.metal:271-293 with rmsScale :98-103 and rotatePair :262-269)
// and the sigmoid output gate (sigmoidMul, Graph.metal:78-85; the gate of
// applyGqa, Reference.metal:350-353). Every product and fp16 rounding of the
// reference is kept (opaque() and explicit _rn operations, so the results do
// not depend on the including file's contraction setting); pow, cos, sin
// and exp are the correctly rounded fp32 functions (see exact_fp.hpp for
// the margin tests that let the fast fp32 evaluation decide).
#pragma once

#include "exact_fp.hpp"

#include <hip/hip_runtime.h>
#include <math.h>
#include <string.h>

namespace llmi {
namespace {

// fp16(cos(phase)), fp16(sin(phase)) of the correctly rounded fp32 values.
__device__ __forceinline__ float2 rope_cos_sin(float phase) {
  float s, c;
  sincosf(phase, &s, &c);
  // sincosf is within 2 ulp; 2^-21 relative is 4 to 8 ulp.
  if (!(f16_settled<21>(c) && f16_settled<21>(s))) {
    double sd, cd;
    sincos((double)phase, &sd, &cd);
    c = (float)cd;
    s = (float)sd;
  }
  return make_float2(round16(c), round16(s));
}

// pow(theta, 2 * pair / rotaryDim) correctly rounded to fp32.
__device__ __forceinline__ float rope_inv_freq(float theta, unsigned pair,
                                               unsigned rot) {
  float e = __fdiv_rn(2.0f * (float)pair, (float)rot);
  return (float)pow((double)theta, (double)e);
}

__device__ __forceinline__ float rms_scale_of(float sum, unsigned width, float eps) {
  return __fdiv_rn(1.0f, sqrt_cr(__fadd_rn(__fdiv_rn(sum, (float)width), eps)));
}

__device__ __forceinline__ float normed_f(float x, float scale, float w1) {
  return round16(mul32(mul32(x, scale), w1));
}
__device__ __forceinline__ float normed(uint16_t v, float scale, float w1) {
  return normed_f(h2f(v), scale, w1);
}

// rotatePair on fp16 values x, y (held in floats) and fp16 cos/sin.
__device__ __forceinline__ uint16_t rotate_x(float x, float y, float2 cs) {
  return f2h(opaque(round16(mul32(x, cs.x)) - round16(mul32(y, cs.y))));
}
__device__ __forceinline__ uint16_t rotate_y(float x, float y, float2 cs) {
  return f2h(opaque(round16(mul32(y, cs.x)) + round16(mul32(x, cs.y))));
}

// pow(theta, 2i/rotaryDim) for i < rotaryDim/2, computed once on the host
// (correctly rounded, as on the device) and passed in the kernel arguments;
// wider rotations compute it in the kernel.
constexpr unsigned kArgFreqs = 256;
struct RopeFreqs {
  float v[kArgFreqs];
};

// fp16(logistic(g)) of the correctly rounded fp32 exp.
__device__ __forceinline__ float logistic16(float g) {
  float s = logistic_estimate(g);
  if (!f16_settled(s))
    s = logistic_exact(g);
  return round16(s);
}

// fp16(fp16(logistic(gate)) * x), gate and x fp16 values held in floats.
__device__ __forceinline__ uint16_t gate16(float gate, float x) {
  return f2h(mul32(logistic16(gate), x));
}

// The output gate of the gated attention forms: fp16(fp16(logistic(gate)) *
// x), or fp16(gate * x) when the gate values are already activated
// (multiplyF16, the product of two fp16 values in fp32, rounded once).
__device__ __forceinline__ uint16_t gate_out(float gate, float x, bool activated) {
  return activated ? f2h(mul32(gate, x)) : gate16(gate, x);
}

__device__ __forceinline__ uint16_t gate_one(uint16_t g, uint16_t x) {
  return gate16(h2f(g), h2f(x));
}

// The host's correctly rounded pow (double, rounded once), per (theta, rot),
// kept for the next call with the same rotation.
static const RopeFreqs &host_freqs(float theta, unsigned rot) {
  static thread_local RopeFreqs table;
  static thread_local float cached_theta = 0.0f;
  static thread_local unsigned cached_rot = 0;
  unsigned half = rot / 2;
  if (half <= kArgFreqs && (cached_rot != rot || memcmp(&cached_theta, &theta, 4) != 0)) {
    for (unsigned i = 0; i < half; ++i)
      table.v[i] = (float)pow((double)theta, (double)(2.0f * (float)i / (float)rot));
    cached_theta = theta;
    cached_rot = rot;
  }
  return table;
}

} // namespace
} // namespace llmi
