// Causal GQA for shapes the tuned kernels do not cover (any head_dim up to
// 512, any Hq/Hkv ratio), e.g. the reference kernel test's head_dim 12
// (tests/FlashAttentionTest.mm:108-109). One wave per (token, query head);
// lanes split the channels, keys are visited in order with an fp32 online
// softmax -- the arithmetic of gqaFlashAttention (FlashAttention.metal:14-82)
// without its tiling. Correctness path only; not on any benchmarked shape.
#include "hip_common.hpp"
#include "kernels.hpp"

#include <math.h>

namespace llmi {
namespace {

constexpr int kMaxPerLane = 8; // 8 * 64 = 512 channels

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1)
    x += __shfl_xor(x, s);
  return x;
}

__global__ __launch_bounds__(64) void gqa_generic_kernel(
    const half_t *__restrict__ q, const half_t *__restrict__ kc,
    const half_t *__restrict__ vc, half_t *__restrict__ out, unsigned Hq,
    unsigned Hkv, unsigned D, unsigned P, float scoreScale) {
  const unsigned t = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
  const unsigned kvh = h / (Hq / Hkv);
  const unsigned visible = P + t + 1;
  const size_t rowStride = (size_t)Hkv * D;
  float qf[kMaxPerLane], o[kMaxPerLane];
#pragma unroll
  for (int i = 0; i < kMaxPerLane; ++i) {
    unsigned x = lane + 64u * i;
    qf[i] = x < D ? (float)q[((size_t)t * Hq + h) * D + x] : 0.0f;
    o[i] = 0.0f;
  }
  float m = -INFINITY, l = 0.0f;
  for (unsigned j = 0; j < visible; ++j) {
    const half_t *kr = kc + (size_t)j * rowStride + (size_t)kvh * D;
    const half_t *vr = vc + (size_t)j * rowStride + (size_t)kvh * D;
    float dot = 0.0f;
#pragma unroll
    for (int i = 0; i < kMaxPerLane; ++i) {
      unsigned x = lane + 64u * i;
      if (x < D)
        dot = fmaf(qf[i], (float)kr[x], dot);
    }
    float s = wave_sum(dot) * scoreScale;
    float mNew = fmaxf(m, s);
    float alpha = m == -INFINITY ? 0.0f : fast_exp2(m - mNew);
    float p = fast_exp2(s - mNew);
    l = l * alpha + p;
#pragma unroll
    for (int i = 0; i < kMaxPerLane; ++i) {
      unsigned x = lane + 64u * i;
      o[i] = o[i] * alpha + (x < D ? p * (float)vr[x] : 0.0f);
    }
    m = mNew;
  }
  float inv = 1.0f / l;
#pragma unroll
  for (int i = 0; i < kMaxPerLane; ++i) {
    unsigned x = lane + 64u * i;
    if (x < D)
      out[((size_t)t * Hq + h) * D + x] = (half_t)(o[i] * inv);
  }
}

} // namespace

bool generic_supported(const GqaShape &s) {
  return s.D >= 1 && s.D <= 64u * kMaxPerLane && s.Hkv >= 1 &&
         s.Hq % s.Hkv == 0 && s.T >= 1;
}

hipError_t launch_gqa_generic(const uint16_t *q, const uint16_t *k,
                              const uint16_t *v, uint16_t *out,
                              const GqaShape &s, hipStream_t stream) {
  float scale = kLog2e / sqrtf((float)s.D);
  hipLaunchKernelGGL(gqa_generic_kernel, dim3(s.T, s.Hq), dim3(64), 0, stream,
                     reinterpret_cast<const half_t *>(q),
                     reinterpret_cast<const half_t *>(k),
                     reinterpret_cast<const half_t *>(v),
                     reinterpret_cast<half_t *>(out), s.Hq, s.Hkv, s.D, s.P,
                     scale);
  return hipGetLastError();
}

} // namespace llmi
