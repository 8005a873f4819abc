// Causal GQA prefill (flash attention) on fp16 MFMA for gfx950.
//
// Replaces gqaFlashAttention (FlashAttention.metal:1-83), which runs one query
// per SIMD group with a scalar per-key reduction. Here:
//
//  * one workgroup = (block of 32 query tokens, KV head); wave w computes the
//    q-head kvh*G + w for those tokens, so the G waves of a GQA group share
//    every K/V tile staged in LDS (K/V leave HBM/L2 once per token block).
//  * scores are computed transposed, S^T = K Q^T, with
//    v_mfma_f32_32x32x16_f16: the accumulator layout then gives each lane one
//    query row (lane % 32) and 16 keys, so the row max/sum of the online
//    softmax needs a single cross-lane exchange (lane ^ 32).
//  * the probabilities are converted to fp16 in registers and used directly
//    as the B operand of O^T += V^T P^T (same MFMA); the key order inside
//    each 16-key MFMA step follows the accumulator layout, and V is staged
//    transposed in LDS so the matching A operand is two 8-byte LDS reads.
//  * softmax state and accumulators are fp32; exp2 on log2e-prescaled
//    scores; fully masked key tiles are skipped (the loop stops at the causal
//    limit of the block's last token), partially masked tiles use -inf.
//  * the next K/V tile is fetched into registers while the current one is
//    being consumed, then written to LDS behind a barrier.
#include "hip_common.hpp"
#include "kernels.hpp"

#include <math.h>

namespace llmi {
namespace {

constexpr int BM = 32;  // query tokens per workgroup (= MFMA N)
constexpr int BN = 64;  // keys per tile
constexpr int KPAD = 8; // halves of padding per K row in LDS
constexpr int VPAD = 8; // halves of padding per V^T row in LDS

__device__ __forceinline__ float16_t mfma32(half8_t a, half8_t b, float16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

template <int D, int G>
__global__ __launch_bounds__(64 * G, 1) void gqa_prefill_kernel(
    const half_t *__restrict__ q, const half_t *__restrict__ kc,
    const half_t *__restrict__ vc, half_t *__restrict__ out, unsigned T,
    unsigned Hq, unsigned Hkv, unsigned P, float scoreScale) {
  constexpr int NT = 64 * G;
  constexpr int KS = D / 16;            // MFMA k-steps over channels
  constexpr int DT = D / 32;            // 32-channel output tiles
  constexpr int KROW = D + KPAD;        // LDS K row pitch (halves)
  constexpr int VROW = BN + VPAD;       // LDS V^T row pitch (halves)
  constexpr int KCHUNKS = BN * D / 8;   // 16-byte chunks per K tile
  constexpr int VPAIRS = (BN / 2) * (D / 8); // (key pair, 8-channel) chunks
  static_assert(KCHUNKS % NT == 0 && VPAIRS % NT == 0, "tile/threads");
  constexpr int KPT = KCHUNKS / NT, VPT = VPAIRS / NT;

  __shared__ __attribute__((aligned(16))) half_t sK[BN * KROW];
  __shared__ __attribute__((aligned(16))) half_t sVt[D * VROW];

  const unsigned tb = blockIdx.x, kvh = blockIdx.y;
  const unsigned tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const unsigned h = kvh * G + wave;
  const unsigned r = lane & 31u, hi = lane >> 5;
  const unsigned t0 = tb * BM;
  const unsigned tq = t0 + r;
  const bool rowValid = tq < T;
  const unsigned tLast = min(t0 + BM, T) - 1;
  const unsigned kend = P + tLast + 1; // keys [0, kend) can be visible
  const size_t rowStride = (size_t)Hkv * D;

  // Q^T as the MFMA B operand: lane holds query row r, channels
  // 16*s + 8*hi + [0, 8).
  half8_t qb[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    if (rowValid)
      qb[s] = load8(q + ((size_t)tq * Hq + h) * D + 16 * s + 8 * hi);
    else
      qb[s] = half8_t{0, 0, 0, 0, 0, 0, 0, 0};
  }

  float16_t oacc[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i)
    oacc[i] = float16_t{0};
  float mRun = -INFINITY, lRun = 0.0f;

  // Register staging of one K/V tile.
  half8_t kreg[KPT];
  half8_t vreg[VPT][2];
  auto fetch = [&](unsigned base) {
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      unsigned c = tid + NT * i;
      unsigned key = c / (D / 8), col = (c % (D / 8)) * 8;
      unsigned abs = base + key;
      kreg[i] = abs < kend ? load8(kc + (size_t)abs * rowStride + (size_t)kvh * D + col)
                           : half8_t{0, 0, 0, 0, 0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      unsigned c = tid + NT * i;
      unsigned kp = c % (BN / 2), cc = c / (BN / 2);
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        unsigned abs = base + 2 * kp + u;
        vreg[i][u] = abs < kend ? load8(vc + (size_t)abs * rowStride + (size_t)kvh * D + cc * 8)
                                : half8_t{0, 0, 0, 0, 0, 0, 0, 0};
      }
    }
  };
  auto stage = [&]() {
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      unsigned c = tid + NT * i;
      unsigned key = c / (D / 8), col = (c % (D / 8)) * 8;
      *reinterpret_cast<half8_t *>(&sK[key * KROW + col]) = kreg[i];
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      unsigned c = tid + NT * i;
      unsigned kp = c % (BN / 2), cc = c / (BN / 2);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        half2_t pair{vreg[i][0][e], vreg[i][1][e]};
        *reinterpret_cast<half2_t *>(&sVt[(cc * 8 + e) * VROW + 2 * kp]) = pair;
      }
    }
  };

  const unsigned tiles = (kend + BN - 1) / BN;
  fetch(0);
  for (unsigned it = 0; it < tiles; ++it) {
    const unsigned base = it * BN;
    __syncthreads(); // everyone is done reading the previous tile
    stage();
    __syncthreads();
    if (it + 1 < tiles)
      fetch(base + BN);

    // S^T = K Q^T for two 32-key halves of the tile.
    float16_t sacc[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      sacc[kt] = float16_t{0};
      const half_t *krow = &sK[(kt * 32 + r) * KROW + 8 * hi];
#pragma unroll
      for (int s = 0; s < KS; ++s)
        sacc[kt] = mfma32(load8(krow + 16 * s), qb[s], sacc[kt]);
    }

    // Scale, causal mask, tile max over this lane's 32 keys and its partner's.
    const bool needMask = base + BN > P + t0 + 1 || base + BN > kend;
    float tmax = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        float s = sacc[kt][v] * scoreScale;
        if (needMask) {
          unsigned key = base + kt * 32 + 8 * (v / 4) + 4 * hi + (v % 4);
          if (!rowValid || key > P + tq)
            s = -INFINITY;
        }
        sacc[kt][v] = s;
        tmax = fmaxf(tmax, s);
      }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
    const float mNew = fmaxf(mRun, tmax);
    const bool live = mNew != -INFINITY;
    const float alpha = (live && mRun != -INFINITY) ? fast_exp2(mRun - mNew) : (live ? 0.0f : 1.0f);
    float psum = 0.0f;
    half8_t pb[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float s = sacc[ks / 2][8 * (ks % 2) + e];
        float p = live ? fast_exp2(s - mNew) : 0.0f;
        psum += p;
        pb[ks][e] = (half_t)p;
      }
    lRun = lRun * alpha + psum;
    mRun = live ? mNew : mRun;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
      oacc[dt] *= alpha;

    // O^T += V^T P^T. A operand: channel row 32*dt + r, keys
    // 16*ks + 4*hi + [0,4) and 16*ks + 8 + 4*hi + [0,4).
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const half_t *vrow = &sVt[(32 * dt + r) * VROW + 4 * hi];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        half4_t lo = *reinterpret_cast<const half4_t *>(vrow + 16 * ks);
        half4_t up = *reinterpret_cast<const half4_t *>(vrow + 16 * ks + 8);
        half8_t a{lo[0], lo[1], lo[2], lo[3], up[0], up[1], up[2], up[3]};
        oacc[dt] = mfma32(a, pb[ks], oacc[dt]);
      }
    }
  }

  const float lTot = lRun + __shfl_xor(lRun, 32);
  if (!rowValid)
    return;
  const float inv = 1.0f / lTot;
  half_t *orow = out + ((size_t)tq * Hq + h) * D;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      half4_t v{(half_t)(oacc[dt][4 * g4 + 0] * inv), (half_t)(oacc[dt][4 * g4 + 1] * inv),
                (half_t)(oacc[dt][4 * g4 + 2] * inv), (half_t)(oacc[dt][4 * g4 + 3] * inv)};
      *reinterpret_cast<half4_t *>(orow + 32 * dt + 8 * g4 + 4 * hi) = v;
    }
}

template <int D, int G>
hipError_t launch_dg(const GqaShape &s, const uint16_t *q, const uint16_t *k,
                     const uint16_t *v, uint16_t *out, hipStream_t stream) {
  float scale = kLog2e / sqrtf((float)D);
  dim3 grid((s.T + BM - 1) / BM, s.Hkv);
  hipLaunchKernelGGL((gqa_prefill_kernel<D, G>), grid, dim3(64 * G), 0, stream,
                     reinterpret_cast<const half_t *>(q),
                     reinterpret_cast<const half_t *>(k),
                     reinterpret_cast<const half_t *>(v),
                     reinterpret_cast<half_t *>(out), s.T, s.Hq, s.Hkv, s.P,
                     scale);
  return hipGetLastError();
}

template <int D>
hipError_t launch_d(const GqaShape &s, const uint16_t *q, const uint16_t *k,
                    const uint16_t *v, uint16_t *out, hipStream_t stream) {
  switch (s.Hq / s.Hkv) {
  case 1:
    return launch_dg<D, 1>(s, q, k, v, out, stream);
  case 2:
    return launch_dg<D, 2>(s, q, k, v, out, stream);
  case 4:
    return launch_dg<D, 4>(s, q, k, v, out, stream);
  case 8:
    return launch_dg<D, 8>(s, q, k, v, out, stream);
  }
  return hipErrorInvalidValue;
}

} // namespace

bool prefill_supported(const GqaShape &s) {
  unsigned G = s.Hkv ? s.Hq / s.Hkv : 0;
  return (s.D == 128 || s.D == 256) && (G == 1 || G == 2 || G == 4 || G == 8) &&
         s.T >= 1;
}

hipError_t launch_gqa_prefill(const uint16_t *q, const uint16_t *k,
                              const uint16_t *v, uint16_t *out,
                              const GqaShape &s, hipStream_t stream) {
  if (s.D == 128)
    return launch_d<128>(s, q, k, v, out, stream);
  return launch_d<256>(s, q, k, v, out, stream);
}

} // namespace llmi
