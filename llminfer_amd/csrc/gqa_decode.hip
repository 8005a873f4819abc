// Causal GQA decode: split-K over the KV cache, one kernel.
//
// Replaces the reference's three decode dispatches gqaScores -> gqaSoftmax ->
// gqaValue (Reference.metal:303-323, Graph.metal:172-230) with one pass over
// K and V. It is an HBM-bandwidth problem (4 FLOP/byte), so no MFMA:
//
//  * grid = (split, kv head, token). A workgroup streams one key range of
//    one KV head and serves all G = Hq/Hkv query heads of the group, so each
//    K/V byte leaves HBM once.
//  * D/16 lanes share one key row: each lane holds 16 channels as two 16-byte
//    loads, so one wave instruction reads whole 256-byte row segments.
//  * q.k is v_dot2_f32_f16 on packed fp16 pairs, reduced over the lanes of a
//    key with DPP row permutes; softmax state (max, sum) and the output
//    accumulator are fp32, with exp2 on log2e-prescaled scores.
//  * each lane group runs its own online softmax over its keys; groups,
//    waves and finally splits are merged with the usual (m, l, o) rescale.
//  * the split merge happens in the same launch: every workgroup writes its
//    (m, l, o) partial to the workspace, and the last one to arrive for a
//    (token, kv head) -- found with a device-scope atomic ticket after a
//    release fence -- merges all partials and writes the fp16 output. It
//    then resets the ticket to zero, so the workspace is ready for the next
//    call without a memset.
#include "hip_common.hpp"
#include "kernels.hpp"

#include <algorithm>
#include <math.h>

#ifndef LLMI_DECODE_MAX_SPLITS
#define LLMI_DECODE_MAX_SPLITS 64
#endif
#ifndef LLMI_DECODE_TARGET_WGS
#define LLMI_DECODE_TARGET_WGS 512
#endif

namespace llmi {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kSlots = 4; // keys per lane group per iteration
constexpr unsigned kMaxSplits = LLMI_DECODE_MAX_SPLITS;

template <int D> struct DecodeGeom {
  static constexpr int LPK = D / 16;            // lanes per key row
  static constexpr int KPR = 64 / LPK;          // key rows per wave instruction
  static constexpr int WaveTile = KPR * kSlots; // keys per wave iteration
  static constexpr int Tile = WaveTile * kWaves;
};

struct Plan {
  unsigned splits, keysPerSplit;
};

unsigned tile_for(unsigned D) {
  switch (D) {
  case 64:
    return DecodeGeom<64>::Tile;
  case 128:
    return DecodeGeom<128>::Tile;
  default:
    return DecodeGeom<256>::Tile;
  }
}

Plan plan_for(const GqaShape &s) {
  unsigned tile = tile_for(s.D);
  unsigned visible = s.P + s.T;
  unsigned tiles = (visible + tile - 1) / tile;
  unsigned rows = s.T * s.Hkv;
  unsigned want = std::max(1u, (unsigned)LLMI_DECODE_TARGET_WGS / std::max(1u, rows));
  unsigned splits = std::min({want, tiles, kMaxSplits});
  unsigned perSplit = (tiles + splits - 1) / splits;
  splits = (tiles + perSplit - 1) / perSplit;
  return {splits, perSplit * tile};
}

struct WsLayout {
  size_t counters, ml, o, total;
};

// Tickets live in the fixed workspace header (kWorkspaceTicketBytes), which
// every kernel that uses tickets leaves zeroed; partials follow it.
WsLayout layout_for(const GqaShape &s, const Plan &p) {
  unsigned G = s.Hq / s.Hkv;
  size_t rows = (size_t)s.T * s.Hkv;
  WsLayout w;
  w.counters = 0;
  w.ml = kWorkspaceTicketBytes;
  w.o = w.ml + ((rows * p.splits * G * 2 * 4 + 255) / 256) * 256;
  w.total = w.o + rows * p.splits * G * s.D * 4;
  return w;
}

__device__ __forceinline__ float rescale(float m, float M) {
  return m == -INFINITY ? 0.0f : fast_exp2(m - M);
}

template <int D, int G>
__global__ __launch_bounds__(kThreads) void gqa_decode_kernel(
    const half_t *__restrict__ q, const half_t *__restrict__ kc,
    const half_t *__restrict__ vc, half_t *__restrict__ out,
    unsigned *__restrict__ tickets, float *__restrict__ wml,
    float *__restrict__ wo, unsigned Hq, unsigned Hkv, unsigned P,
    unsigned keysPerSplit, unsigned splits, float scoreScale) {
  using Geo = DecodeGeom<D>;
  constexpr int LPK = Geo::LPK, KPR = Geo::KPR;
  const unsigned split = blockIdx.x, kvh = blockIdx.y, t = blockIdx.z;
  const unsigned lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const unsigned slice = lane % LPK, kg = lane / LPK;
  const unsigned visible = P + t + 1;
  const unsigned begin = split * keysPerSplit;
  const unsigned end = min(begin + keysPerSplit, visible);
  const size_t rowStride = (size_t)Hkv * D;

  // Channels of this lane: [j*D/2 + slice*8, +8) for j = 0, 1.
  half8_t qv[G][2];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int j = 0; j < 2; ++j)
      qv[g][j] = load8(q + ((size_t)t * Hq + kvh * G + g) * D + j * (D / 2) + slice * 8);

  float m[G], l[G], o[G][16];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.0f;
#pragma unroll
    for (int x = 0; x < 16; ++x)
      o[g][x] = 0.0f;
  }

  const half_t *kbase = kc + (size_t)kvh * D + slice * 8;
  const half_t *vbase = vc + (size_t)kvh * D + slice * 8;
  for (unsigned base = begin; base < end; base += Geo::Tile) {
    const unsigned first = base + wave * Geo::WaveTile + kg;
    half8_t kx[kSlots][2], vx[kSlots][2];
#pragma unroll
    for (int n = 0; n < kSlots; ++n) {
      unsigned key = first + n * KPR;
      bool ok = key < end;
      size_t off = (size_t)(ok ? key : begin) * rowStride;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        kx[n][j] = load8(kbase + off + j * (D / 2));
        vx[n][j] = load8(vbase + off + j * (D / 2));
      }
    }
    float sc[kSlots][G];
#pragma unroll
    for (int n = 0; n < kSlots; ++n) {
      bool ok = first + n * KPR < end;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float acc = dot8(qv[g][0], kx[n][0], 0.0f);
        acc = dot8(qv[g][1], kx[n][1], acc);
        acc = group_sum<LPK>(acc);
        sc[n][g] = ok ? acc * scoreScale : -INFINITY;
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float tileMax = sc[0][g];
#pragma unroll
      for (int n = 1; n < kSlots; ++n)
        tileMax = fmaxf(tileMax, sc[n][g]);
      float mNew = fmaxf(m[g], tileMax);
      if (mNew == -INFINITY)
        continue; // nothing visible yet for this lane group
      float alpha = rescale(m[g], mNew);
      float p[kSlots];
      float psum = 0.0f;
#pragma unroll
      for (int n = 0; n < kSlots; ++n) {
        p[n] = rescale(sc[n][g], mNew);
        psum += p[n];
      }
      l[g] = l[g] * alpha + psum;
      m[g] = mNew;
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float acc = o[g][j * 8 + e] * alpha;
#pragma unroll
          for (int n = 0; n < kSlots; ++n)
            acc = fmaf(p[n], (float)vx[n][j][e], acc);
          o[g][j * 8 + e] = acc;
        }
    }
  }

  // Merge the KPR lane groups of the wave (lanes kg*LPK + slice).
#pragma unroll
  for (int stride = LPK; stride < 64; stride <<= 1) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float m2 = __shfl_xor(m[g], stride);
      float l2 = __shfl_xor(l[g], stride);
      float M = fmaxf(m[g], m2);
      float a1 = rescale(m[g], M), a2 = rescale(m2, M);
      l[g] = l[g] * a1 + l2 * a2;
#pragma unroll
      for (int x = 0; x < 16; ++x) {
        float o2 = __shfl_xor(o[g][x], stride);
        o[g][x] = o[g][x] * a1 + o2 * a2;
      }
      m[g] = M;
    }
  }

  // Merge the waves through LDS, then write this split's partial.
  __shared__ float sM[kWaves][G], sL[kWaves][G];
  __shared__ float sO[kWaves][G][D];
  if (lane == 0)
#pragma unroll
    for (int g = 0; g < G; ++g) {
      sM[wave][g] = m[g];
      sL[wave][g] = l[g];
    }
  if (kg == 0)
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = 0; e < 8; ++e)
          sO[wave][g][j * (D / 2) + slice * 8 + e] = o[g][j * 8 + e];
  __syncthreads();

  const size_t row = (size_t)t * Hkv + kvh;
  float *po = wo + (row * splits + split) * (size_t)(G * D);
  float *pml = wml + (row * splits + split) * (size_t)(G * 2);
  for (unsigned i = threadIdx.x; i < (unsigned)(G * D); i += kThreads) {
    unsigned g = i / D, x = i % D;
    float M = sM[0][g];
#pragma unroll
    for (int w = 1; w < kWaves; ++w)
      M = fmaxf(M, sM[w][g]);
    float acc = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w)
      acc += sO[w][g][x] * rescale(sM[w][g], M);
    po[i] = acc;
  }
  if (threadIdx.x < (unsigned)G) {
    unsigned g = threadIdx.x;
    float M = sM[0][g];
    for (int w = 1; w < kWaves; ++w)
      M = fmaxf(M, sM[w][g]);
    float L = 0.0f;
    for (int w = 0; w < kWaves; ++w)
      L += sL[w][g] * rescale(sM[w][g], M);
    pml[g * 2 + 0] = M;
    pml[g * 2 + 1] = L;
  }

  // Release this partial, take a ticket; the last arrival merges.
  __threadfence();
  __shared__ unsigned sTicket;
  __syncthreads();
  if (threadIdx.x == 0)
    sTicket = atomicAdd(&tickets[row], 1u);
  __syncthreads();
  if (sTicket != splits - 1)
    return;
  __threadfence(); // acquire: see every other split's partial

  __shared__ float sScale[kMaxSplits][G];
  __shared__ float sInvL[G];
  const float *rowMl = wml + row * splits * (size_t)(G * 2);
  if (threadIdx.x < (unsigned)G) {
    unsigned g = threadIdx.x;
    float M = -INFINITY;
    for (unsigned s = 0; s < splits; ++s)
      M = fmaxf(M, rowMl[s * G * 2 + g * 2]);
    float L = 0.0f;
    for (unsigned s = 0; s < splits; ++s) {
      float a = rescale(rowMl[s * G * 2 + g * 2], M);
      sScale[s][g] = a;
      L += a * rowMl[s * G * 2 + g * 2 + 1];
    }
    sInvL[g] = 1.0f / L;
  }
  __syncthreads();
  const float *rowO = wo + row * splits * (size_t)(G * D);
  for (unsigned i = threadIdx.x; i < (unsigned)(G * D); i += kThreads) {
    unsigned g = i / D, x = i % D;
    float acc = 0.0f;
    for (unsigned s = 0; s < splits; ++s)
      acc += rowO[(size_t)s * G * D + i] * sScale[s][g];
    out[((size_t)t * Hq + kvh * G + g) * D + x] = (half_t)(acc * sInvL[g]);
  }
  if (threadIdx.x == 0)
    tickets[row] = 0u; // ready for the next call
}

template <int D, int G>
hipError_t launch_dg(const GqaShape &s, const uint16_t *q, const uint16_t *k,
                     const uint16_t *v, uint16_t *out, void *ws,
                     hipStream_t stream) {
  Plan p = plan_for(s);
  WsLayout w = layout_for(s, p);
  char *base = static_cast<char *>(ws);
  float scale = kLog2e / sqrtf((float)D);
  hipLaunchKernelGGL((gqa_decode_kernel<D, G>), dim3(p.splits, s.Hkv, s.T),
                     dim3(kThreads), 0, stream,
                     reinterpret_cast<const half_t *>(q),
                     reinterpret_cast<const half_t *>(k),
                     reinterpret_cast<const half_t *>(v),
                     reinterpret_cast<half_t *>(out),
                     reinterpret_cast<unsigned *>(base + w.counters),
                     reinterpret_cast<float *>(base + w.ml),
                     reinterpret_cast<float *>(base + w.o), s.Hq, s.Hkv, s.P,
                     p.keysPerSplit, p.splits, scale);
  return hipGetLastError();
}

template <int D>
hipError_t launch_d(const GqaShape &s, const uint16_t *q, const uint16_t *k,
                    const uint16_t *v, uint16_t *out, void *ws,
                    hipStream_t stream) {
  switch (s.Hq / s.Hkv) {
  case 1:
    return launch_dg<D, 1>(s, q, k, v, out, ws, stream);
  case 2:
    return launch_dg<D, 2>(s, q, k, v, out, ws, stream);
  case 4:
    return launch_dg<D, 4>(s, q, k, v, out, ws, stream);
  case 8:
    return launch_dg<D, 8>(s, q, k, v, out, ws, stream);
  }
  return hipErrorInvalidValue;
}

} // namespace

bool decode_supported(const GqaShape &s) {
  unsigned G = s.Hkv ? s.Hq / s.Hkv : 0;
  bool dOk = s.D == 64 || s.D == 128 || s.D == 256;
  bool gOk = G == 1 || G == 2 || G == 4 || G == 8;
  return dOk && gOk && s.T >= 1 && s.T <= 64 &&
         (size_t)s.T * s.Hkv * 4 <= kWorkspaceTicketBytes;
}

size_t decode_workspace_bytes(const GqaShape &s) {
  return layout_for(s, plan_for(s)).total;
}

hipError_t launch_gqa_decode(const uint16_t *q, const uint16_t *k,
                             const uint16_t *v, uint16_t *out, void *ws,
                             const GqaShape &s, hipStream_t stream) {
  switch (s.D) {
  case 64:
    return launch_d<64>(s, q, k, v, out, ws, stream);
  case 128:
    return launch_d<128>(s, q, k, v, out, ws, stream);
  case 256:
    return launch_d<256>(s, q, k, v, out, ws, stream);
  }
  return hipErrorInvalidValue;
}

} // namespace llmi
