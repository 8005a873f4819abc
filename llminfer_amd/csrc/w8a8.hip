// The W8A8 projection path of the whole-graph plan: activation quantization,
// int8 x int8 projections with per-32-group scales and the fused storeLinear
// epilogues, and the embeddings.
//
// Reference kernels: quantizeActivation and embeddingW8 (Graph.metal:16-68),
// linearW8A8Gemv / linearW8A8Gemm (W8A8.metal:28-113), storeLinear and
// embedding (Reference.metal:14-58).
//
//  * quantize: one lane per 32-wide group (64 bytes of fp16 in, 32 int8 and
//    a scale out). x / scale is the IEEE quotient; the reference's
//    floor/fraction tie rule is round half to even (v_rndne_f32).
//  * GEMV (one row, the decode step): bound by the weight stream. A
//    one-wave workgroup serves 4 output columns with 16 lanes each, the
//    reference's linearW8GemvLanes: lane l takes groups l, l + 16, ... of its
//    column, so the 16 lanes of a column read 512 contiguous weight bytes per
//    step. Group dots run on v_dot4_i32_i8 (exact int32); each group adds
//    (float(dot) * a) * w to the lane's fp32 sum in group order and the lanes
//    meet by the xor butterfly, which is the reference's arithmetic order, so
//    outputs are its bits. Eight groups' weight loads go out before their
//    arithmetic.
//  * GEMM (several rows): the reference's 8 lanes per column. Below 16 rows,
//    a lane holds 4 rows and a weight group is loaded once for them; from 16
//    rows the group dots come from int8 MFMA over 32 x 32 tiles, with the 8
//    lanes' fp32 sums kept apart and merged in the butterfly's order.
#include "exact_fp.hpp"
#include "gated_norm.hpp"
#include "hip_common.hpp"
#include "kernels.hpp"
#include "linear_store.hpp"

#include "llminfer_hip.h"

namespace llmi {
namespace {

constexpr unsigned kGroup = 32;

__device__ __forceinline__ int dot4x4(uint4_t a, uint4_t b, int acc) {
#pragma unroll
  for (int e = 0; e < 4; ++e)
    acc = __builtin_amdgcn_sdot4((int)a[e], (int)b[e], acc, false);
  return acc;
}

// The group's exact int32 dot: 32 int8 activations by 32 int8 weights.
__device__ __forceinline__ int group_dot(uint4_t a0, uint4_t a1, uint4_t w0, uint4_t w1) {
  return dot4x4(a1, w1, dot4x4(a0, w0, 0));
}

// One group's term added to a lane's sum: acc + (float(dot) * a) * w, each
// operation rounded on its own.
__device__ __forceinline__ float add_term(float acc, int dot, float a, float w) {
  return __fadd_rn(acc, __fmul_rn(__fmul_rn((float)dot, a), w));
}

// --------------------------------------------------------------- quantize

// One 32-wide group (zeros past the row's end): scale = max|x| / 127 (1 for
// an all-zero or non-finite group), q = x / scale clamped to +-127 and
// rounded half to even (zeros for a non-finite group), written as 32 bytes
// at dst (16-byte aligned). Returns the scale.
__device__ __forceinline__ float quantize_group(const float *x, int8_t *dst, bool &finite) {
  float max_abs = 0.0f;
  finite = true;
#pragma unroll
  for (unsigned j = 0; j < kGroup; ++j) {
    finite = finite && __builtin_isfinite(x[j]);
    max_abs = fmaxf(max_abs, fabsf(x[j]));
  }
  const float scale = finite && max_abs > 0.0f ? __fdiv_rn(max_abs, 127.0f) : 1.0f;
  uint4_t packed[2];
#pragma unroll
  for (unsigned j = 0; j < kGroup; j += 4) {
    uint32_t word = 0;
#pragma unroll
    for (unsigned e = 0; e < 4; ++e) {
      int r = 0;
      if (finite) {
        const float v = fminf(fmaxf(__fdiv_rn(x[j + e], scale), -127.0f), 127.0f);
        r = (int)__builtin_rintf(v);
      }
      word |= ((uint32_t)r & 0xFFu) << (8 * e);
    }
    packed[j / 16][(j / 4) % 4] = word;
  }
  uint4_t *d = reinterpret_cast<uint4_t *>(dst);
  d[0] = packed[0];
  d[1] = packed[1];
  return scale;
}


// Rows of whole 32-wide groups from 16-byte-aligned input: a lane per chunk
// of eight values, four lanes a group (quantize_chunk8, the expressions
// above): a group's 32 divides spread over its four lanes instead of one
// lane's sequence.
__global__ __launch_bounds__(256) void quantize_chunks_kernel(const uint16_t *__restrict__ in,
                                                              int8_t *__restrict__ q,
                                                              float *__restrict__ scales,
                                                              unsigned *invalid, unsigned chunks) {
  const unsigned c = blockIdx.x * 256 + threadIdx.x;
  if (c >= chunks) // (chunks is a multiple of 4: a group's lanes leave together)
    return;
  const uint4_t v = reinterpret_cast<const uint4_t *>(in)[c];
  float y[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    y[2 * e] = h2f((uint16_t)(v[e] & 0xFFFFu));
    y[2 * e + 1] = h2f((uint16_t)(v[e] >> 16));
  }
  quantize_chunk8(y, q + 8 * (size_t)c, scales + c / 4, invalid, (c & 3u) == 0);
}

__global__ __launch_bounds__(256) void quantize_kernel(const uint16_t *__restrict__ in,
                                                       int8_t *__restrict__ q,
                                                       float *__restrict__ scales,
                                                       unsigned *invalid, unsigned rows,
                                                       unsigned width, unsigned groups,
                                                       bool vec) {
  const unsigned i = blockIdx.x * 256 + threadIdx.x;
  if (i >= rows * groups)
    return;
  const unsigned row = i / groups, begin = (i % groups) * kGroup;
  const unsigned length = min(kGroup, width - begin);
  const uint16_t *group = in + (size_t)row * width + begin;
  float x[kGroup];
  if (vec && length == kGroup) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint4_t v = reinterpret_cast<const uint4_t *>(group)[c];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x[8 * c + 2 * e] = h2f((uint16_t)(v[e] & 0xFFFFu));
        x[8 * c + 2 * e + 1] = h2f((uint16_t)(v[e] >> 16));
      }
    }
  } else {
#pragma unroll
    for (unsigned j = 0; j < kGroup; ++j)
      x[j] = j < length ? h2f(group[j]) : 0.0f;
  }
  bool finite;
  scales[i] = quantize_group(x, q + (size_t)i * kGroup, finite);
  if (!finite && invalid)
    atomicOr(invalid, 1u);
}

// residualAdd -> rmsNorm -> quantizeActivation of a row, in three phases that
// the fused launches below share (Reference.metal:105-126, Graph.metal:
// 33-68).
//
// Phase 1: the sum fp16(a + b) (the next residual; written when sum_out is
// given) staged in LDS as fp32, the row padded to whole groups by zeros,
// next to 1 + w. Without b the input row is staged as it is.
template <bool kAdd, unsigned kThreads = 256>
__device__ __forceinline__ void stage_norm_row(const uint16_t *__restrict__ a,
                                               const uint16_t *__restrict__ b, uint16_t *sum_out,
                                               const float *__restrict__ w, float *srow,
                                               float *sw, unsigned width, unsigned padded,
                                               unsigned t) {
  // Eight elements a lane in flight at once: one memory round trip per
  // eight, not per element.
  constexpr unsigned kBatch = 8;
  for (unsigned i0 = 0; i0 < padded; i0 += kBatch * kThreads) {
    uint16_t ha[kBatch], hb[kBatch];
    float wi[kBatch];
#pragma unroll
    for (unsigned j = 0; j < kBatch; ++j) {
      const unsigned i = i0 + j * kThreads + t;
      const bool in = i < width;
      ha[j] = in ? a[i] : (uint16_t)0;
      hb[j] = in && kAdd ? b[i] : (uint16_t)0;
      wi[j] = in ? w[i] : 0.0f;
    }
#pragma unroll
    for (unsigned j = 0; j < kBatch; ++j) {
      const unsigned i = i0 + j * kThreads + t;
      if (i >= padded)
        break;
      float x = 0.0f, w1 = 1.0f;
      if (i < width) {
        uint16_t h = ha[j];
        if (kAdd) {
          h = f2h(__fadd_rn(h2f(h), h2f(hb[j])));
          if (sum_out)
            sum_out[i] = h;
        }
        x = h2f(h);
        w1 = 1.0f + wi[j];
      }
      srow[i] = x;
      sw[i] = w1;
    }
  }
}

// Phase 2 (one lane): the norm's sequential fp32 fma sum over the staged row
// (fma(0, 0, sum) == sum for the padding, sum >= +0).
__device__ __forceinline__ float norm_row_sum(const float *srow, unsigned padded) {
  const float4 *v = reinterpret_cast<const float4 *>(srow);
  float sum = 0.0f;
#pragma unroll 8
  for (unsigned c = 0; c < padded / 4; ++c) {
    const float4 x4 = v[c];
    sum = __builtin_fmaf(x4.x, x4.x, sum);
    sum = __builtin_fmaf(x4.y, x4.y, sum);
    sum = __builtin_fmaf(x4.z, x4.z, sum);
    sum = __builtin_fmaf(x4.w, x4.w, sum);
  }
  return sum;
}

// Phase 3: eight lanes a group, four elements a lane: the group's max |y|
// and finiteness by lane swaps (exact in any order), then each lane
// quantizes its four with the standalone kernel's expressions into q (a
// word per lane) and the group's scale into scales.
template <unsigned kThreads = 256>
__device__ __forceinline__ void quantize_norm_row(const float *srow, const float *sw, float scale,
                                                  unsigned width, unsigned groups, unsigned t,
                                                  uint32_t *q, float *scales, unsigned *invalid) {
  const unsigned sub = t % 8;
  for (unsigned g0 = 0; g0 < groups; g0 += kThreads / 8) {
    const unsigned g = g0 + t / 8;
    const bool live = g < groups;
    const unsigned i0 = (live ? g : 0) * kGroup + 4 * sub;
    float y[4];
    float max_abs = 0.0f;
    bool finite = true;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const unsigned i = i0 + e;
      y[e] = i < width ? normed_f(srow[i], scale, sw[i]) : 0.0f;
      finite = finite && __builtin_isfinite(y[e]);
      max_abs = fmaxf(max_abs, fabsf(y[e]));
    }
#pragma unroll
    for (int m = 1; m < 8; m *= 2) {
      max_abs = fmaxf(max_abs, __shfl_xor(max_abs, m, 8));
      finite = __shfl_xor((int)finite, m, 8) && finite;
    }
    if (!live)
      continue;
    const float qs = finite && max_abs > 0.0f ? __fdiv_rn(max_abs, 127.0f) : 1.0f;
    uint32_t word = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      int r = 0;
      if (finite) {
        const float v = fminf(fmaxf(__fdiv_rn(y[e], qs), -127.0f), 127.0f);
        r = (int)__builtin_rintf(v);
      }
      word |= ((uint32_t)r & 0xFFu) << (8 * e);
    }
    q[g * (kGroup / 4) + sub] = word;
    if (sub == 0) {
      scales[g] = qs;
      if (!finite && invalid)
        atomicOr(invalid, 1u);
    }
  }
}

// The three in one launch, a workgroup per row; the bits equal the three
// launches' (residualAdd, rmsNorm, quantizeActivation).
template <bool kAdd>
__global__ __launch_bounds__(256) void add_norm_quantize_kernel(
    const uint16_t *__restrict__ a, const uint16_t *__restrict__ b, uint16_t *sum_out,
    const float *__restrict__ w, int8_t *__restrict__ q, float *__restrict__ scales,
    unsigned *invalid, unsigned width, unsigned groups, float eps) {
  extern __shared__ __align__(16) float srow[]; // the row, then 1 + w, padded
  __shared__ float sscale;
  const unsigned row = blockIdx.x, t = threadIdx.x;
  const size_t base = (size_t)row * width;
  const unsigned padded = groups * kGroup;
  float *sw = srow + padded;
  stage_norm_row<kAdd>(a + base, kAdd ? b + base : nullptr, kAdd ? sum_out + base : nullptr, w,
                       srow, sw, width, padded, t);
  __syncthreads();
  if (t == 0)
    sscale = rms_scale_of(norm_row_sum(srow, padded), width, eps);
  __syncthreads();
  quantize_norm_row(srow, sw, sscale, width, groups, t,
                    reinterpret_cast<uint32_t *>(q + (size_t)row * groups * kGroup),
                    scales + (size_t)row * groups, invalid);
}

// ------------------------------------------------------------------- GEMV

struct W8Args {
  unsigned outputWidth, firstRow, groups, rows, columns, epilogue, block;
};

// One wave per workgroup (4 columns): even the 2560-column down projection
// spreads over 640 workgroups. A lane requests the weights of 8 of its
// groups (256 bytes) before using any; the activations, read by every
// column, come from L1/L2.
constexpr int kGemvLanes = 16, kGemvThreads = 64, kGemvCols = kGemvThreads / kGemvLanes;
constexpr int kGemvUnroll = 8;

__global__ __launch_bounds__(kGemvThreads) void gemv_kernel(
    const int8_t *__restrict__ act, const float *__restrict__ as, const int8_t *__restrict__ w,
    const uint16_t *__restrict__ ws, void *out, const void *aux, const float *bias, W8Args p) {
  const unsigned col = blockIdx.x * kGemvCols + threadIdx.x / kGemvLanes;
  const unsigned l = threadIdx.x % kGemvLanes;
  float acc = 0.0f;
  if (col < p.columns) {
    const uint4_t *wrow = reinterpret_cast<const uint4_t *>(w + (size_t)col * p.groups * kGroup);
    const uint4_t *arow = reinterpret_cast<const uint4_t *>(act);
    const uint16_t *wsrow = ws + (size_t)col * p.groups;
    for (unsigned g0 = l; g0 < p.groups; g0 += kGemvLanes * kGemvUnroll) {
      uint4_t wv[kGemvUnroll][2];
      float wsv[kGemvUnroll];
#pragma unroll
      for (int u = 0; u < kGemvUnroll; ++u) {
        const unsigned g = min(g0 + kGemvLanes * u, p.groups - 1); // clamped: in bounds
        wv[u][0] = __builtin_nontemporal_load(wrow + 2 * g);
        wv[u][1] = __builtin_nontemporal_load(wrow + 2 * g + 1);
        wsv[u] = h2f(wsrow[g]);
      }
#pragma unroll
      for (int u = 0; u < kGemvUnroll; ++u) {
        const unsigned g = g0 + kGemvLanes * u;
        if (g < p.groups)
          acc = add_term(acc, group_dot(arow[2 * g], arow[2 * g + 1], wv[u][0], wv[u][1]),
                         as[g], wsv[u]);
      }
    }
  }
  // The xor butterfly of the column's 16 lanes (every lane ends with the
  // same sum: fp32 addition is commutative).
#pragma unroll
  for (int m = kGemvLanes / 2; m >= 1; m /= 2)
    acc = __fadd_rn(acc, __shfl_xor(acc, m, kGemvLanes));
  if (l == 0 && col < p.columns) {
    const unsigned column = p.firstRow + col;
    store_linear(out, aux, bias, column, column, p.epilogue, p.block, acc);
  }
}

// Long rows (more than 112 groups: 8 steps a lane or more): four waves share the
// same 4 columns. Wave w computes the group terms (float(dot) * a) * w of the
// w-th quarter of every lane's groups (kPer steps of 16 groups), all its
// loads issued at once, into LDS; wave 0 then adds each lane's terms in
// group order -- the same fp32 sums as one lane would form -- and finishes
// as above. The workgroup's threads first request the activation row and
// its scales, then the weights, and stage the row in LDS once its loads
// (the oldest) are back: read from memory in the dot loop, each step's
// activations waited for the whole weight stream before them and for one
// another. kPer is a template parameter so that every load count is fixed
// and the waits count only what they need.
constexpr int kSplitWaves = 4, kSplitMaxSteps = 64; // groups per lane <= 64
constexpr int kSplitPer = kSplitMaxSteps / kSplitWaves;

template <int kPer>
__global__ __launch_bounds__(64 * kSplitWaves) void gemv_split_kernel(
    const int8_t *__restrict__ act, const float *__restrict__ as, const int8_t *__restrict__ w,
    const uint16_t *__restrict__ ws, void *out, const void *aux, const float *bias, W8Args p) {
  constexpr unsigned kThreads = 64 * kSplitWaves, kGroups = kSplitWaves * kPer * kGemvLanes;
  constexpr int kA = (2 * kGroups + kThreads - 1) / kThreads, kS = (kGroups + kThreads - 1) / kThreads;
  __shared__ float sT[kSplitWaves * kPer][64];
  __shared__ uint4_t sAct[2 * kGroups];
  __shared__ float sAs[kGroups];
  const unsigned tid = threadIdx.x, wave = tid / 64, t = tid % 64;
  const unsigned col = blockIdx.x * kGemvCols + t / kGemvLanes;
  const unsigned l = t % kGemvLanes;
  const unsigned i0 = wave * kPer;
  const unsigned nA = 2 * p.groups; // 16-byte pieces of the row
  const uint4_t *arow = reinterpret_cast<const uint4_t *>(act);
  uint4_t aReg[kA];
  float sReg[kS];
#pragma unroll
  for (int k = 0; k < kA; ++k)
    aReg[k] = arow[min(tid + k * kThreads, nA - 1)]; // clamped: in bounds
#pragma unroll
  for (int k = 0; k < kS; ++k)
    sReg[k] = as[min(tid + k * kThreads, p.groups - 1)];
  asm volatile("" ::: "memory"); // (keeps these loads ahead of the weights')
  // The weights (a column past the end reads the last one and stores
  // nothing); the scales stay fp16 bits, one a register, until the
  // products, so that nothing waits for them here.
  const bool live = col < p.columns;
  const unsigned cc = live ? col : p.columns - 1;
  const uint4_t *wrow = reinterpret_cast<const uint4_t *>(w + (size_t)cc * p.groups * kGroup);
  const uint16_t *wsrow = ws + (size_t)cc * p.groups;
  uint4_t wv[kPer][2];
  uint32_t wsv[kPer];
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const unsigned g = min(l + kGemvLanes * (i0 + u), p.groups - 1); // clamped: in bounds
    wv[u][0] = __builtin_nontemporal_load(wrow + 2 * g);
    wv[u][1] = __builtin_nontemporal_load(wrow + 2 * g + 1);
    wsv[u] = wsrow[g];
  }
#pragma unroll
  for (int k = 0; k < kA; ++k)
    if (tid + k * kThreads < nA)
      sAct[tid + k * kThreads] = aReg[k];
#pragma unroll
  for (int k = 0; k < kS; ++k)
    if (tid + k * kThreads < p.groups)
      sAs[tid + k * kThreads] = sReg[k];
  lds_sync(); // LDS only: the weights stay in flight
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const unsigned g = l + kGemvLanes * (i0 + u);
    if (live && g < p.groups)
      sT[i0 + u][t] = __fmul_rn(
          __fmul_rn((float)group_dot(sAct[2 * g], sAct[2 * g + 1], wv[u][0], wv[u][1]), sAs[g]),
          h2f((uint16_t)wsv[u]));
  }
  __syncthreads();
  if (wave != 0)
    return;
  float acc = 0.0f;
  if (col < p.columns)
    for (unsigned i = 0; l + kGemvLanes * i < p.groups; ++i)
      acc = __fadd_rn(acc, sT[i][t]);
#pragma unroll
  for (int m = kGemvLanes / 2; m >= 1; m /= 2)
    acc = __fadd_rn(acc, __shfl_xor(acc, m, kGemvLanes));
  if (l == 0 && col < p.columns) {
    const unsigned column = p.firstRow + col;
    store_linear(out, aux, bias, column, column, p.epilogue, p.block, acc);
  }
}

// ------------------------------------------------------------------- GEMM

constexpr int kGemmLanes = 8, kGemmCols = 256 / kGemmLanes, kGemmRows = 4;

__global__ __launch_bounds__(256) void gemm_kernel(
    const int8_t *__restrict__ act, const float *__restrict__ as, const int8_t *__restrict__ w,
    const uint16_t *__restrict__ ws, void *out, const void *aux, const float *bias, W8Args p) {
  const unsigned col = blockIdx.x * kGemmCols + threadIdx.x / kGemmLanes;
  const unsigned l = threadIdx.x % kGemmLanes;
  const unsigned row0 = blockIdx.y * kGemmRows;
  const unsigned nr = min((unsigned)kGemmRows, p.rows - row0);
  float acc[kGemmRows] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (col < p.columns) {
    const uint4_t *wrow = reinterpret_cast<const uint4_t *>(w + (size_t)col * p.groups * kGroup);
    const uint16_t *wsrow = ws + (size_t)col * p.groups;
    for (unsigned g = l; g < p.groups; g += kGemmLanes) {
      const uint4_t w0 = __builtin_nontemporal_load(wrow + 2 * g);
      const uint4_t w1 = __builtin_nontemporal_load(wrow + 2 * g + 1);
      const float wsv = h2f(wsrow[g]);
#pragma unroll
      for (int r = 0; r < kGemmRows; ++r) {
        const unsigned row = row0 + min((unsigned)r, nr - 1); // clamped: in bounds
        const uint4_t *arow =
            reinterpret_cast<const uint4_t *>(act + ((size_t)row * p.groups + g) * kGroup);
        const int dot = group_dot(arow[0], arow[1], w0, w1);
        if ((unsigned)r < nr)
          acc[r] = add_term(acc[r], dot, as[(size_t)row * p.groups + g], wsv);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < kGemmRows; ++r)
#pragma unroll
    for (int m = kGemmLanes / 2; m >= 1; m /= 2)
      acc[r] = __fadd_rn(acc[r], __shfl_xor(acc[r], m, kGemmLanes));
  if (l == 0 && col < p.columns) {
    const unsigned column = p.firstRow + col;
    for (unsigned r = 0; r < nr; ++r)
      store_linear(out, aux, bias, (size_t)(row0 + r) * p.outputWidth + column, column,
                   p.epilogue, p.block, acc[r]);
  }
}

// ------------------------------------------------------------- MFMA GEMM

// Many rows (prefill): the group dots come from v_mfma_i32_32x32x32_i8, one
// instruction per 32-row x 32-column tile and group (K = 32 is exactly one
// group, so each int32 result is the group's exact dot), and the VALU adds
// (float(dot) * a) * w to fp32 sums. The reference's GEMM gives each output 8
// lanes, lane l summing groups l, l + 8, ... in order before the xor
// butterfly; here those 8 lane classes are split over the workgroup's waves
// (wave w takes the groups g = w (mod waves), i.e. classes w and w + 4 with 4
// waves, class w with 8), each class keeping its own fp32 sum per output, and
// the sums meet through LDS in the butterfly's order
// ((c0 + c4) + (c2 + c6)) + ((c1 + c5) + (c3 + c7)). So the bits are the
// reference's. The per-element fp32 work (convert, two products, add: 4 VALU
// operations per output and group) is the floor of the kernel.
//
// Staging: a step covers kPer groups per wave, i.e. (waves x kPer x 32)
// consecutive bytes of each of the tile's 32 activation rows and 32 weight
// rows, plus their scales. Each thread loads 16-byte chunks of each operand
// (whole cache lines per row) kDepth - 1 steps ahead into registers and
// writes them to the other of two LDS buffers, before the current step's
// arithmetic (kEarly) or after it; one barrier a step. Rows are padded by 16
// bytes so the MFMA operand reads (lane i: row i % 32) meet no bank
// conflicts. Large grids (at least kMfmaManyTiles tiles) take 8 waves, one
// group each a step, loads one step ahead, staged early: 71 VGPRs, so three
// workgroups share a CU. Small grids (the 2560-column down projection) take
// loads three steps ahead, staged late, which hides more latency inside a
// workgroup when few workgroups share a CU.
//
// Operand layout: lane i supplies row (column) i % 32 of the tile and the
// 16 bytes (i / 32) * 16 of the group for both operands; any K order shared
// by the two operands gives the same exact integer dot. Lane i's results are
// column i % 32 and rows 8 * (r / 4) + 4 * (i / 32) + r % 4 of register r.
//
// Workgroups sharing a column tile run on one XCD (blockIdx % 8 selects the
// XCD), so each weight tile is read from HBM once and then from that XCD's L2.
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr unsigned kTile = 32, kMfmaMinRows = 16, kMfmaManyTiles = 512;

// A step stages kWaves * kPer groups; loads run kDepth - 1 steps ahead.
template <int kWaves, int kPer, int kDepth> struct MfmaCfg {
  static constexpr unsigned kSpan = kWaves * kPer;             // groups per step
  static constexpr unsigned kPitch = kSpan * kGroup + 16;      // bytes per staged row
  static constexpr unsigned kOperand = kTile * kPitch;         // one operand tile
  static constexpr unsigned kScales = kSpan * kTile * 4;       // [group][32] fp32
  static constexpr unsigned kBuffer = 2 * kOperand + 2 * kScales;
  static constexpr unsigned kSums = kWaves * kTile * kTile * 4;
  static constexpr unsigned kBytes = 2 * kBuffer > kSums ? 2 * kBuffer : kSums;
};

template <int kWaves, int kPer, int kDepth, bool kEarly>
__global__ __launch_bounds__(64 * kWaves) void gemm_mfma_kernel(
    const int8_t *__restrict__ act, const float *__restrict__ as, const int8_t *__restrict__ w,
    const uint16_t *__restrict__ ws, void *out, const void *aux, const float *bias, W8Args p,
    unsigned rowTiles) {
  using L = MfmaCfg<kWaves, kPer, kDepth>;
  constexpr int kClasses = 8 / kWaves; // lane classes per wave
  static_assert(L::kSpan % 8 == 0, "a step must hold whole sets of the 8 lane classes");
  __shared__ __align__(16) unsigned char lds[L::kBytes];
  const unsigned nwg = gridDim.x, b = blockIdx.x, x = b % 8;
  const unsigned v = x * (nwg / 8) + min(x, nwg % 8) + b / 8;
  const unsigned row0 = (v % rowTiles) * kTile, col0 = (v / rowTiles) * kTile;
  const unsigned tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
  const size_t k = (size_t)p.groups * kGroup;
  const unsigned nsteps = (p.groups + L::kSpan - 1) / L::kSpan;

  // Staging roles: chunks schunk + 2 * kWaves * j (16 bytes each, j < kPer)
  // of one row of each operand; kPer scales of one row (column) for the
  // first 32 * kWaves threads.
  const unsigned srow = tid / (2 * kWaves), schunk = tid % (2 * kWaves);
  const int8_t *sact = act + min(row0 + srow, p.rows - 1) * k + 16 * (schunk % 2);
  const int8_t *swt = w + min(col0 + srow, p.columns - 1) * k + 16 * (schunk % 2);
  const bool scaler = tid < kTile * kWaves;
  const unsigned sr = tid / kWaves, sg = tid % kWaves;
  const float *sas = as + (size_t)min(row0 + sr, p.rows - 1) * p.groups;
  const uint16_t *sws = ws + (size_t)min(col0 + sr, p.columns - 1) * p.groups;
  v4i ra[kDepth][kPer], rb[kDepth][kPer];
  float rs[kDepth][kPer];
  uint16_t rt[kDepth][kPer];
  auto load = [&](int slot, unsigned step) {
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const unsigned g = min(step * L::kSpan + schunk / 2 + kWaves * j, p.groups - 1); // clamped
      ra[slot][j] = *reinterpret_cast<const v4i *>(sact + (size_t)g * kGroup);
      rb[slot][j] = *reinterpret_cast<const v4i *>(swt + (size_t)g * kGroup);
      if (scaler) {
        const unsigned gs = min(step * L::kSpan + sg + kWaves * j, p.groups - 1);
        rs[slot][j] = sas[gs];
        rt[slot][j] = sws[gs];
      }
    }
  };
  auto stage = [&](int slot, unsigned buf) {
    unsigned char *base = lds + buf * L::kBuffer;
    float *sc = reinterpret_cast<float *>(base + 2 * L::kOperand);
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const unsigned at = srow * L::kPitch + 16 * (schunk + 2 * kWaves * j);
      *reinterpret_cast<v4i *>(base + at) = ra[slot][j];
      *reinterpret_cast<v4i *>(base + L::kOperand + at) = rb[slot][j];
      if (scaler) {
        sc[(sg + kWaves * j) * kTile + sr] = rs[slot][j];
        sc[L::kSpan * kTile + (sg + kWaves * j) * kTile + sr] = h2f(rt[slot][j]);
      }
    }
  };

#pragma unroll
  for (int d = 0; d < kDepth - 1; ++d)
    if ((unsigned)d < nsteps)
      load(d, d);
  stage(0, 0);
  __syncthreads();

  const unsigned m = lane % kTile, h = lane / kTile;
  const v16i zero = {};
  float acc[kClasses][16];
#pragma unroll
  for (int c = 0; c < kClasses; ++c)
#pragma unroll
    for (int r = 0; r < 16; ++r)
      acc[c][r] = 0.0f;
  for (unsigned s0 = 0; s0 < nsteps; s0 += kDepth) {
#pragma unroll
    for (int d = 0; d < kDepth; ++d) {
      const unsigned step = s0 + d;
      if (step >= nsteps)
        break;
      if (step + kDepth - 1 < nsteps)
        load((d + kDepth - 1) % kDepth, step + kDepth - 1);
      // The other buffer was released by the previous step's barrier.
      if (kEarly && step + 1 < nsteps)
        stage((d + 1) % kDepth, (step + 1) % 2);
      const unsigned char *base = lds + (step % 2) * L::kBuffer;
      const float *sc = reinterpret_cast<const float *>(base + 2 * L::kOperand);
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const unsigned gl = wave + kWaves * j; // group within the step
        if (step * L::kSpan + gl < p.groups) {
          const unsigned off = m * L::kPitch + gl * kGroup + 16 * h;
          const v4i a = *reinterpret_cast<const v4i *>(base + off);
          const v4i bw = *reinterpret_cast<const v4i *>(base + L::kOperand + off);
          const float wsv = sc[L::kSpan * kTile + gl * kTile + m];
          const v16i dots = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bw, zero, 0, 0, 0);
          const float4 *sa = reinterpret_cast<const float4 *>(sc + gl * kTile + 4 * h);
          const int c = j % kClasses;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float4 a4 = sa[2 * q];
            acc[c][4 * q + 0] = add_term(acc[c][4 * q + 0], dots[4 * q + 0], a4.x, wsv);
            acc[c][4 * q + 1] = add_term(acc[c][4 * q + 1], dots[4 * q + 1], a4.y, wsv);
            acc[c][4 * q + 2] = add_term(acc[c][4 * q + 2], dots[4 * q + 2], a4.z, wsv);
            acc[c][4 * q + 3] = add_term(acc[c][4 * q + 3], dots[4 * q + 3], a4.w, wsv);
          }
        }
      }
      if (!kEarly && step + 1 < nsteps)
        stage((d + 1) % kDepth, (step + 1) % 2);
      __syncthreads();
    }
  }

  float *sums = reinterpret_cast<float *>(lds) + wave * kTile * kTile;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const unsigned rr = 8 * (r / 4) + 4 * h + r % 4;
    sums[rr * kTile + m] = kClasses == 2 ? __fadd_rn(acc[0][r], acc[kClasses - 1][r]) : acc[0][r];
  }
  __syncthreads();
  for (unsigned e = tid; e < kTile * kTile; e += 64 * kWaves) {
    const unsigned row = row0 + e / kTile, col = col0 + e % kTile;
    if (row >= p.rows || col >= p.columns)
      continue;
    const float *s = reinterpret_cast<const float *>(lds) + e;
    constexpr unsigned T = kTile * kTile;
    float total;
    if (kWaves == 4) // wave w holds c_w + c_(w+4)
      total = __fadd_rn(__fadd_rn(s[0], s[2 * T]), __fadd_rn(s[T], s[3 * T]));
    else
      total = __fadd_rn(__fadd_rn(__fadd_rn(s[0], s[4 * T]), __fadd_rn(s[2 * T], s[6 * T])),
                        __fadd_rn(__fadd_rn(s[T], s[5 * T]), __fadd_rn(s[3 * T], s[7 * T])));
    const unsigned column = p.firstRow + col;
    store_linear(out, aux, bias, (size_t)row * p.outputWidth + column, column, p.epilogue,
                 p.block, total);
  }
}

// ------------------------------------------------- norm + projections, decode

// residualAdd -> rmsNorm -> quantizeActivation of one row and up to four
// W8A8 projections of the quantized row in one launch (the decode step's
// input norms and the projections that read them). The norm's sequential
// sum is one lane's latency-bound chain (~11 us at width 2560) while the
// projections stream their weights: in each 1024-thread workgroup, wave 0
// stages nothing but the norm (every workgroup forms the same bits) and
// runs the chain as soon as the row is in LDS, while waves 1-15 issue their
// weight loads (a wave issues its loads in order, so the chain wave issues
// none: measured, issuing 160 KB of loads a CU takes ~3 us). Waves 1-15
// serve 60 columns of one projection with the GEMV's lanes (16 a column,
// lane l the groups l, l + 16, ...: kLaneGroups of them, 5 up to width 2560,
// 8 up to 4096, one unrolled step) and its arithmetic, so the outputs are
// the separate launches' bits. A paired projection (kPaired, width <= 2560)
// also computes the next one, a SwiGLU projection whose multiplier is this
// one's output, in the same lanes: its weights sit beside the first's and
// the multiplier comes from registers. One workgroup a CU keeps one chain a
// CU (chains sharing a SIMD slow each other down).
constexpr unsigned kNormLinearThreads = 64 + kNormLinearCols * kGemvLanes;
static_assert(kNormLinearThreads == 1024, "the norm wave and 60 columns of 16 lanes");
static_assert(kNormLinearMaxWidth == kGroup * kGemvLanes * 8, "8 groups a lane at most");
static_assert(kNormLinearPairedWidth == kGroup * kGemvLanes * 5, "5 groups a lane paired");

struct NormLinearSeg {
  const int8_t *w;
  const uint16_t *ws;
  void *out;
  const void *aux;
  const float *bias;
  unsigned columns, outputWidth, firstRow, epilogue, block, wgs, paired;
  const uint16_t *cw; // the one-token convolution + SiLU, or null
  uint16_t *ch;
};

// causalConv with applySilu (Reference.metal:137-161) of one token for
// channel c, whose input is the projection's fp32 sum: the input is its
// fp16 rounding, the window the channel's three history values and the
// input, the sum the product of the newest term followed by the fmas of
// the older ones (causal_conv_k4's order), and the history shifts by one.
__device__ __forceinline__ void store_conv_silu(uint16_t *out, const uint16_t *cw, uint16_t *ch,
                                                unsigned c, float acc) {
  const float x = round16(acc);
  const uint16_t h0 = ch[3 * c], h1 = ch[3 * c + 1], h2 = ch[3 * c + 2];
  float y = mul32(x, h2f(cw[4 * c + 3]));
  y = __builtin_fmaf(h2f(h0), h2f(cw[4 * c]), y);
  y = __builtin_fmaf(h2f(h1), h2f(cw[4 * c + 1]), y);
  y = __builtin_fmaf(h2f(h2), h2f(cw[4 * c + 2]), y);
  out[c] = silu16(round16(y));
  ch[3 * c] = h1;
  ch[3 * c + 1] = h2;
  ch[3 * c + 2] = f2h(x);
}

struct NormLinearArgs {
  NormLinearSeg seg[kNormLinearMax];
  unsigned count, width, groups;
  float eps;
  unsigned cols; // columns a workgroup (a multiple of 4, at most 60)
};

// One column's weights for a lane: its kLaneGroups groups (clamped: in
// bounds) and their scales, kept as loaded (fp16 bits): converted where the
// dots use them, so that nothing before then waits for the loads (the norm
// wave issues its own before its chain).
template <int kLaneGroups>
__device__ __forceinline__ void load_lane_weights(const NormLinearSeg &seg, unsigned cc,
                                                  unsigned l, unsigned groups,
                                                  uint4_t (&wv)[kLaneGroups][2],
                                                  uint16_t (&wsv)[kLaneGroups]) {
  const uint4_t *wrow = reinterpret_cast<const uint4_t *>(seg.w + (size_t)cc * groups * kGroup);
  const uint16_t *wsrow = seg.ws + (size_t)cc * groups;
#pragma unroll
  for (int u = 0; u < kLaneGroups; ++u) {
    const unsigned g = min(l + kGemvLanes * u, groups - 1);
    wv[u][0] = __builtin_nontemporal_load(wrow + 2 * g);
    wv[u][1] = __builtin_nontemporal_load(wrow + 2 * g + 1);
    wsv[u] = wsrow[g];
  }
}

// The lane's fp32 sum in group order, then the column's butterfly.
template <int kLaneGroups>
__device__ __forceinline__ float lane_dots(const uint4_t *arow, const float *ss, unsigned l,
                                           unsigned groups, const uint4_t (&wv)[kLaneGroups][2],
                                           const uint16_t (&wsv)[kLaneGroups]) {
  float acc = 0.0f;
#pragma unroll
  for (int u = 0; u < kLaneGroups; ++u) {
    const unsigned g = l + kGemvLanes * u;
    // pinned here (volatile asm keeps its place after the workgroup's
    // barriers): the backend otherwise converts the loaded scale right
    // after its load, which makes the norm wave wait for its weights
    // before its chain
    uint32_t bits = wsv[u];
    asm volatile("" : "+v"(bits));
    if (g < groups)
      acc = add_term(acc, group_dot(arow[2 * g], arow[2 * g + 1], wv[u][0], wv[u][1]), ss[g],
                     h2f((uint16_t)bits));
  }
#pragma unroll
  for (int m = kGemvLanes / 2; m >= 1; m /= 2)
    acc = __fadd_rn(acc, __shfl_xor(acc, m, kGemvLanes));
  return acc;
}

template <bool kAdd, int kLaneGroups, bool kPaired>
__global__ __launch_bounds__(kNormLinearThreads) void norm_linear_kernel(
    const uint16_t *__restrict__ a, const uint16_t *__restrict__ b, uint16_t *sum_out,
    const float *__restrict__ nw, int8_t *q, float *scales, unsigned *invalid,
    NormLinearArgs p) {
  extern __shared__ __align__(16) float srow[]; // row, 1 + w, quantized words, scales
  __shared__ float sscale;
  const unsigned t = threadIdx.x, padded = p.groups * kGroup;
  float *sw = srow + padded;
  uint32_t *sq = reinterpret_cast<uint32_t *>(sw + padded);
  float *ss = reinterpret_cast<float *>(sq + p.groups * (kGroup / 4));
  unsigned blk = blockIdx.x, s = 0;
  bool found = false;
#pragma unroll
  for (unsigned k = 0; k < kNormLinearMax; ++k)
    if (!found && k < p.count) {
      if (blk < p.seg[k].wgs) {
        s = k;
        found = true;
      } else {
        blk -= p.seg[k].wgs;
      }
    }
  // selected with constant indices (no private copy of the table)
  NormLinearSeg seg = p.seg[0], mate = p.seg[0];
#pragma unroll
  for (unsigned k = 1; k < kNormLinearMax; ++k) {
    if (k == s)
      seg = p.seg[k];
    if (kPaired && k == s + 1)
      mate = p.seg[k];
  }
  const bool paired = kPaired && seg.paired;
  const bool norm_wave = t < 64;
  // waves 1-15 serve four columns each, as many as the launch gives a
  // workgroup; the others only help stage and quantize the row
  const unsigned lane_col = (t - 64) / kGemvLanes; // (wraps for the norm wave)
  const unsigned col = blk * p.cols + lane_col;
  const unsigned l = t % kGemvLanes;
  const bool serves = !norm_wave && lane_col < p.cols; // a wave with columns
  const bool live = serves && col < seg.columns;
  const unsigned cc = live ? col : 0; // clamped: in bounds

  // The row, then (waves 1-15) the weights or (wave 0) the chain. The
  // barriers order LDS only: a __syncthreads would wait for the weight
  // stream.
  const bool first = blockIdx.x == 0; // writes the sum, q, scales and the flag
  stage_norm_row<kAdd, kNormLinearThreads>(a, b, first ? sum_out : nullptr, nw, srow, sw,
                                           p.width, padded, t);
  lds_sync();
  uint4_t wv[kLaneGroups][2], mv[kPaired ? kLaneGroups : 1][2];
  uint16_t wsv[kLaneGroups], msv[kPaired ? kLaneGroups : 1];
  if (serves) {
    load_lane_weights<kLaneGroups>(seg, cc, l, p.groups, wv, wsv);
    if constexpr (kPaired)
      if (paired)
        load_lane_weights<kLaneGroups>(mate, cc, l, p.groups, mv, msv);
  }
  if (norm_wave && t == 0)
    sscale = rms_scale_of(norm_row_sum(srow, padded), p.width, p.eps);
  lds_sync();
  quantize_norm_row<kNormLinearThreads>(srow, sw, sscale, p.width, p.groups, t, sq, ss,
                                        first ? invalid : nullptr);
  lds_sync();
  if (first && q)
    for (unsigned i = t; i < p.groups * (kGroup / 4); i += kNormLinearThreads)
      reinterpret_cast<uint32_t *>(q)[i] = sq[i];
  if (first && scales)
    for (unsigned i = t; i < p.groups; i += kNormLinearThreads)
      scales[i] = ss[i];

  if (!serves)
    return;
  const uint4_t *arow = reinterpret_cast<const uint4_t *>(sq);
  const float acc = lane_dots<kLaneGroups>(arow, ss, l, p.groups, wv, wsv);
  if constexpr (kPaired) {
    if (paired) {
      const float macc = lane_dots<kLaneGroups>(arow, ss, l, p.groups, mv, msv);
      if (l == 0 && live) {
        // the first projection has no epilogue: its fp16 output is the
        // SwiGLU multiplier
        const float projected = round16(acc);
        static_cast<uint16_t *>(seg.out)[seg.firstRow + col] = f2h(projected);
        static_cast<uint16_t *>(mate.out)[mate.firstRow + col] =
            silu_mul16(round16(macc), f2h(projected));
      }
      return;
    }
  }
  if (l == 0 && live) {
    const unsigned column = seg.firstRow + col;
    if (seg.cw)
      store_conv_silu(static_cast<uint16_t *>(seg.out), seg.cw, seg.ch, column, acc);
    else
      store_linear(seg.out, seg.aux, seg.bias, column, column, seg.epilogue, seg.block, acc);
  }
}

// ------------------------------------------------------------- embeddings

// embeddingW8 (Graph.metal:16-31): eight outputs per lane (they share a
// 32-wide scale group when hidden is a multiple of 8), or one.
__global__ __launch_bounds__(256) void embedding_w8_kernel(
    const uint32_t *__restrict__ ids, const int8_t *__restrict__ w,
    const uint16_t *__restrict__ sc, uint16_t *__restrict__ out, unsigned tokens,
    unsigned hidden, unsigned first, unsigned count, unsigned groups, unsigned per) {
  const size_t i0 = ((size_t)blockIdx.x * 256 + threadIdx.x) * per;
  if (i0 >= (size_t)tokens * hidden)
    return;
  const uint32_t id = ids[i0 / hidden];
  if (id < first || id - first >= count)
    return;
  const size_t row = id - first;
  const unsigned c0 = (unsigned)(i0 % hidden);
  if (per == 8) {
    const uint2 q = *reinterpret_cast<const uint2 *>(w + row * groups * kGroup + c0);
    const float s = h2f(sc[row * groups + c0 / kGroup]);
    uint4_t o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t word = e < 2 ? q.x : q.y;
      const int8_t lo = (int8_t)(word >> (16 * (e % 2))), hi = (int8_t)(word >> (16 * (e % 2) + 8));
      o[e] = (uint32_t)f2h(mul32((float)lo, s)) | ((uint32_t)f2h(mul32((float)hi, s)) << 16);
    }
    *reinterpret_cast<uint4_t *>(out + i0) = o;
  } else {
    out[i0] = f2h(mul32((float)w[row * groups * kGroup + c0], h2f(sc[row * groups + c0 / kGroup])));
  }
}

// embedding (Reference.metal:49-58).
__global__ __launch_bounds__(256) void embedding_kernel(const uint32_t *__restrict__ ids,
                                                        const uint16_t *__restrict__ w,
                                                        uint16_t *__restrict__ out,
                                                        unsigned tokens, unsigned hidden,
                                                        unsigned first, unsigned count,
                                                        unsigned per) {
  const size_t i0 = ((size_t)blockIdx.x * 256 + threadIdx.x) * per;
  if (i0 >= (size_t)tokens * hidden)
    return;
  const uint32_t id = ids[i0 / hidden];
  if (id < first || id - first >= count)
    return;
  const size_t src = (size_t)(id - first) * hidden + i0 % hidden;
  if (per == 8)
    *reinterpret_cast<uint4_t *>(out + i0) = *reinterpret_cast<const uint4_t *>(w + src);
  else
    out[i0] = w[src];
}

} // namespace

hipError_t launch_quantize_activation(const uint16_t *in, int8_t *q, float *scales,
                                      unsigned *invalid, unsigned rows, unsigned width,
                                      unsigned groups, hipStream_t stream) {
  const unsigned n = rows * groups;
  const bool vec = width % kGroup == 0 && aligned16(in);
  if (vec) {
    const unsigned chunks = n * (kGroup / 8);
    hipLaunchKernelGGL(quantize_chunks_kernel, dim3((chunks + 255) / 256), dim3(256), 0, stream,
                       in, q, scales, invalid, chunks);
  } else {
    hipLaunchKernelGGL(quantize_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, in, q,
                       scales, invalid, rows, width, groups, vec);
  }
  return hipGetLastError();
}

hipError_t launch_add_norm_quantize(const uint16_t *a, const uint16_t *b, uint16_t *sum_out,
                                   const float *w, int8_t *q, float *scales, unsigned *invalid,
                                   unsigned rows, unsigned width, float eps, hipStream_t stream) {
  const unsigned groups = (width + kGroup - 1) / kGroup;
  const size_t lds = 2 * (size_t)groups * kGroup * sizeof(float);
  if (b)
    hipLaunchKernelGGL(add_norm_quantize_kernel<true>, dim3(rows), dim3(256), lds, stream, a, b,
                       sum_out, w, q, scales, invalid, width, groups, eps);
  else
    hipLaunchKernelGGL(add_norm_quantize_kernel<false>, dim3(rows), dim3(256), lds, stream, a,
                       b, sum_out, w, q, scales, invalid, width, groups, eps);
  return hipGetLastError();
}

// Compute units of the current device (256 on MI355X), read once a device.
static unsigned device_cus() {
  static int cus[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
    return 256;
  if (cus[dev] <= 0) {
    int c = 0;
    cus[dev] = hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) ==
                           hipSuccess && c > 0
                   ? c
                   : 256;
  }
  return (unsigned)cus[dev];
}

template <bool kAdd, int kLaneGroups, bool kPaired>
static void launch_norm_linear_as(const uint16_t *a, const uint16_t *b, uint16_t *sum_out,
                                  const float *w, int8_t *q, float *scales, unsigned *invalid,
                                  const NormLinearArgs &p, unsigned wgs, size_t lds,
                                  hipStream_t stream) {
  hipLaunchKernelGGL((norm_linear_kernel<kAdd, kLaneGroups, kPaired>), dim3(wgs),
                     dim3(kNormLinearThreads), lds, stream, a, b, sum_out, w, q, scales, invalid,
                     p);
}

hipError_t launch_add_norm_linear(const uint16_t *a, const uint16_t *b, uint16_t *sum_out,
                                  const float *w, int8_t *q, float *scales, unsigned *invalid,
                                  unsigned width, float eps, const NormLinearProj *proj,
                                  unsigned count, hipStream_t stream) {
  NormLinearArgs p{};
  p.count = count;
  p.width = width;
  p.groups = (width + kGroup - 1) / kGroup;
  p.eps = eps;
  unsigned wgs = 0;
  bool paired = false;
  // The fewest columns a workgroup (a multiple of 4) that still fit the
  // launch in one workgroup a CU: each workgroup's weight stream is then
  // the shortest, with every CU streaming (at 60 columns the MLP's 9216
  // fill 154 CUs, whose streams outlast the norm's chain).
  unsigned perWg = kNormLinearCols;
  const unsigned cus = device_cus();
  for (unsigned c = 4; c < kNormLinearCols; c += 4) {
    unsigned n = 0;
    for (unsigned k = 0; k < count; ++k)
      if (!(k > 0 && proj[k - 1].paired))
        n += (proj[k].shape.columns + c - 1) / c;
    if (n <= cus) {
      perWg = c;
      break;
    }
  }
  p.cols = perWg;
  for (unsigned k = 0; k < count; ++k) {
    const NormLinearProj &x = proj[k];
    const bool mate = k > 0 && proj[k - 1].paired;
    p.seg[k] = {x.w, x.ws, x.out, x.aux, x.bias, x.shape.columns, x.shape.outputWidth,
                x.shape.firstRow, x.shape.epilogue, x.shape.block,
                mate ? 0u : (x.shape.columns + perWg - 1) / perWg, x.paired ? 1u : 0u,
                x.cw, x.ch};
    wgs += p.seg[k].wgs;
    paired = paired || x.paired;
  }
  const size_t lds = 2 * (size_t)p.groups * kGroup * sizeof(float) + (size_t)p.groups * kGroup +
                     (size_t)p.groups * sizeof(float);
  const bool five = width <= kNormLinearPairedWidth;
  if (b) {
    if (paired)
      launch_norm_linear_as<true, 5, true>(a, b, sum_out, w, q, scales, invalid, p, wgs, lds,
                                           stream);
    else if (five)
      launch_norm_linear_as<true, 5, false>(a, b, sum_out, w, q, scales, invalid, p, wgs, lds,
                                            stream);
    else
      launch_norm_linear_as<true, 8, false>(a, b, sum_out, w, q, scales, invalid, p, wgs, lds,
                                            stream);
  } else {
    if (paired)
      launch_norm_linear_as<false, 5, true>(a, b, sum_out, w, q, scales, invalid, p, wgs, lds,
                                            stream);
    else if (five)
      launch_norm_linear_as<false, 5, false>(a, b, sum_out, w, q, scales, invalid, p, wgs, lds,
                                             stream);
    else
      launch_norm_linear_as<false, 8, false>(a, b, sum_out, w, q, scales, invalid, p, wgs, lds,
                                             stream);
  }
  return hipGetLastError();
}

const char *linear_w8a8_kernel(unsigned rows) {
  return rows == 1 ? "linearW8A8Gemv" : "linearW8A8Gemm";
}

// The split GEMV for kPer steps a wave (2 .. kSplitPer).
template <int kPer>
static void launch_gemv_split_as(dim3 grid, hipStream_t stream, const int8_t *act, const float *as,
                                 const int8_t *w, const uint16_t *ws, void *out, const void *aux,
                                 const float *bias, const W8Args &a) {
  hipLaunchKernelGGL(gemv_split_kernel<kPer>, grid, dim3(64 * kSplitWaves), 0, stream, act, as, w,
                     ws, out, aux, bias, a);
}

template <int kPer = kSplitPer>
static void launch_gemv_split(unsigned per, dim3 grid, hipStream_t stream, const int8_t *act,
                              const float *as, const int8_t *w, const uint16_t *ws, void *out,
                              const void *aux, const float *bias, const W8Args &a) {
  if constexpr (kPer > 2)
    if (per < (unsigned)kPer)
      return launch_gemv_split<kPer - 1>(per, grid, stream, act, as, w, ws, out, aux, bias, a);
  launch_gemv_split_as<kPer>(grid, stream, act, as, w, ws, out, aux, bias, a);
}

hipError_t launch_linear_w8a8(const int8_t *act, const float *as, const int8_t *w,
                              const uint16_t *ws, void *out, const void *aux, const float *bias,
                              const W8Shape &s, hipStream_t stream) {
  const W8Args a{s.outputWidth, s.firstRow, s.groups, s.rows, s.columns, s.epilogue, s.block};
  const unsigned steps = (s.groups + kGemvLanes - 1) / kGemvLanes;
  if (s.rows == 1 && steps >= kGemvUnroll && steps <= kSplitMaxSteps)
    launch_gemv_split((steps + kSplitWaves - 1) / kSplitWaves,
                      dim3((s.columns + kGemvCols - 1) / kGemvCols), stream, act, as, w, ws, out,
                      aux, bias, a);
  else if (s.rows == 1)
    hipLaunchKernelGGL(gemv_kernel, dim3((s.columns + kGemvCols - 1) / kGemvCols),
                       dim3(kGemvThreads), 0, stream, act, as, w, ws, out, aux, bias, a);
  else if (s.rows >= kMfmaMinRows) {
    const unsigned rowTiles = (s.rows + kTile - 1) / kTile;
    const unsigned tiles = rowTiles * ((s.columns + kTile - 1) / kTile);
    if (tiles >= kMfmaManyTiles)
      hipLaunchKernelGGL((gemm_mfma_kernel<8, 1, 2, true>), dim3(tiles), dim3(512), 0, stream,
                         act, as, w, ws, out, aux, bias, a, rowTiles);
    else
      hipLaunchKernelGGL((gemm_mfma_kernel<8, 1, 4, false>), dim3(tiles), dim3(512), 0, stream,
                         act, as, w, ws, out, aux, bias, a, rowTiles);
  } else
    hipLaunchKernelGGL(gemm_kernel,
                       dim3((s.columns + kGemmCols - 1) / kGemmCols,
                            (s.rows + kGemmRows - 1) / kGemmRows),
                       dim3(256), 0, stream, act, as, w, ws, out, aux, bias, a);
  return hipGetLastError();
}

hipError_t launch_embedding_w8(const uint32_t *ids, const int8_t *w, const uint16_t *sc,
                               uint16_t *out, unsigned tokens, unsigned hidden, unsigned first,
                               unsigned count, unsigned groups, hipStream_t stream) {
  const unsigned per = hidden % 8 == 0 && aligned16(out) && aligned16(w) ? 8u : 1u;
  const size_t n = ((size_t)tokens * hidden + per - 1) / per;
  hipLaunchKernelGGL(embedding_w8_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                     ids, w, sc, out, tokens, hidden, first, count, groups, per);
  return hipGetLastError();
}

hipError_t launch_embedding(const uint32_t *ids, const uint16_t *w, uint16_t *out,
                            unsigned tokens, unsigned hidden, unsigned first, unsigned count,
                            hipStream_t stream) {
  const unsigned per = hidden % 8 == 0 && aligned16(out) && aligned16(w) ? 8u : 1u;
  const size_t n = ((size_t)tokens * hidden + per - 1) / per;
  hipLaunchKernelGGL(embedding_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                     ids, w, out, tokens, hidden, first, count, per);
  return hipGetLastError();
}

} // namespace llmi
