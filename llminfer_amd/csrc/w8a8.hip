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
//  * GEMM (several rows): the reference's 8 lanes per column and 4 rows per
//    lane; a weight group is loaded once for its four rows.
#include "exact_fp.hpp"
#include "hip_common.hpp"
#include "kernels.hpp"
#include "rope_gate.hpp"

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

// storeLinear (Reference.metal:14-47): the projection rounded to fp16, then
// the consumer's fused epilogue.
__device__ __forceinline__ void store_linear(void *out, const void *aux, const float *bias,
                                             size_t i, unsigned col, unsigned epilogue,
                                             unsigned block, float acc) {
  const float projected = round16(acc);
  uint16_t *o16 = static_cast<uint16_t *>(out);
  float *o32 = static_cast<float *>(out);
  switch (epilogue) {
  case LLMI_LINEAR_SILU:
    o16[i] = silu16(projected);
    return;
  case LLMI_LINEAR_SILU_MUL:
    o16[i] = f2h(mul32(h2f(silu16(projected)), h2f(static_cast<const uint16_t *>(aux)[i])));
    return;
  case LLMI_LINEAR_SIGMOID_COLUMNS:
    o16[i] = f2h((col / block) % 2 ? logistic16(projected) : projected);
    return;
  case LLMI_LINEAR_SILU_F32:
    o32[i] = mul32(projected, logistic_exact(projected));
    return;
  case LLMI_LINEAR_DELTA_BETA:
    o32[i] = logistic16(projected);
    return;
  case LLMI_LINEAR_DELTA_DECAY: {
    const float *a_log = static_cast<const float *>(aux);
    o32[i] = exp_cr(mul32(-exp_cr(a_log[col]), stable_softplus(__fadd_rn(projected, bias[col]))));
    return;
  }
  default:
    o16[i] = f2h(projected);
    return;
  }
}

// --------------------------------------------------------------- quantize

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
  float max_abs = 0.0f;
  bool finite = true;
#pragma unroll
  for (unsigned j = 0; j < kGroup; ++j) {
    finite = finite && __builtin_isfinite(x[j]);
    max_abs = fmaxf(max_abs, fabsf(x[j]));
  }
  if (!finite && invalid)
    atomicOr(invalid, 1u);
  const float scale = finite && max_abs > 0.0f ? __fdiv_rn(max_abs, 127.0f) : 1.0f;
  scales[i] = scale;
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
  uint4_t *dst = reinterpret_cast<uint4_t *>(q + (size_t)i * kGroup);
  dst[0] = packed[0];
  dst[1] = packed[1];
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

// Long rows (more than 128 groups: 8 per lane or more): four waves share the
// same 4 columns. Wave w computes the group terms (float(dot) * a) * w of the
// w-th quarter of every lane's groups, all its loads issued at once, into
// LDS; wave 0 then adds each lane's terms in group order -- the same fp32
// sums as one lane would form -- and finishes as above.
constexpr int kSplitWaves = 4, kSplitMaxSteps = 64; // groups per lane <= 64
constexpr int kSplitPer = kSplitMaxSteps / kSplitWaves;

__global__ __launch_bounds__(64 * kSplitWaves) void gemv_split_kernel(
    const int8_t *__restrict__ act, const float *__restrict__ as, const int8_t *__restrict__ w,
    const uint16_t *__restrict__ ws, void *out, const void *aux, const float *bias, W8Args p) {
  __shared__ float sT[kSplitMaxSteps][64];
  const unsigned wave = threadIdx.x / 64, t = threadIdx.x % 64;
  const unsigned col = blockIdx.x * kGemvCols + t / kGemvLanes;
  const unsigned l = t % kGemvLanes;
  const unsigned steps = (p.groups + kGemvLanes - 1) / kGemvLanes; // a lane's steps, at most
  const unsigned per = (steps + kSplitWaves - 1) / kSplitWaves, i0 = wave * per;
  if (col < p.columns) {
    const uint4_t *wrow = reinterpret_cast<const uint4_t *>(w + (size_t)col * p.groups * kGroup);
    const uint4_t *arow = reinterpret_cast<const uint4_t *>(act);
    const uint16_t *wsrow = ws + (size_t)col * p.groups;
    uint4_t wv[kSplitPer][2];
    float wsv[kSplitPer];
#pragma unroll
    for (int u = 0; u < kSplitPer; ++u) {
      const unsigned g = min(l + kGemvLanes * (i0 + u), p.groups - 1); // clamped: in bounds
      if ((unsigned)u < per) {
        wv[u][0] = __builtin_nontemporal_load(wrow + 2 * g);
        wv[u][1] = __builtin_nontemporal_load(wrow + 2 * g + 1);
        wsv[u] = h2f(wsrow[g]);
      }
    }
#pragma unroll
    for (int u = 0; u < kSplitPer; ++u) {
      const unsigned g = l + kGemvLanes * (i0 + u);
      if ((unsigned)u < per && g < p.groups)
        sT[i0 + u][t] = __fmul_rn(
            __fmul_rn((float)group_dot(arow[2 * g], arow[2 * g + 1], wv[u][0], wv[u][1]), as[g]),
            wsv[u]);
    }
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

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

} // namespace

hipError_t launch_quantize_activation(const uint16_t *in, int8_t *q, float *scales,
                                      unsigned *invalid, unsigned rows, unsigned width,
                                      unsigned groups, hipStream_t stream) {
  const unsigned n = rows * groups;
  const bool vec = width % kGroup == 0 && aligned16(in);
  hipLaunchKernelGGL(quantize_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, in, q,
                     scales, invalid, rows, width, groups, vec);
  return hipGetLastError();
}

const char *linear_w8a8_kernel(unsigned rows) {
  return rows == 1 ? "linearW8A8Gemv" : "linearW8A8Gemm";
}

hipError_t launch_linear_w8a8(const int8_t *act, const float *as, const int8_t *w,
                              const uint16_t *ws, void *out, const void *aux, const float *bias,
                              const W8Shape &s, hipStream_t stream) {
  const W8Args a{s.outputWidth, s.firstRow, s.groups, s.rows, s.columns, s.epilogue, s.block};
  const unsigned steps = (s.groups + kGemvLanes - 1) / kGemvLanes;
  if (s.rows == 1 && steps > kGemvUnroll && steps <= kSplitMaxSteps)
    hipLaunchKernelGGL(gemv_split_kernel, dim3((s.columns + kGemvCols - 1) / kGemvCols),
                       dim3(64 * kSplitWaves), 0, stream, act, as, w, ws, out, aux, bias, a);
  else if (s.rows == 1)
    hipLaunchKernelGGL(gemv_kernel, dim3((s.columns + kGemvCols - 1) / kGemvCols),
                       dim3(kGemvThreads), 0, stream, act, as, w, ws, out, aux, bias, a);
  else
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
