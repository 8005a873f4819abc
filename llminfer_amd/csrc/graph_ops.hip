// The remaining ops of the whole-graph plan: residualAdd, swiGlu, siluF16
// and multiplyF16 (Reference.metal:119-136, Graph.metal:70-95), copyHalfView
// (Graph.metal:1-14) and linearF16 (Reference.metal:61-103).
//
//  * The elementwise ops are HBM-bound: 8 halves (16 bytes) per lane when
//    the count is a multiple of 8 and the buffers are 16-byte aligned, else
//    one. Each result is the reference's fp32 expression rounded to fp16:
//    the sum and product of two fp16 values are exact or singly rounded in
//    fp32 (24 >= 2 x 11 + 2 bits), so any instruction form gives the same
//    bits; SiLU goes through the same correctly rounded helper as the
//    projections' epilogue.
//  * linearF16 keeps the reference's arithmetic: each output is one fp32
//    fma chain over k = 0 .. K-1 in order, then storeLinear. A workgroup of
//    256 lanes serves 256 output columns and up to 8 rows; 64-wide k chunks
//    of the 256 weight rows are staged in LDS (rows padded by 16 bytes, so
//    lane c's 16-byte reads of its own row meet no bank conflicts) and a
//    lane runs its rows' chains side by side.
#include "exact_fp.hpp"
#include "hip_common.hpp"
#include "kernels.hpp"
#include "linear_store.hpp"

#include "llminfer_hip.h"

namespace llmi {
namespace {

__device__ __forceinline__ uint16_t elementwise(ElementwiseKind kind, uint16_t a, uint16_t b) {
  switch (kind) {
  case ElementwiseKind::Add:
    return f2h(__fadd_rn(h2f(a), h2f(b)));
  case ElementwiseKind::SwiGlu:
    return f2h(mul32(h2f(silu16(h2f(a))), h2f(b)));
  case ElementwiseKind::Silu:
    return silu16(h2f(a));
  case ElementwiseKind::Multiply:
    return f2h(mul32(h2f(a), h2f(b)));
  }
  return 0;
}

template <ElementwiseKind K>
__global__ __launch_bounds__(256) void elementwise_kernel(const uint16_t *__restrict__ a,
                                                          const uint16_t *__restrict__ b,
                                                          uint16_t *__restrict__ out,
                                                          unsigned count, bool vec) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (vec) {
    if (i * 8 >= count)
      return;
    const uint4_t va = reinterpret_cast<const uint4_t *>(a)[i];
    const uint4_t vb = K == ElementwiseKind::Silu ? va : reinterpret_cast<const uint4_t *>(b)[i];
    uint4_t r;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint16_t lo = elementwise(K, (uint16_t)(va[e] & 0xFFFFu), (uint16_t)(vb[e] & 0xFFFFu));
      const uint16_t hi = elementwise(K, (uint16_t)(va[e] >> 16), (uint16_t)(vb[e] >> 16));
      r[e] = (uint32_t)lo | ((uint32_t)hi << 16);
    }
    reinterpret_cast<uint4_t *>(out)[i] = r;
  } else if (i < count) {
    out[i] = elementwise(K, a[i], K == ElementwiseKind::Silu ? a[i] : b[i]);
  }
}

__global__ __launch_bounds__(256) void copy_view_kernel(const uint16_t *__restrict__ src,
                                                        uint16_t *__restrict__ out,
                                                        HalfViewParams p) {
  const unsigned i = blockIdx.x * 256 + threadIdx.x;
  if (i >= p.count)
    return;
  unsigned rest = i, offset = p.offset;
#pragma unroll
  for (int d = 2; d >= 0; --d) {
    offset += (rest % p.dims[d]) * p.strides[d];
    rest /= p.dims[d];
  }
  out[i] = src[offset];
}

constexpr unsigned kF16Cols = 256, kF16Rows = 8, kF16Chunk = 64;
constexpr unsigned kF16Pitch = kF16Chunk + 8; // halves per staged weight row

__global__ __launch_bounds__(kF16Cols) void linear_f16_kernel(
    const uint16_t *__restrict__ in, const uint16_t *__restrict__ w, void *out, const void *aux,
    const float *bias, LinearParams p) {
  __shared__ __align__(16) uint16_t sW[kF16Cols * kF16Pitch];
  __shared__ __align__(16) float sIn[kF16Rows][kF16Chunk];
  const unsigned t = threadIdx.x;
  const unsigned col0 = blockIdx.x * kF16Cols, row0 = blockIdx.y * kF16Rows;
  const unsigned nr = min(kF16Rows, p.tokens - row0);
  float acc[kF16Rows];
#pragma unroll
  for (unsigned r = 0; r < kF16Rows; ++r)
    acc[r] = 0.0f;
  for (unsigned base = 0; base < p.inputWidth; base += kF16Chunk) {
    __syncthreads(); // the previous chunk is consumed
    // Weight rows col0 .. col0+255, halves base .. base+63 (zero past the
    // ends): 8 threads per row, 8 halves each, 8 passes.
    for (unsigned e = t; e < kF16Cols * (kF16Chunk / 8); e += kF16Cols) {
      const unsigned c = e / (kF16Chunk / 8), k8 = (e % (kF16Chunk / 8)) * 8;
      const unsigned col = col0 + c;
      uint16_t v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const unsigned k = base + k8 + j;
        v[j] = col < p.rowCount && k < p.inputWidth ? w[(size_t)col * p.inputWidth + k] : 0;
      }
      uint4_t packed;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        packed[j] = (uint32_t)v[2 * j] | ((uint32_t)v[2 * j + 1] << 16);
      *reinterpret_cast<uint4_t *>(&sW[c * kF16Pitch + k8]) = packed;
    }
    for (unsigned e = t; e < kF16Rows * kF16Chunk; e += kF16Cols) {
      const unsigned r = e / kF16Chunk, k = base + e % kF16Chunk;
      sIn[r][e % kF16Chunk] =
          r < nr && k < p.inputWidth ? h2f(in[(size_t)(row0 + r) * p.inputWidth + k]) : 0.0f;
    }
    __syncthreads();
#pragma unroll 2
    for (unsigned k8 = 0; k8 < kF16Chunk; k8 += 8) {
      const uint4_t wv = *reinterpret_cast<const uint4_t *>(&sW[t * kF16Pitch + k8]);
      float wf[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        wf[2 * j] = h2f((uint16_t)(wv[j] & 0xFFFFu));
        wf[2 * j + 1] = h2f((uint16_t)(wv[j] >> 16));
      }
#pragma unroll
      for (unsigned r = 0; r < kF16Rows; ++r)
#pragma unroll
        for (int j = 0; j < 8; ++j)
          acc[r] = __builtin_fmaf(sIn[r][k8 + j], wf[j], acc[r]);
    }
  }
  const unsigned col = col0 + t;
  if (col >= p.rowCount)
    return;
  const unsigned column = p.firstRow + col;
  for (unsigned r = 0; r < nr; ++r)
    store_linear(out, aux, bias, (size_t)(row0 + r) * p.outputWidth + column, column, p.epilogue,
                 p.epilogueBlock, acc[r]);
}

} // namespace

hipError_t launch_elementwise(ElementwiseKind kind, const uint16_t *a, const uint16_t *b,
                              uint16_t *out, unsigned count, hipStream_t stream) {
  const bool vec = count % 8 == 0 && aligned16(a) && aligned16(out) &&
                   (kind == ElementwiseKind::Silu || aligned16(b));
  const size_t lanes = vec ? count / 8 : count;
  const dim3 grid((unsigned)((lanes + 255) / 256));
  switch (kind) {
  case ElementwiseKind::Add:
    hipLaunchKernelGGL(elementwise_kernel<ElementwiseKind::Add>, grid, dim3(256), 0, stream, a,
                       b, out, count, vec);
    break;
  case ElementwiseKind::SwiGlu:
    hipLaunchKernelGGL(elementwise_kernel<ElementwiseKind::SwiGlu>, grid, dim3(256), 0, stream,
                       a, b, out, count, vec);
    break;
  case ElementwiseKind::Silu:
    hipLaunchKernelGGL(elementwise_kernel<ElementwiseKind::Silu>, grid, dim3(256), 0, stream, a,
                       b, out, count, vec);
    break;
  case ElementwiseKind::Multiply:
    hipLaunchKernelGGL(elementwise_kernel<ElementwiseKind::Multiply>, grid, dim3(256), 0,
                       stream, a, b, out, count, vec);
    break;
  }
  return hipGetLastError();
}

hipError_t launch_copy_half_view(const uint16_t *src, uint16_t *out, const HalfViewParams &p,
                                 hipStream_t stream) {
  hipLaunchKernelGGL(copy_view_kernel, dim3((p.count + 255) / 256), dim3(256), 0, stream, src,
                     out, p);
  return hipGetLastError();
}

hipError_t launch_linear_f16(const uint16_t *in, const uint16_t *w, void *out, const void *aux,
                             const float *bias, const LinearParams &p, hipStream_t stream) {
  const dim3 grid((p.rowCount + kF16Cols - 1) / kF16Cols, (p.tokens + kF16Rows - 1) / kF16Rows);
  hipLaunchKernelGGL(linear_f16_kernel, grid, dim3(kF16Cols), 0, stream, in, w, out, aux, bias,
                     p);
  return hipGetLastError();
}

} // namespace llmi
