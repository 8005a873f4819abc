// Gated delta rule, token-recurrent form: the DeltaNet decode step.
//
// Same arithmetic as graphDeltaUpdate / updateDeltaColumn
// (Graph.metal:146-170, Reference.metal:182-197), which gives one thread a
// whole state column in device memory and walks it twice per token. Here
// the state lives in registers for the whole call:
//
//  * one wave serves 8 state columns of one value head; 8 lanes share a
//    column and each holds 16 of its dk = 128 rows (dk = 64: 8 rows);
//  * per token the two column dot products (k.S for the prediction and q.S
//    for the output) are partial sums over a lane's rows, finished with
//    3 DPP row permutes over the 8 lanes of the column;
//  * the state is read from HBM once at the start and written once at the
//    end, so a decode step moves exactly the 2 x Hv*dk*dv*4 state bytes plus
//    the step's q/k/v/gates.
//
// Summation order inside a dot product differs from the reference's single
// fma chain (four interleaved chains per lane plus the lane tree); the
// result stays within fp32 rounding of the sequential order.
#include "hip_common.hpp"
#include "kernels.hpp"

namespace llmi {
namespace {

constexpr int kLanesPerCol = 8;
constexpr int kColsPerWave = 64 / kLanesPerCol;

template <int DK>
__global__ __launch_bounds__(64) void delta_recurrent_kernel(
    const float *__restrict__ q, const float *__restrict__ k,
    const half_t *__restrict__ v, const float *__restrict__ beta,
    const float *__restrict__ decay, float *__restrict__ state,
    half_t *__restrict__ out, unsigned T, unsigned Hk, unsigned Hv,
    unsigned DV) {
  constexpr int RPL = DK / kLanesPerCol; // rows per lane
  static_assert(RPL % 4 == 0, "rows per lane must be a multiple of 4");
  const unsigned lane = threadIdx.x;
  const unsigned cw = lane / kLanesPerCol, rg = lane % kLanesPerCol;
  const unsigned colsPerHead = DV / kColsPerWave;
  const unsigned h = blockIdx.x / colsPerHead;
  const unsigned col = (blockIdx.x % colsPerHead) * kColsPerWave + cw;
  const unsigned kh = h / (Hv / Hk);
  const unsigned row0 = rg * RPL;
  const size_t vwidth = (size_t)Hv * DV;

  float S[RPL];
  float *sbase = state + ((size_t)h * DK + row0) * DV + col;
#pragma unroll
  for (int m = 0; m < RPL; ++m)
    S[m] = sbase[(size_t)m * DV];

  for (unsigned t = 0; t < T; ++t) {
    const float *kt = k + ((size_t)t * Hk + kh) * DK + row0;
    const float *qt = q + ((size_t)t * Hk + kh) * DK + row0;
    float kr[RPL], qr[RPL];
#pragma unroll
    for (int m = 0; m < RPL; m += 4) {
      float4_t kv4 = *reinterpret_cast<const float4_t *>(kt + m);
      float4_t qv4 = *reinterpret_cast<const float4_t *>(qt + m);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        kr[m + e] = kv4[e];
        qr[m + e] = qv4[e];
      }
    }
    const float a = decay[(size_t)t * Hv + h];
    const float b = beta[(size_t)t * Hv + h];
    const float vj = (float)v[(size_t)t * vwidth + (size_t)h * DV + col];

    float p4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int m = 0; m < RPL; ++m)
      p4[m % 4] = fmaf(S[m] * a, kr[m], p4[m % 4]);
    float pred = group_sum<kLanesPerCol>((p4[0] + p4[1]) + (p4[2] + p4[3]));
    const float delta = (vj - pred) * b;

    float y4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int m = 0; m < RPL; ++m) {
      S[m] = fmaf(kr[m], delta, S[m] * a);
      y4[m % 4] = fmaf(S[m], qr[m], y4[m % 4]);
    }
    float y = group_sum<kLanesPerCol>((y4[0] + y4[1]) + (y4[2] + y4[3]));
    if (rg == 0)
      out[(size_t)t * vwidth + (size_t)h * DV + col] = (half_t)y;
  }

#pragma unroll
  for (int m = 0; m < RPL; ++m)
    sbase[(size_t)m * DV] = S[m];
}

// Any-shape fallback (e.g. the reference test models' dk = 7, dv = 5):
// one thread per state column, the column kept in device memory, exactly
// the loop structure of updateDeltaColumn. Correctness path only.
__global__ __launch_bounds__(64) void delta_generic_kernel(
    const float *__restrict__ q, const float *__restrict__ k,
    const half_t *__restrict__ v, const float *__restrict__ beta,
    const float *__restrict__ decay, float *__restrict__ state,
    half_t *__restrict__ out, unsigned T, unsigned Hk, unsigned DK,
    unsigned Hv, unsigned DV) {
  const unsigned column = blockIdx.x * 64u + threadIdx.x;
  const unsigned width = Hv * DV;
  if (column >= width)
    return;
  const unsigned h = column / DV, kh = h / (Hv / Hk);
  float *col = state + (size_t)h * DK * DV + column % DV;
  for (unsigned t = 0; t < T; ++t) {
    const float *qt = q + ((size_t)t * Hk + kh) * DK;
    const float *kt = k + ((size_t)t * Hk + kh) * DK;
    const float a = decay[(size_t)t * Hv + h], b = beta[(size_t)t * Hv + h];
    float pred = 0.0f;
    for (unsigned i = 0; i < DK; ++i)
      pred = fmaf(col[(size_t)i * DV] * a, kt[i], pred);
    const float delta = ((float)v[(size_t)t * width + column] - pred) * b;
    float y = 0.0f;
    for (unsigned i = 0; i < DK; ++i) {
      float next = fmaf(kt[i], delta, col[(size_t)i * DV] * a);
      col[(size_t)i * DV] = next;
      y = fmaf(next, qt[i], y);
    }
    out[(size_t)t * width + column] = (half_t)y;
  }
}

} // namespace

hipError_t launch_delta_generic(const float *q, const float *k,
                                const uint16_t *v, const float *beta,
                                const float *decay, float *state,
                                uint16_t *out, const DeltaShape &s,
                                hipStream_t stream) {
  unsigned width = s.Hv * s.Dv;
  hipLaunchKernelGGL(delta_generic_kernel, dim3((width + 63) / 64), dim3(64), 0,
                     stream, q, k, reinterpret_cast<const half_t *>(v), beta,
                     decay, state, reinterpret_cast<half_t *>(out), s.T, s.Hk,
                     s.Dk, s.Hv, s.Dv);
  return hipGetLastError();
}

bool delta_recurrent_supported(const DeltaShape &s) {
  return (s.Dk == 64 || s.Dk == 128) && s.Dv % kColsPerWave == 0 &&
         s.Hk >= 1 && s.Hv % s.Hk == 0 && s.T >= 1;
}

hipError_t launch_delta_recurrent(const float *q, const float *k,
                                  const uint16_t *v, const float *beta,
                                  const float *decay, float *state,
                                  uint16_t *out, const DeltaShape &s,
                                  hipStream_t stream) {
  dim3 grid(s.Hv * (s.Dv / kColsPerWave));
  if (s.Dk == 64)
    hipLaunchKernelGGL(delta_recurrent_kernel<64>, grid, dim3(64), 0, stream,
                       q, k, reinterpret_cast<const half_t *>(v), beta, decay,
                       state, reinterpret_cast<half_t *>(out), s.T, s.Hk, s.Hv,
                       s.Dv);
  else
    hipLaunchKernelGGL(delta_recurrent_kernel<128>, grid, dim3(64), 0, stream,
                       q, k, reinterpret_cast<const half_t *>(v), beta, decay,
                       state, reinterpret_cast<half_t *>(out), s.T, s.Hk, s.Hv,
                       s.Dv);
  return hipGetLastError();
}

} // namespace llmi
