// Gated delta rule, token-recurrent form: the DeltaNet decode step.
//
// Same arithmetic as graphDeltaUpdate / updateDeltaColumn
// (Graph.metal:146-170, Reference.metal:182-197), which gives one thread a
// whole state column in device memory and walks it twice per token. Here
// the state lives in registers for the whole call:
//
//  * a workgroup of NW waves serves a slice of CW consecutive state columns
//    of one value head; lane l of a wave holds column l % CW, and the wave's
//    64 / CW lane groups and the NW waves split the dk rows between them
//    (RPL rows per lane). A state load instruction therefore reads whole
//    CW * 4-byte row segments (64 lanes over 64 / CW rows), and the grid
//    has Hv * dv / CW workgroups;
//  * per token the two column dot products (k.S for the prediction and q.S
//    for the output) are partial sums over a lane's rows; the partials of
//    a column meet in LDS, where every lane of the column adds them in the
//    same order, so all of them hold the same prediction;
//  * the state is read from HBM once at the start and written once at the
//    end, so a decode step moves exactly the 2 x Hv*dk*dv*4 state bytes plus
//    the step's q/k/v/gates.
//
// Summation order inside a dot product differs from the reference's single
// fma chain (four interleaved chains per lane plus the partials in LDS); the
// result stays within fp32 rounding of the sequential order.
#include "hip_common.hpp"
#include "kernels.hpp"

#include <stdlib.h>

namespace llmi {
namespace {

template <int DK, int CW, int NW>
__global__ __launch_bounds__(64 * NW) void delta_recurrent_kernel(
    const float *__restrict__ q, const float *__restrict__ k,
    const half_t *__restrict__ v, const float *__restrict__ beta,
    const float *__restrict__ decay, float *__restrict__ state,
    half_t *__restrict__ out, unsigned T, unsigned Hk, unsigned Hv,
    unsigned DV) {
  constexpr int RG = 64 / CW;  // row groups per wave
  constexpr int NP = NW * RG;  // partial sums per column
  constexpr int RPL = DK / NP; // rows per lane
  static_assert(RPL % 4 == 0 && RPL * NP == DK, "rows per lane must be a multiple of 4");
  const unsigned tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const unsigned c = lane % CW, part = wave * RG + lane / CW;
  const unsigned slices = DV / CW;
  const unsigned h = blockIdx.x / slices;
  const unsigned col = (blockIdx.x % slices) * CW + c;
  const unsigned kh = h / (Hv / Hk);
  const unsigned row0 = part * RPL;
  const size_t vwidth = (size_t)Hv * DV;

  float S[RPL];
  float *sbase = state + ((size_t)h * DK + row0) * DV + col;
#pragma unroll
  for (int m = 0; m < RPL; ++m)
    S[m] = sbase[(size_t)m * DV];

  __shared__ float sPred[NP][CW], sY[NP][CW];
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
    sPred[part][c] = (p4[0] + p4[1]) + (p4[2] + p4[3]);
    __syncthreads();
    float pred = 0.0f;
#pragma unroll
    for (int i = 0; i < NP; ++i)
      pred += sPred[i][c];
    const float delta = (vj - pred) * b;

    float y4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int m = 0; m < RPL; ++m) {
      S[m] = fmaf(kr[m], delta, S[m] * a);
      y4[m % 4] = fmaf(S[m], qr[m], y4[m % 4]);
    }
    sY[part][c] = (y4[0] + y4[1]) + (y4[2] + y4[3]);
    __syncthreads();
    if (part == 0) {
      float y = 0.0f;
#pragma unroll
      for (int i = 0; i < NP; ++i)
        y += sY[i][c];
      out[(size_t)t * vwidth + (size_t)h * DV + col] = (half_t)y;
    }
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

namespace {

// Column slice of a workgroup: 32 columns when dv allows, else 16.
// LLMI_DELTA_DECODE_CW (64, 32 or 16) and LLMI_DELTA_DECODE_NW (waves per
// workgroup: 2, 4 or 8) override the choice for tuning.
unsigned env_or(const char *name, unsigned dflt) {
  const char *e = getenv(name);
  if (!e || !*e)
    return dflt;
  long x = strtol(e, nullptr, 10);
  return x > 0 ? (unsigned)x : dflt;
}

unsigned slice_cols(unsigned dv) {
  static const unsigned forced = env_or("LLMI_DELTA_DECODE_CW", 0);
  if (forced && dv % forced == 0)
    return forced;
  return dv % 32 == 0 ? 32 : 16;
}

unsigned waves_per_group() {
  static const unsigned v = env_or("LLMI_DELTA_DECODE_NW", 4);
  return v;
}

template <int DK, int CW, int NW>
hipError_t launch_rec(const float *q, const float *k, const uint16_t *v, const float *beta,
                      const float *decay, float *state, uint16_t *out, const DeltaShape &s,
                      hipStream_t stream) {
  hipLaunchKernelGGL((delta_recurrent_kernel<DK, CW, NW>), dim3(s.Hv * (s.Dv / CW)),
                     dim3(64 * NW), 0, stream, q, k, reinterpret_cast<const half_t *>(v),
                     beta, decay, state, reinterpret_cast<half_t *>(out), s.T, s.Hk, s.Hv,
                     s.Dv);
  return hipGetLastError();
}

template <int DK, int CW>
hipError_t launch_rec_cw(const float *q, const float *k, const uint16_t *v, const float *beta,
                         const float *decay, float *state, uint16_t *out, const DeltaShape &s,
                         hipStream_t stream) {
  // Rows per lane DK / (NW * 64 / CW) must stay a multiple of 4.
  constexpr bool ok8 = DK % (8 * (64 / CW) * 4) == 0, ok2 = DK % (2 * (64 / CW) * 4) == 0;
  const unsigned nw = waves_per_group();
  if constexpr (ok8)
    if (nw == 8)
      return launch_rec<DK, CW, 8>(q, k, v, beta, decay, state, out, s, stream);
  if constexpr (ok2)
    if (nw == 2)
      return launch_rec<DK, CW, 2>(q, k, v, beta, decay, state, out, s, stream);
  return launch_rec<DK, CW, 4>(q, k, v, beta, decay, state, out, s, stream);
}

} // namespace

bool delta_recurrent_supported(const DeltaShape &s) {
  return (s.Dk == 64 || s.Dk == 128) && s.Dv % 16 == 0 && s.Hk >= 1 &&
         s.Hv % s.Hk == 0 && s.T >= 1;
}

hipError_t launch_delta_recurrent(const float *q, const float *k,
                                  const uint16_t *v, const float *beta,
                                  const float *decay, float *state,
                                  uint16_t *out, const DeltaShape &s,
                                  hipStream_t stream) {
  const unsigned cw = slice_cols(s.Dv);
  if (s.Dk == 64) {
    if (cw == 64)
      return launch_rec_cw<64, 64>(q, k, v, beta, decay, state, out, s, stream);
    if (cw == 32)
      return launch_rec_cw<64, 32>(q, k, v, beta, decay, state, out, s, stream);
    return launch_rec_cw<64, 16>(q, k, v, beta, decay, state, out, s, stream);
  }
  if (cw == 64)
    return launch_rec_cw<128, 64>(q, k, v, beta, decay, state, out, s, stream);
  if (cw == 32)
    return launch_rec_cw<128, 32>(q, k, v, beta, decay, state, out, s, stream);
  return launch_rec_cw<128, 16>(q, k, v, beta, decay, state, out, s, stream);
}

} // namespace llmi
