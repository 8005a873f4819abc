// The DeltaNet layer's front end, ahead of DeltaUpdate: the depthwise causal
// convolution with its history rows and SiLU (causalConv,
// Reference.metal:137-161), the per-head L2 normalisation of q and k to fp32
// (l2NormF32, Graph.metal:96-109) and the gates (deltaGates,
// Graph.metal:131-144, with logistic and stableSoftplus,
// Reference.metal:4-12). Results equal the reference's expressions in IEEE
// fp32, in its order, bit for bit, with exp and log correctly rounded (the
// oracle's convention; see exact_fp.hpp for how the roundings are kept).
//
// causalConv: the recurrence over tokens is only the sliding window of the
// last k-1 inputs, so a thread takes one channel and a block of 16 tokens
// (coalesced 2-byte loads across the wave's channels),
// reading its window from the inputs before the block (or, for the first
// block, from the history rows). Only the first block's thread reads the
// history, and it writes the new history (the last k-1 positions of the
// sequence) after reading, so no thread races it. Loads and stores are
// coalesced across the channels of a wave.
//
// l2NormF32: one wave per 16 rows; the rows are staged in LDS with 16-byte
// coalesced loads, lane r sums row r in index order (the reference's fma
// chain), and the fp32 outputs leave as 16-byte stores. Other widths and
// unaligned buffers take a thread per row.
//
// deltaGates: one thread per (token, head).
//
// gatedRmsNorm (the DeltaNet output's norm, Reference.metal:228-259): the
// l2NormF32 tile structure with the rmsNorm scale, the gate applied per
// element in the output pass.
#include "exact_fp.hpp"
#include "gated_norm.hpp"
#include "hip_common.hpp"
#include "kernels.hpp"

namespace llmi {
namespace {

constexpr unsigned kConvBlock = 16; // tokens per thread
constexpr unsigned kMaxKernel = 8;  // filter taps supported (history 7)
constexpr unsigned kL2Rows = 16;    // l2NormF32 rows per wave (16K rows fill 1024 waves)

__global__ __launch_bounds__(256) void causal_conv_kernel(
    const uint16_t *__restrict__ in, const uint16_t *__restrict__ w, uint16_t *hist,
    uint16_t *__restrict__ out, unsigned T, unsigned C, unsigned k, unsigned silu) {
  const unsigned c = blockIdx.x * 256 + threadIdx.x;
  if (c >= C)
    return;
  const unsigned hs = k - 1;
  const unsigned t0 = blockIdx.y * kConvBlock;
  const unsigned t1 = min(T, t0 + kConvBlock);
  float wf[kMaxKernel];
#pragma unroll
  for (unsigned j = 0; j < kMaxKernel; ++j)
    wf[j] = j < k ? h2f(w[c * k + j]) : 0.0f;
  // window[j] = the input at position t - hs + j (negative positions are
  // history slot hs + position)
  uint16_t win[kMaxKernel - 1];
  uint16_t old[kMaxKernel - 1];
#pragma unroll
  for (unsigned j = 0; j < kMaxKernel - 1; ++j) {
    old[j] = (t0 == 0 && j < hs) ? hist[c * hs + j] : 0;
    int pos = (int)t0 - (int)hs + (int)j;
    win[j] = j < hs ? (pos < 0 ? old[j] : in[(unsigned)pos * C + c]) : 0;
  }
  for (unsigned t = t0; t < t1; ++t) {
    uint16_t cur = in[t * C + c];
    float acc = mul32(h2f(cur), wf[hs]);
#pragma unroll
    for (unsigned j = 0; j < kMaxKernel - 1; ++j)
      if (j < hs)
        acc = __builtin_fmaf(h2f(win[j]), wf[j], acc);
    out[t * C + c] = silu ? silu16(round16(acc)) : f2h(acc);
#pragma unroll
    for (unsigned j = 0; j + 1 < kMaxKernel - 1; ++j)
      if (j + 1 < hs)
        win[j] = win[j + 1];
    if (hs)
      win[hs - 1] = cur;
  }
  if (t0 == 0) {
    // new history: positions T - hs .. T - 1 of [old history, inputs]
#pragma unroll
    for (unsigned j = 0; j < kMaxKernel - 1; ++j) {
      if (j < hs) {
        int pos = (int)T - (int)hs + (int)j;
        uint16_t v = 0;
        if (pos >= 0) {
          v = in[(unsigned)pos * C + c];
        } else {
#pragma unroll
          for (unsigned m = 0; m < kMaxKernel - 1; ++m)
            v = (int)m == (int)hs + pos ? old[m] : v;
        }
        hist[c * hs + j] = v;
      }
    }
  }
}

// The 4-tap case (Qwen3.5's conv) with the filter length known: a thread's
// 16 token loads are all issued before the first output is computed (the
// general kernel's loop waits one load latency per token), and the window
// lives in registers with fixed indices.
__global__ __launch_bounds__(256) void causal_conv_k4(
    const uint16_t *__restrict__ in, const uint16_t *__restrict__ w, uint16_t *hist,
    uint16_t *__restrict__ out, unsigned T, unsigned C, unsigned silu) {
  constexpr unsigned hs = 3;
  const unsigned c = blockIdx.x * 256 + threadIdx.x;
  if (c >= C)
    return;
  const unsigned t0 = blockIdx.y * kConvBlock;
  float wf[4];
#pragma unroll
  for (unsigned j = 0; j < 4; ++j)
    wf[j] = h2f(w[c * 4 + j]);
  // xs[u] = the input at position t0 - 3 + u (history for negative positions)
  uint16_t xs[kConvBlock + hs];
  uint16_t old[hs];
#pragma unroll
  for (unsigned j = 0; j < hs; ++j)
    old[j] = t0 == 0 ? hist[c * hs + j] : 0;
#pragma unroll
  for (unsigned u = 0; u < kConvBlock + hs; ++u) {
    int pos = (int)t0 - (int)hs + (int)u;
    xs[u] = pos < 0 ? old[u] : (pos < (int)T ? in[(unsigned)pos * C + c] : 0);
  }
#pragma unroll
  for (unsigned u = 0; u < kConvBlock; ++u) {
    if (t0 + u < T) {
      float acc = mul32(h2f(xs[u + hs]), wf[hs]);
#pragma unroll
      for (unsigned j = 0; j < hs; ++j)
        acc = __builtin_fmaf(h2f(xs[u + j]), wf[j], acc);
      out[(t0 + u) * C + c] = silu ? silu16(round16(acc)) : f2h(acc);
    }
  }
  if (t0 == 0) {
#pragma unroll
    for (unsigned j = 0; j < hs; ++j) {
      int pos = (int)T - (int)hs + (int)j;
      uint16_t v = 0;
      if (pos >= 0) {
        v = in[(unsigned)pos * C + c];
      } else {
#pragma unroll
        for (unsigned m = 0; m < hs; ++m)
          v = (int)m == (int)hs + pos ? old[m] : v;
      }
      hist[c * hs + j] = v;
    }
  }
}

__device__ __forceinline__ float l2_factor(float sum, float eps, float scale) {
  return l2_row_factor(sum, eps, scale);
}

// Rows of `width` (a multiple of 8, <= 256) halves, kL2Rows per wave.
__global__ __launch_bounds__(64) void l2_norm_tile(const uint16_t *__restrict__ in,
                                                   float *__restrict__ out, unsigned rows,
                                                   unsigned width, float eps, float scale) {
  __shared__ __align__(16) uint16_t tile[kL2Rows * (256 + 8)];
  __shared__ float fac[kL2Rows];
  const unsigned lane = threadIdx.x, pitch = width + 8, cpr = width / 8;
  const unsigned row0 = blockIdx.x * kL2Rows, nrows = min(kL2Rows, rows - row0);
  const unsigned chunks = nrows * cpr;
  for (unsigned c = lane; c < chunks; c += 64) {
    unsigned r = c / cpr, col = c - r * cpr;
    *reinterpret_cast<uint4_t *>(tile + r * pitch + col * 8) =
        *reinterpret_cast<const uint4_t *>(in + (row0 + r) * width + col * 8);
  }
  __syncthreads();
  if (lane < nrows) {
    const uint16_t *row = tile + lane * pitch;
    float sum = 0.0f;
    for (unsigned k = 0; k < cpr; ++k) {
      uint4_t q = *reinterpret_cast<const uint4_t *>(row + 8 * k);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float lo = h2f((uint16_t)(q[e] & 0xFFFFu)), hi = h2f((uint16_t)(q[e] >> 16));
        sum = __builtin_fmaf(lo, lo, sum);
        sum = __builtin_fmaf(hi, hi, sum);
      }
    }
    fac[lane] = l2_factor(sum, eps, scale);
  }
  __syncthreads();
  const unsigned quads = nrows * (width / 4), qpr = width / 4;
  for (unsigned c = lane; c < quads; c += 64) {
    unsigned r = c / qpr, col = c - r * qpr;
    const uint16_t *src = tile + r * pitch + col * 4;
    float f = fac[r];
    float4_t o;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      o[e] = mul32(h2f(src[e]), f);
    *reinterpret_cast<float4_t *>(out + (row0 + r) * width + col * 4) = o;
  }
}

__global__ __launch_bounds__(256) void l2_norm_rows(const uint16_t *__restrict__ in,
                                                    float *__restrict__ out, unsigned rows,
                                                    unsigned width, float eps, float scale) {
  unsigned r = blockIdx.x * 256 + threadIdx.x;
  if (r >= rows)
    return;
  const uint16_t *x = in + (size_t)r * width;
  float sum = 0.0f;
  for (unsigned i = 0; i < width; ++i) {
    float f = h2f(x[i]);
    sum = __builtin_fmaf(f, f, sum);
  }
  float f = l2_factor(sum, eps, scale);
  for (unsigned i = 0; i < width; ++i)
    out[(size_t)r * width + i] = mul32(h2f(x[i]), f);
}

// gatedRmsNorm for any width: one thread per row, the tile kernel's
// arithmetic (fma sum of squares in order, the same factor and products,
// the exact SiLU) on one element at a time.
template <bool kActivated>
__global__ __launch_bounds__(256) void gated_rms_norm_rows(const uint16_t *__restrict__ in,
                                                           const void *__restrict__ gate,
                                                           const float *__restrict__ w,
                                                           uint16_t *__restrict__ out,
                                                           unsigned rows, unsigned width,
                                                           float eps) {
  const unsigned r = blockIdx.x * 256 + threadIdx.x;
  if (r >= rows)
    return;
  const size_t base = (size_t)r * width;
  float sum = 0.0f;
  for (unsigned i = 0; i < width; ++i) {
    const float f = h2f(in[base + i]);
    sum = __builtin_fmaf(f, f, sum);
  }
  const float f = gated_norm_factor(sum, width, eps);
  for (unsigned i = 0; i < width; ++i) {
    const float norm = gated_norm_scaled(h2f(in[base + i]), f, w[i]);
    const float y =
        kActivated ? mul32(norm, static_cast<const float *>(gate)[base + i])
                   : gated_norm_silu_exact(norm, h2f(static_cast<const uint16_t *>(gate)[base + i]));
    out[base + i] = f2h(y);
  }
}

// gatedRmsNorm (Reference.metal:228-259): kL2Rows rows of `width` (a
// multiple of 8, <= 256) per wave, staged in LDS like l2_norm_tile; out =
// fp16(fp16(x * scale) * w * g) with g = silu(gate) for an fp16 gate (an
// estimate that the margin test accepts, else exact) or the fp32 gate.
// kQuant: the stored fp16 rows also quantized (quantizeActivation's
// expressions over the flattened rows: 32-wide groups, four lanes' chunks
// of eight, width a multiple of 32) into qout, scales and the invalid flag.
template <bool kActivated, bool kQuant>
__global__ __launch_bounds__(64) void gated_rms_norm_tile(const uint16_t *__restrict__ in,
                                                          const void *__restrict__ gate,
                                                          const float *__restrict__ w,
                                                          uint16_t *__restrict__ out,
                                                          unsigned rows, unsigned width,
                                                          float eps, int8_t *__restrict__ qout,
                                                          float *__restrict__ scales,
                                                          unsigned *invalid) {
  __shared__ __align__(16) uint16_t tile[kL2Rows * (256 + 8)];
  __shared__ float fac[kL2Rows];
  const unsigned lane = threadIdx.x, pitch = width + 8, cpr = width / 8;
  const unsigned row0 = blockIdx.x * kL2Rows, nrows = min(kL2Rows, rows - row0);
  const unsigned chunks = nrows * cpr;
  for (unsigned c = lane; c < chunks; c += 64) {
    unsigned r = c / cpr, col = c - r * cpr;
    *reinterpret_cast<uint4_t *>(tile + r * pitch + col * 8) =
        *reinterpret_cast<const uint4_t *>(in + (row0 + r) * width + col * 8);
  }
  __syncthreads();
  if (lane < nrows) {
    const uint16_t *row = tile + lane * pitch;
    float sum = 0.0f;
    for (unsigned k = 0; k < cpr; ++k) {
      uint4_t q = *reinterpret_cast<const uint4_t *>(row + 8 * k);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float lo = h2f((uint16_t)(q[e] & 0xFFFFu)), hi = h2f((uint16_t)(q[e] >> 16));
        sum = __builtin_fmaf(lo, lo, sum);
        sum = __builtin_fmaf(hi, hi, sum);
      }
    }
    fac[lane] = gated_norm_factor(sum, width, eps);
  }
  __syncthreads();
  for (unsigned c = lane; c < chunks; c += 64) {
    unsigned r = c / cpr, col = c - r * cpr;
    const unsigned base = (row0 + r) * width + col * 8;
    uint4_t q = *reinterpret_cast<const uint4_t *>(tile + r * pitch + col * 8);
    float gv[8];
    if (kActivated) {
      const float *g = static_cast<const float *>(gate) + base;
      float4_t g0 = *reinterpret_cast<const float4_t *>(g);
      float4_t g1 = *reinterpret_cast<const float4_t *>(g + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        gv[e] = g0[e];
        gv[e + 4] = g1[e];
      }
    } else {
      uint4_t g = *reinterpret_cast<const uint4_t *>(static_cast<const uint16_t *>(gate) + base);
#pragma unroll
      for (int e = 0; e < 8; ++e)
        gv[e] = h2f((uint16_t)(g[e / 2] >> (16 * (e & 1))));
    }
    const float f = fac[r];
    float norm[8], y[8];
    unsigned need = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      norm[e] = gated_norm_scaled(h2f((uint16_t)(q[e / 2] >> (16 * (e & 1)))), f, w[col * 8 + e]);
      if (kActivated) {
        y[e] = mul32(norm[e], gv[e]);
      } else {
        y[e] = gated_norm_silu_estimate(norm[e], gv[e]);
        need |= f16_settled(y[e]) ? 0u : 1u << e;
      }
    }
    // the few that the margin test rejects, one shared pass each (as in
    // sigmoid_mul_vec)
    while (need) {
      unsigned k = __builtin_ctz(need);
      need &= need - 1;
      float gk = gv[0], nk = norm[0];
#pragma unroll
      for (int e = 1; e < 8; ++e) {
        gk = k == (unsigned)e ? gv[e] : gk;
        nk = k == (unsigned)e ? norm[e] : nk;
      }
      float yk = gated_norm_silu_exact(nk, gk);
#pragma unroll
      for (int e = 0; e < 8; ++e)
        y[e] = k == (unsigned)e ? yk : y[e];
    }
    uint4_t o;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      o[e] = (uint32_t)f2h(y[2 * e]) | ((uint32_t)f2h(y[2 * e + 1]) << 16);
    *reinterpret_cast<uint4_t *>(out + base) = o;
    if constexpr (kQuant)
      quantize_chunk8(y, qout + base, scales + base / 32, invalid, (c & 3u) == 0);
  }
}

__global__ __launch_bounds__(256) void delta_gates_kernel(
    const uint16_t *__restrict__ a, const uint16_t *__restrict__ b,
    const float *__restrict__ a_log, const float *__restrict__ dt_bias,
    float *__restrict__ beta, float *__restrict__ decay, unsigned count, unsigned width) {
  unsigned i = blockIdx.x * 256 + threadIdx.x;
  if (i >= count)
    return;
  unsigned head = i % width;
  float bf = h2f(b[i]);
  float s = logistic_estimate(bf);
  if (!f16_settled(s))
    s = logistic_exact(bf);
  beta[i] = round16(s);
  float sp = stable_softplus(__fadd_rn(h2f(a[i]), dt_bias[head]));
  decay[i] = exp_cr(mul32(-exp_cr(a_log[head]), sp));
}

} // namespace

bool causal_conv_supported(unsigned k) { return k >= 1 && k <= kMaxKernel; }

hipError_t launch_causal_conv(const uint16_t *in, const uint16_t *w, uint16_t *hist,
                              uint16_t *out, unsigned T, unsigned C, unsigned k,
                              unsigned silu, hipStream_t stream) {
  if (T == 0 || C == 0)
    return hipSuccess;
  dim3 grid((C + 255) / 256, (T + kConvBlock - 1) / kConvBlock);
  if (k == 4)
    hipLaunchKernelGGL(causal_conv_k4, grid, dim3(256), 0, stream, in, w, hist, out, T, C, silu);
  else
    hipLaunchKernelGGL(causal_conv_kernel, grid, dim3(256), 0, stream, in, w, hist, out, T,
                       C, k, silu);
  return hipGetLastError();
}

bool l2_norm_tiled(unsigned width, const void *in, const void *out) {
  return width % 8 == 0 && width <= 256 && aligned16(in) && aligned16(out);
}

hipError_t launch_l2_norm(const uint16_t *in, float *out, unsigned rows, unsigned width,
                          float eps, float scale, hipStream_t stream) {
  if (rows == 0 || width == 0)
    return hipSuccess;
  if (l2_norm_tiled(width, in, out))
    hipLaunchKernelGGL(l2_norm_tile, dim3((rows + kL2Rows - 1) / kL2Rows), dim3(64), 0, stream, in, out,
                       rows, width, eps, scale);
  else
    hipLaunchKernelGGL(l2_norm_rows, dim3((rows + 255) / 256), dim3(256), 0, stream, in, out,
                       rows, width, eps, scale);
  return hipGetLastError();
}

bool gated_rms_norm_tiled(unsigned width, const void *in, const void *gate, const void *out) {
  return width % 8 == 0 && width <= 256 && aligned16(in) && aligned16(gate) && aligned16(out);
}

hipError_t launch_gated_rms_norm(const uint16_t *in, const void *gate, bool activated,
                                 const float *w, uint16_t *out, unsigned rows, unsigned width,
                                 float eps, hipStream_t stream) {
  if (rows == 0 || width == 0)
    return hipSuccess;
  if (!gated_rms_norm_tiled(width, in, gate, out)) {
    const dim3 g((rows + 255) / 256);
    if (activated)
      hipLaunchKernelGGL(gated_rms_norm_rows<true>, g, dim3(256), 0, stream, in, gate, w, out,
                         rows, width, eps);
    else
      hipLaunchKernelGGL(gated_rms_norm_rows<false>, g, dim3(256), 0, stream, in, gate, w, out,
                         rows, width, eps);
    return hipGetLastError();
  }
  dim3 grid((rows + kL2Rows - 1) / kL2Rows);
  if (activated)
    hipLaunchKernelGGL((gated_rms_norm_tile<true, false>), grid, dim3(64), 0, stream, in, gate,
                       w, out, rows, width, eps, nullptr, nullptr, nullptr);
  else
    hipLaunchKernelGGL((gated_rms_norm_tile<false, false>), grid, dim3(64), 0, stream, in, gate,
                       w, out, rows, width, eps, nullptr, nullptr, nullptr);
  return hipGetLastError();
}

bool gated_rms_norm_quantize_supported(unsigned width, const void *in, const void *gate,
                                       const void *out, const void *q) {
  return width % 32 == 0 && gated_rms_norm_tiled(width, in, gate, out) && aligned16(q);
}

hipError_t launch_gated_rms_norm_quantize(const uint16_t *in, const float *gate, const float *w,
                                          uint16_t *out, int8_t *q, float *scales,
                                          unsigned *invalid, unsigned rows, unsigned width,
                                          float eps, hipStream_t stream) {
  if (rows == 0)
    return hipSuccess;
  hipLaunchKernelGGL((gated_rms_norm_tile<true, true>), dim3((rows + kL2Rows - 1) / kL2Rows),
                     dim3(64), 0, stream, in, gate, w, out, rows, width, eps, q, scales,
                     invalid);
  return hipGetLastError();
}

hipError_t launch_delta_gates(const uint16_t *a, const uint16_t *b, const float *a_log,
                              const float *dt_bias, float *beta, float *decay,
                              unsigned rows, unsigned width, hipStream_t stream) {
  unsigned count = rows * width;
  if (count == 0)
    return hipSuccess;
  hipLaunchKernelGGL(delta_gates_kernel, dim3((count + 255) / 256), dim3(256), 0, stream, a, b,
                     a_log, dt_bias, beta, decay, count, width);
  return hipGetLastError();
}

} // namespace llmi
