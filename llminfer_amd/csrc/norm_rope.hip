// The attention block's row work around CausalGqa: the q/k RmsNorm fused with
// the partial rotary embedding (normRope, Reference.metal:271-293, with
// rmsScale :98-103 and rotatePair :262-269), its two halves on their own
// (rmsNorm, Reference.metal:105-117; partialRope, Graph.metal:111-129), and
// the output gate (sigmoidMul, Graph.metal:78-85).
//
// Results are bit for bit those of the reference's expressions, evaluated
// with IEEE fp32 arithmetic in the reference's order:
//  * the sum of squares is the reference's sequential fma chain, one lane per
//    row (the rows are staged through LDS so that HBM reads stay coalesced);
//  * rsqrt is 1/sqrt, both correctly rounded (the float square root is taken
//    in double and rounded once, which is exact rounding for a float
//    argument; HIP's __fsqrt_rn is the native, not always rounded-to-nearest
//    instruction);
//  * every rounding of the reference is kept. The file is compiled with
//    -ffp-contract=off (llminfer_amd/build.py), and each product and each
//    fp16 rounding passes through opaque(), an empty asm statement: without
//    it the gfx950 backend selects v_fma_mixlo_f16 for an fp32 product
//    converted to fp16 (one rounding instead of two, and +0 for a -0
//    product) and v_fma_mix_f32 for an fp16-rounded product added to
//    another, whatever the contraction setting.
//  * pow, cos, sin and exp are the correctly rounded fp32 functions. cos, sin
//    and exp are used only through their fp16 rounding, so the fast fp32
//    library function decides whenever every value within 2^-19 relative of
//    its result rounds to the same fp16 (its error is a few ulp, far inside
//    that; 2^-21 for cos and sin); otherwise, and always for pow, the value
//    is evaluated in double and rounded to float once.
//
// normRope tile kernel: one wave per block owns `rw` consecutive rows.
//   1. the wave loads the rows' headDim halves with 16-byte coalesced loads
//      and stores them to LDS (row pitch headDim + 8 halves); the inverse
//      frequencies pow(theta, 2i/rotaryDim) come precomputed in the kernel
//      arguments;
//   2. the lanes fill the (token, pair) -> (cos, sin) table of the rows'
//      tokens, and lane r sums row r sequentially from LDS;
//   3. the rotary pairs (per item a row and 8 pairs: the chunks at columns j
//      and j + rotaryDim/2), then the copied columns (per item one chunk),
//      are normalised, rotated and stored with 16-byte stores.
// Shapes outside the tile kernel's alignment rules (headDim, headStride or
// rotaryDim/2 not a multiple of 8 halves, unaligned pointers, headDim > 2048)
// run the row kernel: one thread per row, the reference's own structure,
// with the same arithmetic.
#include "exact_fp.hpp"
#include "hip_common.hpp"
#include "kernels.hpp"
#include "rope_gate.hpp"

#include <math.h>
#include <string.h>


namespace llmi {
namespace {

constexpr int kPad = 8;                 // halves of LDS padding per tile row
// Rows past the tile's width limit, up to 16K halves, take a workgroup each.
constexpr unsigned kWideMin = 256, kWideMax = 16384;
constexpr unsigned kTileHalves = 8192;  // rows * headDim bound of one tile
constexpr unsigned kTileIters = kTileHalves / 8 / 64;

struct TileArgs {
  unsigned rows, heads, D, rot, stride, past, out_row0, rw, maxtok;
  float eps, theta;
};

__device__ __forceinline__ float inv_freq(const RopeFreqs &f, const TileArgs &a,
                                          unsigned i) {
  return a.rot / 2 <= kArgFreqs ? f.v[i] : rope_inv_freq(a.theta, i, a.rot);
}

template <bool kNorm>
__global__ __launch_bounds__(64) void norm_rope_tile(const uint16_t *in,
                                                     const float *__restrict__ w,
                                                     uint16_t *out, TileArgs a,
                                                     RopeFreqs f) {
  extern __shared__ __align__(16) unsigned char smem[];
  const unsigned lane = threadIdx.x;
  const unsigned pitch = a.D + kPad;
  const unsigned half = a.rot / 2;
  uint16_t *tile = reinterpret_cast<uint16_t *>(smem);
  float *sc = reinterpret_cast<float *>(tile + a.rw * pitch);
  unsigned *rtok = reinterpret_cast<unsigned *>(sc + ((a.rw + 1) & ~1u));
  float *wt1 = reinterpret_cast<float *>(rtok + ((a.rw + 1) & ~1u));
  float2 *cs = reinterpret_cast<float2 *>(wt1 + (kNorm ? a.D : 0));

  const unsigned row0 = blockIdx.x * a.rw;
  const unsigned nrows = min(a.rw, a.rows - row0);
  const unsigned cpr = a.D / 8; // 16-byte chunks per row
  // Lane l owns chunks l, l + 64, ... of the tile, row-major; (r, col) of
  // the next one follows by a uniform step, without a division per chunk.
  const unsigned step_r = 64 / cpr, step_c = 64 - step_r * cpr;
  const unsigned lane_r = lane / cpr, lane_c = lane - lane_r * cpr;
  auto advance = [&](unsigned &r, unsigned &col) {
    col += step_c;
    r += step_r;
    if (col >= cpr) {
      col -= cpr;
      ++r;
    }
  };

  // 1. coalesced loads of the tile, after the first inverse frequency each
  //    lane needs for the cos/sin table (so that it is there before them).
  const unsigned tok0 = row0 / a.heads;
  const unsigned ntok = (row0 + nrows - 1) / a.heads - tok0 + 1;
  const unsigned entries = ntok * half;
  float inv0 = lane < entries ? inv_freq(f, a, lane % half) : 1.0f;
  uint4_t v[kTileIters];
  {
    unsigned r = lane_r, col = lane_c;
#pragma unroll
    for (unsigned it = 0; it < kTileIters; ++it) {
      if (r < nrows)
        v[it] = *reinterpret_cast<const uint4_t *>(in + (row0 + r) * a.stride + col * 8);
      advance(r, col);
    }
  }
  if (kNorm)
    for (unsigned i = lane; i < a.D; i += 64)
      wt1[i] = 1.0f + w[i];
  if (lane < nrows)
    rtok[lane] = ((row0 + lane) / a.heads - tok0) * half;
  {
    unsigned r = lane_r, col = lane_c;
#pragma unroll
    for (unsigned it = 0; it < kTileIters; ++it) {
      if (r < nrows)
        *reinterpret_cast<uint4_t *>(tile + r * pitch + col * 8) = v[it];
      advance(r, col);
    }
  }
  __syncthreads();

  // 2. the cos/sin table and the sequential sums (lane = row; every lane
  //    runs the chain, on a valid row, so that the code stays straight and
  //    the table's arithmetic fills the chain's latency).
  if (lane < entries) {
    float position = (float)(a.past + tok0 + lane / half);
    cs[lane] = rope_cos_sin(__fdiv_rn(position, inv0));
  }
  for (unsigned e = lane + 64; e < entries; e += 64) {
    unsigned t = e / half, i = e - t * half;
    float position = (float)(a.past + tok0 + t);
    cs[e] = rope_cos_sin(__fdiv_rn(position, inv_freq(f, a, i)));
  }
  if (kNorm) {
    const uint16_t *row = tile + min(lane, nrows - 1) * pitch;
    float sum = 0.0f;
    unsigned k = 0;
    for (; k + 4 <= cpr; k += 4) {
      uint4_t q[4];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        q[u] = *reinterpret_cast<const uint4_t *>(row + 8 * (k + u));
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float lo = h2f((uint16_t)(q[u][e] & 0xFFFFu));
          float hi = h2f((uint16_t)(q[u][e] >> 16));
          sum = __builtin_fmaf(lo, lo, sum);
          sum = __builtin_fmaf(hi, hi, sum);
        }
    }
    for (; k < cpr; ++k) {
      uint4_t q = *reinterpret_cast<const uint4_t *>(row + 8 * k);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float lo = h2f((uint16_t)(q[e] & 0xFFFFu));
        float hi = h2f((uint16_t)(q[e] >> 16));
        sum = __builtin_fmaf(lo, lo, sum);
        sum = __builtin_fmaf(hi, hi, sum);
      }
    }
    if (lane < nrows)
      sc[lane] = rms_scale_of(sum, a.D, a.eps);
  }
  __syncthreads();

  // 3. normalise, rotate, store: first the rotary pairs (an item is a row
  //    and 8 pairs: two 16-byte chunks, columns j0 and j0 + rotaryDim/2),
  //    then the copied columns (an item is one chunk), so that every lane
  //    of a pass does the same kind of work.
  const unsigned pchunks = half / 8;
  if (pchunks) {
    const unsigned sr = 64 / pchunks, sc_ = 64 - sr * pchunks;
    unsigned r = lane / pchunks, k = lane - r * pchunks;
    for (; r < nrows;) {
      unsigned j0 = 8 * k, j1 = j0 + half;
      const uint16_t *row = tile + r * pitch;
      uint4_t qx = *reinterpret_cast<const uint4_t *>(row + j0);
      uint4_t qy = *reinterpret_cast<const uint4_t *>(row + j1);
      float scale = kNorm ? sc[r] : 1.0f;
      const float2 *csr = cs + rtok[r] + j0;
      uint16_t ox[8], oy[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        uint16_t bx = (uint16_t)(qx[e / 2] >> (16 * (e & 1)));
        uint16_t by = (uint16_t)(qy[e / 2] >> (16 * (e & 1)));
        float x = kNorm ? normed(bx, scale, wt1[j0 + e]) : h2f(bx);
        float y = kNorm ? normed(by, scale, wt1[j1 + e]) : h2f(by);
        float2 t = csr[e];
        ox[e] = rotate_x(x, y, t);
        oy[e] = rotate_y(x, y, t);
      }
      uint4_t sx, sy;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        sx[e] = (uint32_t)ox[2 * e] | ((uint32_t)ox[2 * e + 1] << 16);
        sy[e] = (uint32_t)oy[2 * e] | ((uint32_t)oy[2 * e + 1] << 16);
      }
      uint16_t *dst = out + (a.out_row0 + row0 + r) * a.D;
      *reinterpret_cast<uint4_t *>(dst + j0) = sx;
      *reinterpret_cast<uint4_t *>(dst + j1) = sy;
      k += sc_;
      r += sr;
      if (k >= pchunks) {
        k -= pchunks;
        ++r;
      }
    }
  }
  const unsigned first = a.rot / 8, pass = cpr - first;
  if (pass) {
    const unsigned sr = 64 / pass, sc_ = 64 - sr * pass;
    unsigned r = lane / pass, k = lane - r * pass;
    for (; r < nrows;) {
      unsigned j0 = 8 * (first + k);
      uint4_t q = *reinterpret_cast<const uint4_t *>(tile + r * pitch + j0);
      float scale = kNorm ? sc[r] : 1.0f;
      uint4_t st;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        uint16_t lo = (uint16_t)(q[e] & 0xFFFFu), hi = (uint16_t)(q[e] >> 16);
        if (kNorm) {
          lo = f2h(normed(lo, scale, wt1[j0 + 2 * e]));
          hi = f2h(normed(hi, scale, wt1[j0 + 2 * e + 1]));
        }
        st[e] = (uint32_t)lo | ((uint32_t)hi << 16);
      }
      *reinterpret_cast<uint4_t *>(out + (a.out_row0 + row0 + r) * a.D + j0) = st;
      k += sc_;
      r += sr;
      if (k >= pass) {
        k -= pass;
        ++r;
      }
    }
  }
}

// One thread per row: the reference kernel's structure, for any alignment.
template <bool kNorm>
__global__ __launch_bounds__(256) void norm_rope_rows(const uint16_t *in,
                                                      const float *__restrict__ w,
                                                      uint16_t *out, TileArgs a,
                                                      RopeFreqs f) {
  unsigned row = blockIdx.x * 256 + threadIdx.x;
  if (row >= a.rows)
    return;
  const uint16_t *head = in + (size_t)row * a.stride;
  uint16_t *dst = out + (size_t)(a.out_row0 + row) * a.D;
  float scale = 1.0f;
  if (kNorm) {
    float sum = 0.0f;
    for (unsigned i = 0; i < a.D; ++i) {
      float f = h2f(head[i]);
      sum = __builtin_fmaf(f, f, sum);
    }
    scale = rms_scale_of(sum, a.D, a.eps);
  }
  unsigned half = a.rot / 2;
  float position = (float)(a.past + row / a.heads);
  for (unsigned i = 0; i < half; ++i) {
    unsigned j = i + half;
    float x = kNorm ? normed(head[i], scale, 1.0f + w[i]) : h2f(head[i]);
    float y = kNorm ? normed(head[j], scale, 1.0f + w[j]) : h2f(head[j]);
    float2 t = rope_cos_sin(__fdiv_rn(position, inv_freq(f, a, i)));
    uint16_t ox = rotate_x(x, y, t), oy = rotate_y(x, y, t);
    dst[i] = ox;
    dst[j] = oy;
  }
  for (unsigned i = a.rot; i < a.D; ++i)
    dst[i] = kNorm ? f2h(normed(head[i], scale, 1.0f + w[i])) : head[i];
}

// Rows wider than the tile (the 2560-wide hidden rows of the model's
// RMSNorms): a workgroup per row. All 256 threads stage the row in LDS as
// fp32 (x itself and, for the norm, nothing else: x * x is exact in fp32
// for an fp16 x, so the chain needs only the fma); one lane then runs
// rmsScale's fma chain in order -- the reference's one sequential fp32
// sum, bound by one wave's VALU issue (~8 cycles an instruction, ~9 us at
// width 2560) -- reading 4 terms per LDS load; every thread then writes its
// share of the outputs.
template <bool kNorm>
__global__ __launch_bounds__(256) void norm_rope_wide(const uint16_t *in,
                                                      const float *__restrict__ w,
                                                      uint16_t *out, TileArgs a, RopeFreqs f) {
  extern __shared__ __align__(16) float srow[];
  __shared__ float sscale;
  const unsigned row = blockIdx.x, t = threadIdx.x;
  const uint16_t *head = in + (size_t)row * a.stride;
  uint16_t *dst = out + (size_t)(a.out_row0 + row) * a.D;
  const unsigned padded = (a.D + 31) / 32 * 32;
  for (unsigned i = t; i < padded; i += 256)
    srow[i] = i < a.D ? h2f(head[i]) : 0.0f;
  __syncthreads();
  if (kNorm && t == 0) {
    // fma(0, 0, sum) == sum for the padding: sum starts at +0 and a sum of
    // squares is never -0.
    const float4 *v = reinterpret_cast<const float4 *>(srow);
    const unsigned n = padded / 4; // a multiple of 8
    float sum = 0.0f;
#pragma unroll 8
    for (unsigned c = 0; c < n; ++c) {
      const float4 q = v[c];
      sum = __builtin_fmaf(q.x, q.x, sum);
      sum = __builtin_fmaf(q.y, q.y, sum);
      sum = __builtin_fmaf(q.z, q.z, sum);
      sum = __builtin_fmaf(q.w, q.w, sum);
    }
    sscale = rms_scale_of(sum, a.D, a.eps);
  }
  __syncthreads();
  const float scale = kNorm ? sscale : 1.0f;
  const unsigned half = a.rot / 2;
  const float position = (float)(a.past + row / a.heads);
  for (unsigned i = t; i < half; i += 256) {
    const unsigned j = i + half;
    const float x = kNorm ? normed_f(srow[i], scale, 1.0f + w[i]) : srow[i];
    const float y = kNorm ? normed_f(srow[j], scale, 1.0f + w[j]) : srow[j];
    const float2 cs = rope_cos_sin(__fdiv_rn(position, inv_freq(f, a, i)));
    dst[i] = rotate_x(x, y, cs);
    dst[j] = rotate_y(x, y, cs);
  }
  for (unsigned i = a.rot + t; i < a.D; i += 256)
    dst[i] = kNorm ? f2h(normed_f(srow[i], scale, 1.0f + w[i])) : f2h(srow[i]);
}

// Eight gates per lane: the estimates first, then the exact evaluation for
// the few that need it, one per pass (a pass costs the wave one double exp,
// so the lanes share passes instead of running one per element slot).
__global__ __launch_bounds__(256) void sigmoid_mul_vec(const uint4_t *__restrict__ gate,
                                                       const uint4_t *__restrict__ in,
                                                       uint4_t *__restrict__ out,
                                                       unsigned vectors) {
  unsigned i = blockIdx.x * 256 + threadIdx.x;
  if (i >= vectors)
    return;
  uint4_t gv = __builtin_nontemporal_load(gate + i);
  uint4_t xv = __builtin_nontemporal_load(in + i);
  float g[8], s[8];
  unsigned need = 0;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    g[e] = h2f((uint16_t)(gv[e / 2] >> (16 * (e & 1))));
    s[e] = logistic_estimate(g[e]);
    need |= f16_settled(s[e]) ? 0u : 1u << e;
  }
  while (need) {
    unsigned k = __builtin_ctz(need);
    need &= need - 1;
    float gk = g[0];
#pragma unroll
    for (int e = 1; e < 8; ++e)
      gk = k == (unsigned)e ? g[e] : gk;
    float sk = logistic_exact(gk);
#pragma unroll
    for (int e = 0; e < 8; ++e)
      s[e] = k == (unsigned)e ? sk : s[e];
  }
  uint4_t o;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    uint16_t lo = f2h(mul32(round16(s[2 * e]), h2f((uint16_t)(xv[e] & 0xFFFFu))));
    uint16_t hi = f2h(mul32(round16(s[2 * e + 1]), h2f((uint16_t)(xv[e] >> 16))));
    o[e] = (uint32_t)lo | ((uint32_t)hi << 16);
  }
  __builtin_nontemporal_store(o, out + i);
}

__global__ __launch_bounds__(256) void sigmoid_mul_scalar(const uint16_t *__restrict__ gate,
                                                          const uint16_t *__restrict__ in,
                                                          uint16_t *__restrict__ out,
                                                          unsigned count) {
  unsigned i = blockIdx.x * 256 + threadIdx.x;
  if (i < count)
    out[i] = gate_one(gate[i], in[i]);
}

// Rows per tile and the table bound for a shape the tile kernel takes.
struct TilePlan {
  unsigned rw, maxtok;
  size_t lds;
};

TilePlan plan_tile(const RopeShape &s) {
  unsigned rw = kTileHalves / s.D;
  rw = rw > s.rows_per_tile ? s.rows_per_tile : rw;
  rw = rw < 1 ? 1 : rw;
  TilePlan p{};
  const unsigned half = s.rot / 2;
  for (;;) {
    p.rw = rw;
    p.maxtok = (rw - 1) / s.heads + 2;
    if (p.maxtok > rw)
      p.maxtok = rw;
    size_t table = (size_t)p.maxtok * half * sizeof(float2);
    if (rw <= 8 || table <= 16384)
      break;
    rw /= 2;
  }
  p.lds = (size_t)p.rw * (s.D + kPad) * 2 + (size_t)((p.rw + 1) & ~1u) * 8 +
          (s.norm ? (size_t)s.D * 4 : 0) + (size_t)p.maxtok * half * sizeof(float2);
  return p;
}


} // namespace

bool norm_rope_tiled(const RopeShape &s, const void *in, const void *out) {
  return s.D % 8 == 0 && s.D <= 2048 && s.stride % 8 == 0 && (s.rot / 2) % 8 == 0 &&
         aligned16(in) && aligned16(out);
}

bool norm_rope_wide_rows(const RopeShape &s) { return s.D > kWideMin && s.D <= kWideMax; }

hipError_t launch_norm_rope(const uint16_t *in, const float *w, uint16_t *out,
                            const RopeShape &s, hipStream_t stream) {
  if (s.rows == 0 || s.D == 0)
    return hipSuccess;
  TileArgs a{s.rows, s.heads, s.D, s.rot, s.stride, s.past, s.out_row0, 0, 0,
             s.eps, s.theta};
  const RopeFreqs &f = host_freqs(s.theta, s.rot);
  if (norm_rope_tiled(s, in, out)) {
    TilePlan p = plan_tile(s);
    a.rw = p.rw;
    a.maxtok = p.maxtok;
    dim3 grid((s.rows + p.rw - 1) / p.rw);
    if (s.norm)
      hipLaunchKernelGGL(norm_rope_tile<true>, grid, dim3(64), p.lds, stream, in, w, out, a, f);
    else
      hipLaunchKernelGGL(norm_rope_tile<false>, grid, dim3(64), p.lds, stream, in, w, out, a, f);
  } else if (norm_rope_wide_rows(s)) {
    const size_t lds = (size_t)(s.D + 31) / 32 * 32 * 4;
    if (s.norm)
      hipLaunchKernelGGL(norm_rope_wide<true>, dim3(s.rows), dim3(256), lds, stream, in, w, out,
                         a, f);
    else
      hipLaunchKernelGGL(norm_rope_wide<false>, dim3(s.rows), dim3(256), lds, stream, in, w,
                         out, a, f);
  } else {
    dim3 grid((s.rows + 255) / 256);
    if (s.norm)
      hipLaunchKernelGGL(norm_rope_rows<true>, grid, dim3(256), 0, stream, in, w, out, a, f);
    else
      hipLaunchKernelGGL(norm_rope_rows<false>, grid, dim3(256), 0, stream, in, w, out, a, f);
  }
  return hipGetLastError();
}

bool sigmoid_mul_vectorised(unsigned count, const void *g, const void *x, const void *o) {
  return count % 8 == 0 && aligned16(g) && aligned16(x) && aligned16(o);
}

hipError_t launch_sigmoid_mul(const uint16_t *gate, const uint16_t *in, uint16_t *out,
                              unsigned count, hipStream_t stream) {
  if (count == 0)
    return hipSuccess;
  if (sigmoid_mul_vectorised(count, gate, in, out)) {
    unsigned vectors = count / 8;
    hipLaunchKernelGGL(sigmoid_mul_vec, dim3((vectors + 255) / 256), dim3(256), 0, stream,
                       reinterpret_cast<const uint4_t *>(gate),
                       reinterpret_cast<const uint4_t *>(in),
                       reinterpret_cast<uint4_t *>(out), vectors);
  } else {
    hipLaunchKernelGGL(sigmoid_mul_scalar, dim3((count + 255) / 256), dim3(256), 0, stream,
                       gate, in, out, count);
  }
  return hipGetLastError();
}

} // namespace llmi
