// Gated delta rule, chunk-wise (WY / UT-transform) form: the DeltaNet
// prefill.
//
// Same result as the token recurrence of graphDeltaUpdate / updateDeltaColumn
// (Graph.metal:146-170, Reference.metal:182-197), which walks the tokens one
// by one. The published chunk algorithm (Yang, Kautz, Hatamizadeh, "Gated
// Delta Networks", arXiv:2412.06464; Yang et al., "Parallelizing Linear
// Transformers with the Delta Rule over Sequence Length", arXiv:2406.06484)
// splits the tokens into chunks of C = 64. With g the cumulative log decay
// inside a chunk, per chunk and value head:
//
//   A[t][s] = beta_t e^(g_t - g_s) k_t.k_s  (s < t),  T = (I + A)^-1
//   M[t][s] = e^(g_t - g_s) q_t.k_s        (s <= t)
//   X = diag(beta) V - diag(beta e^g) K S    U = T X
//   Y = diag(e^g) Q S + M U                  S <- e^(g_C) S + K^T diag(e^(g_C - g)) U
//
// Two launches:
//
//  * deltaChunkPrep, grid (chunk, key head): everything that does not depend
//    on the state, for every chunk at once -- the Gram matrices K K^T and
//    Q K^T on fp16 MFMA (v_mfma_f32_32x32x16_f16), then per value head the
//    decay weighting, M, and T by forward substitution in fp32 (one lane
//    per column of T). Written to the workspace, already split into the
//    hi/lo fp16 pairs the scan's products take: K and Q per (chunk, key
//    head); T, M and the token weights per (chunk, value head). The scan's
//    per-chunk staging is then plain 16-byte copies.
//
//  * deltaChunkScan, grid (value head, 32-column dv tile): walks the chunks
//    in order with the state tile S [dk x 32] resident in MFMA accumulators.
//    Every product that involves the state (K S, Q S, T X, M U, K^T Z) runs
//    on fp16 MFMA in a split form: x = hi + lo 2^-11 with hi = fp16(x),
//    lo = fp16((x - hi) 2^11), a.b ~ ah.bh + (ah.bl + al.bh) 2^-11, the
//    cross terms in a second fp32 accumulator -- 22 significant bits per
//    operand. A plain fp16 product leaves the fp32
//    state ~8e-4 relative off the recurrence after 1024 tokens; the split
//    form ~1e-5 (measured on the cfg4 shapes), well inside the 1e-3 bound.
//    The Gram matrices only feed T and M and stay plain fp16.
//
// Decays are linear at the op boundary (Graph.metal:143). The cumulative
// log decay is summed, and differenced, in double: log(0) is clamped to -1e4
// (e^-1e4 = 0), and in fp32 a difference of two sums near -1e4 would keep
// only ~1e-3 absolute precision. Only non-positive differences are
// exponentiated; the scan receives the weights e^(g_t) and e^(g_C - g_t)
// ready-made.
#include "hip_common.hpp"
#include "kernels.hpp"

#include "capi_internal.hpp"

#include <math.h>

namespace llmi {
namespace {

constexpr int C = 64;        // chunk length
constexpr int DK = 128;      // key dimension handled by these kernels
constexpr int DT = 32;       // dv columns per scan workgroup
constexpr int KST = DK + 8;  // fp16 stride of [token][dk] rows
constexpr int CST = C + 8;   // fp16 stride of [*][token] rows
constexpr int kMaxRatio = 4; // value heads per key head handled by one prep workgroup

// Workspace. Per (chunk, value head) a record of T and M as hi/lo fp16
// [C][C] each (Th, Tl, Mh, Ml), then per token e^(g_t), e^(g_C - g_t) and
// beta_t (fp32). After all records, per (chunk, key head): K and Q of the
// chunk as hi/lo fp16 [C][DK] (Kh, Kl, Qh, Ql; rows past T are zero).
constexpr size_t kRecHalves = 4 * C * C;
constexpr size_t kRecBytes = kRecHalves * 2 + 3 * C * 4;
constexpr size_t kRecEg = 0, kRecEz = C, kRecBeta = 2 * C; // floats after the halves
constexpr size_t kKQHalves = 4 * C * DK;

__device__ __forceinline__ half_t *rec_halves(void *ws, size_t c, size_t Hv, size_t h) {
  return reinterpret_cast<half_t *>(static_cast<char *>(ws) + (c * Hv + h) * kRecBytes);
}
__device__ __forceinline__ float *rec_weights(void *ws, size_t c, size_t Hv, size_t h) {
  return reinterpret_cast<float *>(rec_halves(ws, c, Hv, h) + kRecHalves);
}
__device__ __forceinline__ half_t *kq_halves(void *ws, size_t chunks, size_t Hv, size_t c,
                                             size_t Hk, size_t kh) {
  return reinterpret_cast<half_t *>(static_cast<char *>(ws) + chunks * Hv * kRecBytes) +
         (c * Hk + kh) * kKQHalves;
}

// Split four floats into hi/lo fp16.
__device__ __forceinline__ void split4(float4_t x, half4_t &hi, half4_t &lo) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    half_t a, b;
    split_f16(x[e], a, b);
    hi[e] = a;
    lo[e] = b;
  }
}

// --------------------------------------------------------------- prep

__global__ __launch_bounds__(256, 1) void delta_prep_kernel(
    const float *__restrict__ q, const float *__restrict__ k,
    const float *__restrict__ beta, const float *__restrict__ decay,
    void *__restrict__ ws, unsigned T, unsigned Hk, unsigned Hv) {
  const unsigned c = blockIdx.x, kh = blockIdx.y;
  const unsigned R = Hv / Hk, chunks = (T + C - 1) / C;
  const unsigned t0 = c * C, n = min((unsigned)C, T - t0);
  const unsigned tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const unsigned r = lane & 31u, hh = lane >> 5;

  __shared__ __attribute__((aligned(16))) half_t sK[C * KST], sQ[C * KST];
  __shared__ __attribute__((aligned(16))) float sKK[C * C], sQK[C * C];
  __shared__ __attribute__((aligned(16))) float sA[kMaxRatio][C * C];
  __shared__ double sG[kMaxRatio][C];
  __shared__ float sB[kMaxRatio][C];

  // Keys and queries of the chunk as fp16 (rows past the end are zero):
  // the hi halves to LDS for the Gram matrices, hi and lo to the workspace
  // for the scan.
  half_t *kq = kq_halves(ws, chunks, Hv, c, Hk, kh);
  for (unsigned i = tid; i < C * DK / 4; i += 256) {
    const unsigned t = i / (DK / 4), d4 = (i % (DK / 4)) * 4;
    float4_t kv{0.0f, 0.0f, 0.0f, 0.0f}, qv{0.0f, 0.0f, 0.0f, 0.0f};
    if (t < n) {
      const size_t off = ((size_t)(t0 + t) * Hk + kh) * DK + d4;
      kv = *reinterpret_cast<const float4_t *>(k + off);
      qv = *reinterpret_cast<const float4_t *>(q + off);
    }
    half4_t khi, klo, qhi, qlo;
    split4(kv, khi, klo);
    split4(qv, qhi, qlo);
    *reinterpret_cast<half4_t *>(sK + t * KST + d4) = khi;
    *reinterpret_cast<half4_t *>(sQ + t * KST + d4) = qhi;
    *reinterpret_cast<half4_t *>(kq + 4 * i) = khi;
    *reinterpret_cast<half4_t *>(kq + C * DK + 4 * i) = klo;
    *reinterpret_cast<half4_t *>(kq + 2 * C * DK + 4 * i) = qhi;
    *reinterpret_cast<half4_t *>(kq + 3 * C * DK + 4 * i) = qlo;
  }
  // Cumulative log decay (double) and beta of each value head of this key
  // head: wave w scans head w (padding tokens: decay 1, beta 0).
  if (wave < R) {
    const unsigned h = kh * R + wave, t = lane;
    const float a = t < n ? decay[(size_t)(t0 + t) * Hv + h] : 1.0f;
    const float b = t < n ? beta[(size_t)(t0 + t) * Hv + h] : 0.0f;
    double g = a > 0.0f ? (double)logf(a) : -1.0e4;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const double up = __shfl_up(g, off);
      if (lane >= (unsigned)off)
        g += up;
    }
    sG[wave][t] = g;
    sB[wave][t] = b;
  }
  __syncthreads();

  // K K^T and Q K^T, four 32x32 tiles each; wave w takes tiles w and w + 4.
#pragma unroll
  for (int rep = 0; rep < 2; ++rep) {
    const int tile = wave + 4 * rep;
    const half_t *a = tile < 4 ? sK : sQ;
    const int mt = (tile % 4) / 2, nt = tile % 2;
    float16_t acc = float16_t{0};
#pragma unroll
    for (int ks = 0; ks < DK / 16; ++ks)
      acc = mfma32x32x16(load8(a + (32 * mt + r) * KST + 16 * ks + 8 * hh),
                         load8(sK + (32 * nt + r) * KST + 16 * ks + 8 * hh), acc);
    float *dst = tile < 4 ? sKK : sQK;
#pragma unroll
    for (int v = 0; v < 16; ++v)
      dst[(32 * mt + mfma_c_row(v, hh)) * C + 32 * nt + r] = acc[v];
  }
  __syncthreads();

  // Decay weighting. Thread (row group tq, column s) covers rows tq + 4i:
  // A (to LDS), M (hi/lo), e^(g_t), e^(g_C - g_t), beta (to the workspace).
  {
    const unsigned s = tid % C, tq = tid / C;
    for (unsigned hr = 0; hr < R; ++hr) {
      half_t *rh = rec_halves(ws, c, Hv, kh * R + hr);
      float *rw = rec_weights(ws, c, Hv, kh * R + hr);
      const double gs = sG[hr][s];
#pragma unroll
      for (int i = 0; i < C / 4; ++i) {
        const unsigned t = tq + 4 * i, idx = t * C + s;
        const float e = s <= t ? expf((float)(sG[hr][t] - gs)) : 0.0f;
        sA[hr][idx] = s < t ? sB[hr][t] * e * sKK[idx] : 0.0f;
        split_f16(e * sQK[idx], rh[2 * C * C + idx], rh[3 * C * C + idx]);
      }
      if (tid < C) {
        rw[kRecEg + tid] = expf((float)sG[hr][tid]);
        rw[kRecEz + tid] = expf((float)(sG[hr][C - 1] - sG[hr][tid]));
        rw[kRecBeta + tid] = sB[hr][tid];
      }
    }
  }
  __syncthreads();

  // T = (I + A)^-1 by forward substitution: lane j of wave w owns column j
  // of value head w's T, T[t][j] = delta_tj - sum_{s<t} A[t][s] T[s][j].
  if (wave < R) {
    const float *A = sA[wave];
    const unsigned j = lane;
    float col[C];
#pragma unroll
    for (int t = 0; t < C; ++t) {
      float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int u = 0; u < t; ++u)
        acc[u & 3] = fmaf(A[t * C + u], col[u], acc[u & 3]);
      const float sum = (acc[0] + acc[1]) + (acc[2] + acc[3]);
      col[t] = (unsigned)t == j ? 1.0f : ((unsigned)t > j ? -sum : 0.0f);
    }
    half_t *rh = rec_halves(ws, c, Hv, kh * R + wave);
#pragma unroll
    for (int t = 0; t < C; ++t)
      split_f16(col[t], rh[t * C + j], rh[C * C + t * C + j]);
  }
}

// --------------------------------------------------------------- scan

// Split a float4 into hi/lo fp16 and store them at hi/lo (4 halves each).
__device__ __forceinline__ void store_split4(half_t *hi, half_t *lo, float4_t x) {
  half4_t h, l;
  split4(x, h, l);
  *reinterpret_cast<half4_t *>(hi) = h;
  *reinterpret_cast<half4_t *>(lo) = l;
}

// ds_read_b64_tr_b16: in each 16-lane group, lane j receives element j % 4 of
// the 8-byte chunks addressed by lanes j/4, 4 + j/4, 8 + j/4, 12 + j/4.
__device__ __forceinline__ half4_t read_tr(const half_t *base, unsigned byteOff) {
  typedef __attribute__((address_space(3))) char lds_char_t;
  typedef __fp16 fp16x4_t __attribute__((__vector_size__(4 * sizeof(__fp16))));
  return __builtin_bit_cast(
      half4_t, __builtin_amdgcn_ds_read_tr16_b64_v4f16(
                   (__attribute__((address_space(3))) fp16x4_t *)((lds_char_t *)base + byteOff)));
}

// One 32x32x16 step of a split product: acc += ah.bh and
// cross += ah.bl + al.bh (the scaled remainders; the lo.lo term is dropped).
struct SplitAcc {
  float16_t acc, cross;
};
__device__ __forceinline__ void mfma_split(const half_t *ah, const half_t *al,
                                           const half_t *bh, const half_t *bl,
                                           SplitAcc &p) {
  const half8_t a = load8(ah), b = load8(bh);
  p.acc = mfma32x32x16(a, b, p.acc);
  p.cross = mfma32x32x16(a, load8(bl), p.cross);
  p.cross = mfma32x32x16(load8(al), b, p.cross);
}
__device__ __forceinline__ void mfma_split_a(half8_t ah, half8_t al, const half_t *bh,
                                             const half_t *bl, SplitAcc &p) {
  const half8_t b = load8(bh);
  p.acc = mfma32x32x16(ah, b, p.acc);
  p.cross = mfma32x32x16(ah, load8(bl), p.cross);
  p.cross = mfma32x32x16(al, b, p.cross);
}
__device__ __forceinline__ float split_value(const SplitAcc &p, int v) {
  return p.acc[v] + p.cross[v] * kSplitUnscale;
}

// Write a C-layout 32x32 tile transposed, as hi/lo fp16, to dst[col][row]
// (row stride `stride` halves): lane (r, h) holds column r and rows
// 8q + 4h + [0, 4) of register group q, i.e. four consecutive rows.
__device__ __forceinline__ void store_tile_T(half_t *dh, half_t *dl, int stride,
                                             int row0, unsigned r, unsigned hh,
                                             const float (&x)[16]) {
#pragma unroll
  for (int qd = 0; qd < 4; ++qd) {
    const int row = row0 + 8 * qd + 4 * (int)hh;
    store_split4(dh + r * stride + row, dl + r * stride + row,
                 float4_t{x[4 * qd], x[4 * qd + 1], x[4 * qd + 2], x[4 * qd + 3]});
  }
}

// One chunk's scan inputs as this thread loads them: its share of the
// pre-split K, Q (8 halves of a token row each), T and M, of the V tile,
// and (threads < C) the token weights. Loaded one chunk ahead so that the
// global latency hides behind the previous chunk's products.
constexpr int kKQPer = C * DK / 8 / 256; // half8s of each of Kh, Kl, Qh, Ql per thread
constexpr int kTMPer = C * C / 8 / 256;  // half8s of each of Th, Tl, Mh, Ml per thread
struct ChunkRegs {
  half8_t kq[4][kKQPer], tm[4][kTMPer];
  half8_t v;
  float eg, ez, b;
};

__device__ __forceinline__ void load_chunk(ChunkRegs &cr, const half_t *__restrict__ kq,
                                           const half_t *__restrict__ rec,
                                           const half_t *__restrict__ v, unsigned t0,
                                           unsigned n, size_t vcol, size_t vwidth,
                                           unsigned tid) {
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int it = 0; it < kKQPer; ++it)
      cr.kq[a][it] = load8(kq + a * C * DK + 8 * (tid + 256 * it));
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int it = 0; it < kTMPer; ++it)
      cr.tm[a][it] = load8(rec + a * C * C + 8 * (tid + 256 * it));
  const unsigned t = tid / (DT / 8), jj = (tid % (DT / 8)) * 8;
  cr.v = half8_t{0, 0, 0, 0, 0, 0, 0, 0};
  if (t < n)
    cr.v = load8(v + (size_t)(t0 + t) * vwidth + vcol + jj);
  if (tid < C) {
    const float *w = reinterpret_cast<const float *>(rec + kRecHalves);
    cr.eg = w[kRecEg + tid];
    cr.ez = w[kRecEz + tid];
    cr.b = w[kRecBeta + tid];
  }
}

__global__ __launch_bounds__(256, 1) void delta_scan_kernel(
    const half_t *__restrict__ v, float *__restrict__ state, half_t *__restrict__ out,
    void *__restrict__ ws, unsigned T, unsigned Hk, unsigned Hv, unsigned DV) {
  // Workgroups are dealt to the 8 XCDs round-robin by block index. Order
  // the (value head, column tile) pairs key head by key head and give each
  // XCD a contiguous run of them, so that the workgroups reading one key
  // head's K and Q share an L2 (exactly so when Hk is a multiple of 8).
  const unsigned tilesPerHead = DV / DT;
  const unsigned nblocks = gridDim.x;
  const unsigned L = nblocks % 8 == 0 ? (blockIdx.x % 8) * (nblocks / 8) + blockIdx.x / 8
                                      : blockIdx.x;
  const unsigned h = L / tilesPerHead, jt = L % tilesPerHead;
  const unsigned kh = h / (Hv / Hk), j0 = jt * DT;
  const unsigned tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const unsigned r = lane & 31u, hh = lane >> 5;
  const unsigned chunks = (T + C - 1) / C;
  const size_t vwidth = (size_t)Hv * DV;

  // K and Q token-major, T, M, the state transposed S^T [j][d], X^T (later
  // Z^T) and U^T, all hi/lo.
  __shared__ __attribute__((aligned(16))) half_t sKh[C * KST], sKl[C * KST];
  __shared__ __attribute__((aligned(16))) half_t sQh[C * KST], sQl[C * KST];
  __shared__ __attribute__((aligned(16))) half_t sTh[C * CST], sTl[C * CST];
  __shared__ __attribute__((aligned(16))) half_t sMh[C * CST], sMl[C * CST];
  __shared__ __attribute__((aligned(16))) half_t sSh[DT * KST], sSl[DT * KST];
  __shared__ __attribute__((aligned(16))) half_t sXh[DT * CST], sXl[DT * CST];
  __shared__ __attribute__((aligned(16))) half_t sUh[DT * CST], sUl[DT * CST];
  __shared__ float sV[C * DT];
  __shared__ float sEg[C], sEz[C], sB[C];

  // The state tile: wave w holds rows d in [32w, 32w + 32), column r.
  float S[16];
  float *stile = state + (size_t)h * DK * DV + j0 + r;
#pragma unroll
  for (int x = 0; x < 16; ++x)
    S[x] = stile[(size_t)(32 * wave + mfma_c_row(x, hh)) * DV];
  store_tile_T(sSh, sSl, KST, 32 * wave, r, hh, S);

  const size_t vcol = (size_t)h * DV + j0;
  auto kq_of = [&](unsigned c) { return kq_halves(ws, chunks, Hv, c, Hk, kh); };
  auto rec_of = [&](unsigned c) { return rec_halves(ws, c, Hv, h); };
  ChunkRegs cr;
  load_chunk(cr, kq_of(0), rec_of(0), v, 0, min((unsigned)C, T), vcol, vwidth, tid);

  for (unsigned c = 0; c < chunks; ++c) {
    const unsigned t0 = c * C, n = min((unsigned)C, T - t0);

    // 1. Stage the chunk from registers: K, Q, T, M (hi/lo); V; weights.
#pragma unroll
    for (int it = 0; it < kKQPer; ++it) {
      const unsigned i = tid + 256 * it, t = i / (DK / 8), d8 = (i % (DK / 8)) * 8;
      half_t *const dst[4] = {sKh, sKl, sQh, sQl};
#pragma unroll
      for (int a = 0; a < 4; ++a)
        *reinterpret_cast<half8_t *>(dst[a] + t * KST + d8) = cr.kq[a][it];
    }
#pragma unroll
    for (int it = 0; it < kTMPer; ++it) {
      const unsigned i = tid + 256 * it, t = i / (C / 8), s8 = (i % (C / 8)) * 8;
      half_t *const dst[4] = {sTh, sTl, sMh, sMl};
#pragma unroll
      for (int a = 0; a < 4; ++a)
        *reinterpret_cast<half8_t *>(dst[a] + t * CST + s8) = cr.tm[a][it];
    }
    {
      const unsigned t = tid / (DT / 8), jj = (tid % (DT / 8)) * 8;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        sV[t * DT + jj + e] = (float)cr.v[e];
    }
    if (tid < C) {
      sEg[tid] = cr.eg;
      sEz[tid] = cr.ez;
      sB[tid] = cr.b;
    }
    __syncthreads();

    // 2. Waves 0-1: K S, waves 2-3: Q S (row tile mt of the chunk). The
    //    per-token scalars of this lane's 16 rows are read first, so their
    //    LDS latency hides behind the products.
    const int mt = wave & 1;
    float tEg[16], tB[16], tV[16];
#pragma unroll
    for (int x = 0; x < 16; ++x) {
      const int t = 32 * mt + mfma_c_row(x, hh);
      tEg[x] = sEg[t];
      if (wave < 2) {
        tB[x] = sB[t];
        tV[x] = sV[t * DT + r];
      }
    }
    float16_t acc;
    {
      SplitAcc p{float16_t{0}, float16_t{0}};
      const half_t *ah = wave < 2 ? sKh : sQh, *al = wave < 2 ? sKl : sQl;
#pragma unroll
      for (int ks = 0; ks < DK / 16; ++ks) {
        const int ko = 16 * ks + 8 * hh;
        mfma_split(ah + (32 * mt + r) * KST + ko, al + (32 * mt + r) * KST + ko,
                   sSh + r * KST + ko, sSl + r * KST + ko, p);
      }
#pragma unroll
      for (int x = 0; x < 16; ++x)
        acc[x] = split_value(p, x);
    }
    // 3. X = beta (V - e^g K S) -> X^T; Q S -> e^g Q S (kept in acc).
    float x16[16];
#pragma unroll
    for (int x = 0; x < 16; ++x) {
      if (wave < 2)
        x16[x] = tB[x] * (tV[x] - tEg[x] * acc[x]);
      else
        acc[x] *= tEg[x];
    }
    if (wave < 2)
      store_tile_T(sXh, sXl, CST, 32 * mt, r, hh, x16);
    __syncthreads();

    // 4. Fetch the next chunk while this one finishes.
    if (c + 1 < chunks)
      load_chunk(cr, kq_of(c + 1), rec_of(c + 1), v, t0 + C, min((unsigned)C, T - t0 - C),
                 vcol, vwidth, tid);
    // 5. Waves 0-1: U = T X.
    float u[16];
    if (wave < 2) {
      SplitAcc p{float16_t{0}, float16_t{0}};
#pragma unroll
      for (int ks = 0; ks < C / 16; ++ks) {
        const int ko = 16 * ks + 8 * hh;
        mfma_split(sTh + (32 * mt + r) * CST + ko, sTl + (32 * mt + r) * CST + ko,
                   sXh + r * CST + ko, sXl + r * CST + ko, p);
      }
#pragma unroll
      for (int x = 0; x < 16; ++x)
        u[x] = split_value(p, x);
    }
    __syncthreads();
    // 6. U^T, and Z^T = (e^(g_C - g) U)^T into X's space.
    if (wave < 2) {
      float zz[16];
#pragma unroll
      for (int x = 0; x < 16; ++x) {
        const int t = 32 * mt + mfma_c_row(x, hh);
        zz[x] = sEz[t] * u[x];
      }
      store_tile_T(sUh, sUl, CST, 32 * mt, r, hh, u);
      store_tile_T(sXh, sXl, CST, 32 * mt, r, hh, zz);
    }
    __syncthreads();

    // 7. Waves 2-3: Y = e^g Q S + M U -> out.
    if (wave >= 2) {
      SplitAcc p{acc, float16_t{0}};
#pragma unroll
      for (int ks = 0; ks < C / 16; ++ks) {
        const int ko = 16 * ks + 8 * hh;
        mfma_split(sMh + (32 * mt + r) * CST + ko, sMl + (32 * mt + r) * CST + ko,
                   sUh + r * CST + ko, sUl + r * CST + ko, p);
      }
#pragma unroll
      for (int x = 0; x < 16; ++x) {
        const unsigned t = 32 * mt + mfma_c_row(x, hh);
        if (t < n)
          out[(size_t)(t0 + t) * vwidth + (size_t)h * DV + j0 + r] =
              (half_t)split_value(p, x);
      }
    }
    // 8. S <- e^(g_C) S + K^T Z (wave w: rows d in [32w, 32w + 32)). The
    //    K^T operand (channel d, tokens 16 ks + 8 hh .. +8) comes from the
    //    token-major K tile through transposing reads: lane L of a 16-lane
    //    group addresses token row ko + L/4 (+ 4), channels d0 + 4 (L%4),
    //    and receives 4 tokens of channel d0 + L.
    {
      const float eC = sEg[C - 1];
      SplitAcc p{float16_t{0}, float16_t{0}};
#pragma unroll
      for (int x = 0; x < 16; ++x)
        p.acc[x] = S[x] * eC;
      const unsigned L = lane % 16;
      const unsigned d0 = 32 * wave + 16 * ((lane % 32) / 16);
#pragma unroll
      for (int ks = 0; ks < C / 16; ++ks) {
        const unsigned ko = 16 * ks + 8 * hh;
        const unsigned off = ((ko + L / 4) * KST + d0 + 4 * (L % 4)) * 2;
        const half4_t h0 = read_tr(sKh, off), h1 = read_tr(sKh, off + 4 * KST * 2);
        const half4_t l0 = read_tr(sKl, off), l1 = read_tr(sKl, off + 4 * KST * 2);
        const half8_t ah{h0[0], h0[1], h0[2], h0[3], h1[0], h1[1], h1[2], h1[3]};
        const half8_t al{l0[0], l0[1], l0[2], l0[3], l1[0], l1[1], l1[2], l1[3]};
        mfma_split_a(ah, al, sXh + r * CST + ko, sXl + r * CST + ko, p);
      }
#pragma unroll
      for (int x = 0; x < 16; ++x)
        S[x] = split_value(p, x);
    }
    // 9. S^T for the next chunk (nothing reads S^T after step 2).
    store_tile_T(sSh, sSl, KST, 32 * wave, r, hh, S);
    __syncthreads();
  }

#pragma unroll
  for (int x = 0; x < 16; ++x)
    stile[(size_t)(32 * wave + mfma_c_row(x, hh)) * DV] = S[x];
}

} // namespace

bool delta_chunked_supported(const DeltaShape &s) {
  return s.Dk == DK && s.Dv % DT == 0 && s.Hk >= 1 && s.Hv % s.Hk == 0 &&
         s.Hv / s.Hk <= (unsigned)kMaxRatio && s.T >= 32;
}

size_t delta_chunked_workspace_bytes(const DeltaShape &s) {
  const size_t chunks = (s.T + C - 1) / C;
  return chunks * s.Hv * kRecBytes + chunks * s.Hk * kKQHalves * sizeof(half_t);
}

hipError_t launch_delta_chunked(const float *q, const float *k, const uint16_t *v,
                                const float *beta, const float *decay, float *state,
                                uint16_t *out, void *ws, const DeltaShape &s,
                                hipStream_t stream) {
  const unsigned chunks = (s.T + C - 1) / C;
  hipLaunchKernelGGL(delta_prep_kernel, dim3(chunks, s.Hk), dim3(256), 0, stream, q, k,
                     beta, decay, ws, s.T, s.Hk, s.Hv);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return e;
  hipLaunchKernelGGL(delta_scan_kernel, dim3(s.Hv * (s.Dv / DT)), dim3(256), 0, stream,
                     reinterpret_cast<const half_t *>(v), state,
                     reinterpret_cast<half_t *>(out), ws, s.T, s.Hk, s.Hv, s.Dv);
  return hipGetLastError();
}

unsigned delta_chunked_dispatches() { return 2; }

const char *delta_chunked_kernel_name(unsigned index) {
  return index == 0 ? "deltaChunkPrep" : "deltaChunkScan";
}

} // namespace llmi
