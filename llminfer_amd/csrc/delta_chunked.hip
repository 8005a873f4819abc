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
//   U = T diag(beta) (V - diag(e^g) K S)
//   Y = diag(e^g) Q S + M U                  S <- e^(g_C) S + K^T diag(e^(g_C - g)) U
//
// Everything that does not involve the state S is moved out of the serial
// chain over the chunks. With W = T diag(beta e^g) K and U0 = T diag(beta) V:
//
//   Z  = diag(e^(g_C - g)) U = Z0 + Wn S      Wn = -diag(e^(g_C - g)) W
//                                             Z0 = diag(e^(g_C - g)) U0
//   Y  = Y0 + Q' S                            Q' = diag(e^g) Q - (M T diag(beta e^g)) K
//                                             Y0 = M U0
//   S <- e^(g_C) S + K^T Z
//
// so that a chunk costs the serial chain only two products (Wn S, then
// K^T Z) plus Q' S beside them.
//
// Two launches:
//
//  * deltaChunkPrep, grid (chunk, key head), 256 threads: every chunk at
//    once. The Gram matrices K K^T and Q K^T on fp16 MFMA (kept in
//    registers); per value head the decay weighting, T by blocked
//    substitution (diagonal blocks in fp32, off-diagonal blocks on MFMA), and
//    the products Wn, Q', Z0, Y0 on fp16 MFMA in split form. The results go to
//    the workspace already in the register order of the scan's MFMA operands.
//
//  * deltaChunkScan, grid (value head, 16-column dv slice), 4 compute waves
//    and an L2-warming wave. Wave w keeps rows [32 w, 32 w + 32) of the
//    state slice S [dk x 16] in registers and computes token tile w of each
//    chunk's Z and Y; S and Z pass between the waves through LDS, two
//    barriers per chunk. Every product runs on v_mfma_f32_16x16x32_f16,
//    with the state (and Z) as the B operand straight from the C-layout
//    registers of the product that made it: the k index of an operand block
//    is permuted (sigma below) so that the 8 halves a lane supplies are the
//    8 rows it holds in two consecutive 16-row C tiles; the A operands (Wn,
//    Q', K^T) were written by the prep with the same permutation. Each wave
//    loads its own operand blocks one chunk ahead into registers.
//
// Split form: x = hi + lo 2^-11 with hi = fp16(x), lo = fp16((x - hi) 2^11),
// a.b ~ ah.bh + (ah.bl + al.bh) 2^-11, the cross terms in a second fp32
// accumulator -- 22 significant bits per operand. A plain fp16 product
// leaves the fp32 state ~8e-4 relative off the recurrence after 1024 tokens;
// the split form ~1e-5, well inside the 1e-3 bound. The Gram matrices are
// split too: in plain fp16 they leave the outputs of small-RMS rows a few
// percent off (relative to the row), which the gated norm after the update
// turns into errors of a few output ulps.
//
// Decays are linear at the op boundary (Graph.metal:143). The cumulative
// log decay is summed, and differenced, in double: log(0) is clamped to -1e4
// (e^-1e4 = 0), and in fp32 a difference of two sums near -1e4 would keep
// only ~1e-3 absolute precision. Only non-positive differences are
// exponentiated.
#include "exact_fp.hpp"
#include "gated_norm.hpp"
#include "hip_common.hpp"
#include "kernels.hpp"

#include "capi_internal.hpp"

#include <math.h>

#include <vector>

namespace llmi {
namespace {

constexpr int C = 64;       // chunk length
constexpr int DK = 128;     // key dimension handled by these kernels
constexpr int KS = DK + 8;  // fp16 stride of [token][dk] rows in LDS (and of V rows)
constexpr int CS = C + 8;   // fp16 stride of [*][token] rows in LDS
constexpr int FS = C + 1;   // fp32 stride of the prep's A and T^T rows
constexpr int VB = 128;     // dv columns of V the prep stages at a time

// MFMA operand blocks (v_mfma_f32_16x16x32_f16) in register order: lane l
// holds 8 halves at halves [8 l, 8 l + 8) of the block.
//
// Permuted k: in a 32-wide k block, element e of lane l (g = l / 16) stands
// for k = sigma(g, e) = 4g + e (e < 4) or 16 + 4g + (e - 4) (e >= 4) -- the
// rows a lane holds in the C layout of the two 16-row tiles of that block
// (register r of tile m holds row 16m + 4g + r). A product whose k is
// permuted the same way in both operands is unchanged.
//
// A piece is the operand of one scan product for one chunk: 16 blocks of hi
// halves, then 16 blocks of lo halves. Wn and Q' pieces: block 4m + kb
// holds rows t of tile m against permuted k = d in block kb. K^T piece:
// block 2i + kb holds rows d of tile i against permuted k = t in block kb.
constexpr int kBlk = 64 * 8;
constexpr int kPieceBlocks = 16;
constexpr int kPieceHalves = 2 * kPieceBlocks * kBlk;
constexpr int kPieceBytes = kPieceHalves * 2;      // 32 KiB
constexpr int kBufferWord3 = 0x00020000;           // gfx9 raw buffer descriptor, dword 3
typedef __attribute__((address_space(3))) void lds_void_t;

// Workspace. Per (chunk, value head) a record: the Wn piece (hi and lo),
// the Q' piece (plain fp16: the 16 hi blocks only, Q' feeds the outputs
// alone), then Z0 and Y0 as fp32 in C-layout register order, per 16-column
// slice js and 16-row tile m a 64-lane block of float4 (block 4 js + m),
// then 64 floats of scalars (e^(g_C) first). After all records, per (chunk,
// key head) the K^T piece.
constexpr int kScalarBytes = 256;
constexpr int kQPieceBytes = kPieceBlocks * kBlk * 2; // 16 KiB
__host__ __device__ inline size_t rec_z0(unsigned) {
  return (size_t)kPieceBytes + kQPieceBytes;
}
__host__ __device__ inline size_t rec_scalars(unsigned DV) {
  return rec_z0(DV) + 2 * (size_t)C * DV * sizeof(float);
}
__host__ __device__ inline size_t rec_bytes(unsigned DV) {
  return rec_scalars(DV) + kScalarBytes;
}
__device__ __forceinline__ char *rec_ptr(void *ws, size_t recB, size_t Hv, size_t c,
                                         size_t h) {
  return static_cast<char *>(ws) + (c * Hv + h) * recB;
}
__device__ __forceinline__ char *kpiece_ptr(void *ws, size_t recB, size_t chunks, size_t Hv,
                                            size_t Hk, size_t c, size_t kh) {
  return static_cast<char *>(ws) + chunks * Hv * recB + (c * Hk + kh) * kPieceBytes;
}

__device__ __forceinline__ float4_t mfma16(half8_t a, half8_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
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

// B operand (or permuted-k A operand) of one 32-wide k block from two
// C-layout tiles: elements 0-3 from `a`, 4-7 from `b`, split hi/lo.
__device__ __forceinline__ void split8(float4_t a, float4_t b, half8_t &hi, half8_t &lo) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    half_t x, y;
    split_f16(a[e], x, y);
    hi[e] = x;
    lo[e] = y;
    split_f16(b[e], x, y);
    hi[4 + e] = x;
    lo[4 + e] = y;
  }
}

__device__ __forceinline__ half8_t cat8(half4_t a, half4_t b) {
  return half8_t{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}
__device__ __forceinline__ half4_t load4(const half_t *p) {
  return *reinterpret_cast<const half4_t *>(p);
}

// ds_read_b64_tr_b16: in each 16-lane group, lane L addresses the 8 bytes at
// row r0 + L/4, columns c0 + 4 (L%4) and receives the column c0 + L of rows
// r0 .. r0 + 3.
__device__ __forceinline__ half4_t read_tr(const half_t *base, unsigned byteOff) {
  typedef __attribute__((address_space(3))) char lds_char_t;
  typedef __fp16 fp16x4_t __attribute__((__vector_size__(4 * sizeof(__fp16))));
  return __builtin_bit_cast(
      half4_t, __builtin_amdgcn_ds_read_tr16_b64_v4f16(
                   (__attribute__((address_space(3))) fp16x4_t *)((lds_char_t *)base + byteOff)));
}

// Operand of 8 consecutive k for one row/column, from a row-major [k][x]
// LDS matrix with `stride` halves: lane (g, L) gets X[k0 + 8g + e][x0 + L].
__device__ __forceinline__ half8_t read_kcol(const half_t *X, int stride, unsigned k0,
                                             unsigned x0, unsigned g, unsigned L) {
  const unsigned off = ((k0 + 8 * g + L / 4) * stride + x0 + 4 * (L % 4)) * 2;
  return cat8(read_tr(X, off), read_tr(X, off + 4 * stride * 2));
}

// --------------------------------------------------------------- prep

__device__ __forceinline__ float4_t mfma16k16(half4_t a, half4_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}
// Four floats at p, p + stride, ... split into hi/lo fp16.
__device__ __forceinline__ void load_split4(const float *p, int stride, half4_t &hi,
                                            half4_t &lo) {
  split4(float4_t{p[0], p[stride], p[2 * stride], p[3 * stride]}, hi, lo);
}

// QK16: q and k arrive as fp16 rows and are L2-normalised here exactly as
// l2NormF32 (Graph.metal:96-109) would: one lane per (token, q or k) row of
// the chunk runs the reference's sequential sum of squares, and each fp32
// element is the single product x * factor -- the bits l2NormF32 writes.
template <bool QK16>
__global__ __launch_bounds__(256, 1) void delta_prep_kernel(
    const void *__restrict__ qp, const void *__restrict__ kp, const half_t *__restrict__ v,
    const float *__restrict__ beta, const float *__restrict__ decay, void *__restrict__ ws,
    unsigned T, unsigned Hk, unsigned Hv, unsigned DV, float eps, float qscale, unsigned *cnt) {
  const float *q = static_cast<const float *>(qp), *k = static_cast<const float *>(kp);
  const half_t *q16 = static_cast<const half_t *>(qp), *k16 = static_cast<const half_t *>(kp);
  const unsigned c = blockIdx.x, kh = blockIdx.y;
  const unsigned R = Hv / Hk, chunks = (T + C - 1) / C;
  const unsigned t0 = c * C, n = min((unsigned)C, T - t0);
  const unsigned tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const unsigned g = lane >> 4, L = lane & 15u;
  const size_t recB = rec_bytes(DV);
  const size_t qkStride = (size_t)Hk * DK, vStride = (size_t)Hv * DV;
  // The fused norm's per-value-head arrival records (4 words each), zeroed
  // here (the scan runs after this launch on the same stream).
  if (cnt && c == 0 && tid < 4 * R)
    cnt[4 * kh * R + tid] = 0;

  __shared__ __attribute__((aligned(16))) half_t sKh[C * KS], sKl[C * KS];
  __shared__ __attribute__((aligned(16))) half_t sQV[C * KS]; // Q hi, later a V block
  // A and T^T (fp32); before them, during the Gram products, Q lo
  __shared__ __attribute__((aligned(16))) float sATT[2 * C * FS];
  float *const sA = sATT, *const sTT = sATT + C * FS;
  half_t *const sQl = reinterpret_cast<half_t *>(sATT);
  static_assert(C * KS * sizeof(half_t) <= 2 * C * FS * sizeof(float), "Q lo fits");
  __shared__ __attribute__((aligned(16))) half_t sTwh[C * CS], sTwl[C * CS];
  __shared__ __attribute__((aligned(16))) half_t sTbh[C * CS], sTbl[C * CS];
  __shared__ __attribute__((aligned(16))) half_t sMh[C * CS], sMl[C * CS];
  __shared__ __attribute__((aligned(16))) half_t sNh[C * CS], sNl[C * CS];
  __shared__ double sG[C];
  __shared__ float sB[C], sEg[C], sEz[C];
  __shared__ float sFac[QK16 ? 2 * C : 1]; // QK16: L2 factors of the k rows, then the q rows

  // Loads that later phases need, issued up front so that their latency
  // hides behind the K/Q split and the Gram products: the fp32 queries of
  // the Q' initial values (wave w: d tiles 2w, 2w + 1, all t), the gates
  // of the first value head (wave 0) and its first block of V.
  float4_t qinit[2][4];
  half4_t qraw[2][4]; // QK16: the fp16 queries, normalised once the factors are known
#pragma unroll
  for (int hf = 0; hf < 2; ++hf)
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const unsigned t = 16 * mt + L, tc = min(t, n - 1); // rows past the end read row n-1
      const size_t off =
          (size_t)(t0 + tc) * qkStride + (size_t)kh * DK + 16 * (2 * wave + hf) + 4 * g;
      if constexpr (QK16) {
        qraw[hf][mt] = *reinterpret_cast<const half4_t *>(q16 + off);
      } else {
        const float4_t x = *reinterpret_cast<const float4_t *>(q + off);
        qinit[hf][mt] = t < n ? x : float4_t{0.0f, 0.0f, 0.0f, 0.0f};
      }
    }
  float gateA = 1.0f, gateB = 0.0f;
  auto load_gates = [&](unsigned h) {
    if (wave == 0 && lane < n) {
      gateA = decay[(size_t)(t0 + lane) * Hv + h];
      gateB = beta[(size_t)(t0 + lane) * Hv + h];
    }
  };
  load_gates(kh * R);
  // V rows of one head's dv block [jb, jb + w): thread tid holds items
  // tid + 256 i (8 halves each), w <= VB.
  constexpr int kVItems = C * VB / 8 / 256;
  half8_t vreg[kVItems];
  auto fetch_v = [&](unsigned h, unsigned jb, unsigned w) {
#pragma unroll
    for (int it = 0; it < kVItems; ++it) {
      const unsigned i = tid + 256 * it, t = i / (w / 8), j8 = (i % (w / 8)) * 8;
      const unsigned tc = min(t, n - 1); // rows past the end (or items past w) read row n-1
      const half8_t x =
          load8(v + (size_t)(t0 + tc) * vStride + (size_t)h * DV + jb + (i < C * w / 8 ? j8 : 0));
      vreg[it] = t < n ? x : half8_t{0, 0, 0, 0, 0, 0, 0, 0};
    }
  };
  auto store_v = [&](unsigned w) {
#pragma unroll
    for (int it = 0; it < kVItems; ++it) {
      const unsigned i = tid + 256 * it, t = i / (w / 8), j8 = (i % (w / 8)) * 8;
      if (i < C * w / 8)
        *reinterpret_cast<half8_t *>(sQV + t * KS + j8) = vreg[it];
    }
  };
  const unsigned w0 = min((unsigned)VB, DV);
  fetch_v(kh * R, 0, w0);

  // QK16: the L2 factors of the chunk's k rows (threads 0-63) and q rows
  // (64-127), each the sequential sum over one row.
  if constexpr (QK16) {
    if (tid < 2 * C) {
      const unsigned t = tid % C, isq = tid / C;
      const uint4_t *row = reinterpret_cast<const uint4_t *>(
          (isq ? q16 : k16) + (size_t)(t0 + min(t, n - 1)) * qkStride + (size_t)kh * DK);
      uint4_t x[DK / 8];
#pragma unroll
      for (int c8 = 0; c8 < DK / 8; ++c8)
        x[c8] = row[c8];
      float sum = 0.0f;
#pragma unroll
      for (int c8 = 0; c8 < DK / 8; ++c8)
        sum = sumsq8(x[c8], sum);
      sFac[tid] = l2_row_factor(sum, eps, isq ? qscale : 1.0f);
    }
    lds_sync();
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const unsigned t = 16 * mt + L;
        const float f = sFac[C + min(t, n - 1)];
        float4_t x;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          x[e] = __fmul_rn((float)qraw[hf][mt][e], f);
        qinit[hf][mt] = t < n ? x : float4_t{0.0f, 0.0f, 0.0f, 0.0f};
      }
  }

  // Keys and queries of the chunk as fp16 hi/lo (rows past the end are
  // zero); every load is issued before the first store.
  {
    constexpr int NI = C * DK / 4 / 256;
    float4_t kv[NI], qv[NI];
#pragma unroll
    for (int it = 0; it < NI; ++it) {
      const unsigned i = tid + 256 * it, t = i / (DK / 4), d4 = (i % (DK / 4)) * 4;
      const unsigned tc = min(t, n - 1);
      const size_t off = (size_t)(t0 + tc) * qkStride + (size_t)kh * DK + d4;
      if constexpr (QK16) {
        const half4_t kr = *reinterpret_cast<const half4_t *>(k16 + off);
        const half4_t qr = *reinterpret_cast<const half4_t *>(q16 + off);
        const float fk = sFac[tc], fq = sFac[C + tc];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          kv[it][e] = __fmul_rn((float)kr[e], fk);
          qv[it][e] = __fmul_rn((float)qr[e], fq);
        }
      } else {
        kv[it] = *reinterpret_cast<const float4_t *>(k + off);
        qv[it] = *reinterpret_cast<const float4_t *>(q + off);
      }
    }
#pragma unroll
    for (int it = 0; it < NI; ++it) {
      const unsigned i = tid + 256 * it, t = i / (DK / 4), d4 = (i % (DK / 4)) * 4;
      const float4_t zero{0.0f, 0.0f, 0.0f, 0.0f};
      half4_t khi, klo, qhi, qlo;
      split4(t < n ? kv[it] : zero, khi, klo);
      split4(t < n ? qv[it] : zero, qhi, qlo);
      *reinterpret_cast<half4_t *>(sKh + t * KS + d4) = khi;
      *reinterpret_cast<half4_t *>(sKl + t * KS + d4) = klo;
      *reinterpret_cast<half4_t *>(sQV + t * KS + d4) = qhi;
      *reinterpret_cast<half4_t *>(sQl + t * KS + d4) = qlo;
    }
  }
  lds_sync();

  // The K^T piece of this (chunk, key head): block b = 2i + kb, lane (g, L)
  // element e = K[32 kb + sigma(g, e)][16 i + L].
  {
    half_t *kp = reinterpret_cast<half_t *>(kpiece_ptr(ws, recB, chunks, Hv, Hk, c, kh));
#pragma unroll
    for (int bi = 0; bi < 4; ++bi) {
      const unsigned b = 4 * wave + bi, i = b / 2, kb = b % 2;
      const unsigned off0 = ((32 * kb + 4 * g + L / 4) * KS + 16 * i + 4 * (L % 4)) * 2;
      const unsigned off1 = off0 + 16 * KS * 2;
      *reinterpret_cast<half8_t *>(kp + b * kBlk + 8 * lane) =
          cat8(read_tr(sKh, off0), read_tr(sKh, off1));
      *reinterpret_cast<half8_t *>(kp + (kPieceBlocks + b) * kBlk + 8 * lane) =
          cat8(read_tr(sKl, off0), read_tr(sKl, off1));
    }
  }

  // K K^T and Q K^T stay in registers: wave w holds the tiles of key
  // columns s in [16 w, 16 w + 16) for the four row tiles (register r of
  // tile mt: t = 16 mt + 4 g + r, s = 16 w + L). Split form: both feed M,
  // and through M the outputs Y0 = M U0 and Q', where a row's output is
  // often much smaller than the terms that cancel in it, so a plain fp16
  // product (2^-11 relative per term) would show in rows of small RMS.
  float4_t kk[4], qk[4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    float4_t kx{0.0f, 0.0f, 0.0f, 0.0f}, qx{0.0f, 0.0f, 0.0f, 0.0f};
    kk[mt] = qk[mt] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int ks = 0; ks < DK / 32; ++ks) {
      const unsigned bo = (16 * wave + L) * KS + 32 * ks + 8 * g;
      const unsigned ao = (16 * mt + L) * KS + 32 * ks + 8 * g;
      const half8_t bh = load8(sKh + bo), bl = load8(sKl + bo);
      const half8_t kah = load8(sKh + ao), kal = load8(sKl + ao);
      const half8_t qah = load8(sQV + ao), qal = load8(sQl + ao);
      kk[mt] = mfma16(kah, bh, kk[mt]);
      qk[mt] = mfma16(qah, bh, qk[mt]);
      kx = mfma16(kah, bl, kx);
      qx = mfma16(qah, bl, qx);
      kx = mfma16(kal, bh, kx);
      qx = mfma16(qal, bh, qx);
    }
    kk[mt] += kx * kSplitUnscale;
    qk[mt] += qx * kSplitUnscale;
  }

  for (unsigned hr = 0; hr < R; ++hr) {
    const unsigned h = kh * R + hr;
    char *const rec = rec_ptr(ws, recB, Hv, c, h);
    lds_sync(); // the previous head is done with every LDS buffer

    // Cumulative log decay (double) and beta (padding tokens: decay 1,
    // beta 0), e^(g_t), e^(g_C - g_t) and e^(g_C); V of the head's first
    // dv block.
    if (wave == 0) {
      const unsigned t = lane;
      const float a = gateA, b = gateB;
      double gg = a > 0.0f ? (double)logf(a) : -1.0e4;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const double up = __shfl_up(gg, off);
        if (lane >= (unsigned)off)
          gg += up;
      }
      const double gC = __shfl(gg, 63);
      sG[t] = gg;
      sB[t] = b;
      sEg[t] = expf((float)gg);
      sEz[t] = expf((float)(gC - gg));
      if (t == 63)
        *reinterpret_cast<float *>(rec + rec_scalars(DV)) = expf((float)gg);
    }
    store_v(w0);
    // The next head's gates and first V block, in flight during this head
    // (with DV > VB the V registers carry this head's further blocks, and
    // the next head's first block is fetched after them).
    if (hr + 1 < R) {
      load_gates(h + 1);
      if (DV <= VB)
        fetch_v(h + 1, 0, w0);
    }
    lds_sync();

    // A (fp32) and M (hi/lo) from the Gram registers:
    // A[t][s] = beta_t e^(g_t - g_s) k_t.k_s (s < t), M[t][s] = e^(g_t - g_s)
    // q_t.k_s (s <= t), zero above.
    // Branch-free: every operand is read, the masks are selects.
    {
      const unsigned s = 16 * wave + L;
      const double gs = sG[s];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const unsigned t = 16 * mt + 4 * g + r;
          const float d = fminf((float)(sG[t] - gs), 0.0f);
          const float e = s <= t ? __builtin_amdgcn_exp2f(d * kLog2e) : 0.0f;
          const float a = sB[t] * e * kk[mt][r];
          sA[t * FS + s] = s < t ? a : 0.0f;
          split_f16(e * qk[mt][r], sMh[t * CS + s], sMl[t * CS + s]);
        }
    }
    lds_sync();

    // T = (I + A)^-1 into sTT[s][t] = T[t][s], on 16x16 blocks. The
    // diagonal blocks D_i = (I + A_ii)^-1 by forward substitution (wave i,
    // lane j < 16 owns column j); then block rows i = 1..3 on MFMA
    // (v_mfma_f32_16x16x16_f16, split form), whose C layout is also its B
    // layout: T_ij = -D_i sum_{k=j}^{i-1} A_ik T_kj, wave j computing T_ij.
    if (lane < 16) {
      const unsigned j = lane, b0 = 16 * wave;
      float col[16];
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        float acc = 0.0f;
#pragma unroll
        for (int u = 0; u < t; ++u)
          acc = fmaf(sA[(b0 + t) * FS + b0 + u], col[u], acc);
        col[t] = (unsigned)t == j ? 1.0f : ((unsigned)t > j ? -acc : 0.0f);
      }
#pragma unroll
      for (int t = 0; t < 16; ++t)
        sTT[(b0 + j) * FS + b0 + t] = col[t];
    }
    lds_sync();
    for (unsigned i = 1; i < 4; ++i) {
      if (wave < i) {
        const unsigned jb = wave;
        float4_t p{0.0f, 0.0f, 0.0f, 0.0f}, px{0.0f, 0.0f, 0.0f, 0.0f};
        for (unsigned kq = jb; kq < i; ++kq) {
          half4_t ah, al, bh, bl;
          // A_ik[L][4g + e] and T_kj[4g + e][L] = sTT[16j + L][16k + 4g + e].
          load_split4(sA + (16 * i + L) * FS + 16 * kq + 4 * g, 1, ah, al);
          load_split4(sTT + (16 * jb + L) * FS + 16 * kq + 4 * g, 1, bh, bl);
          p = mfma16k16(ah, bh, p);
          px = mfma16k16(ah, bl, px);
          px = mfma16k16(al, bh, px);
        }
        half4_t bh, bl, dh, dl;
        split4(p + px * kSplitUnscale, bh, bl);
        // D_i[L][4g + e] = sTT[16i + 4g + e][16i + L].
        load_split4(sTT + (16 * i + 4 * g) * FS + 16 * i + L, FS, dh, dl);
        float4_t tt{0.0f, 0.0f, 0.0f, 0.0f}, tx{0.0f, 0.0f, 0.0f, 0.0f};
        tt = mfma16k16(dh, bh, tt);
        tx = mfma16k16(dh, bl, tx);
        tx = mfma16k16(dl, bh, tx);
        const float4_t res = -(tt + tx * kSplitUnscale);
#pragma unroll
        for (int r = 0; r < 4; ++r)
          sTT[(16 * jb + L) * FS + 16 * i + 4 * g + r] = res[r];
      }
      lds_sync();
    }

    // T_w^T[s][t] = beta_s e^(g_s) T[t][s] and T_b^T[s][t] = beta_s T[t][s],
    // hi/lo.
    {
      const unsigned s = tid / 4, tb = 16 * (tid % 4);
      const float bw = sB[s] * sEg[s], bb = sB[s];
#pragma unroll
      for (int x4 = 0; x4 < 4; ++x4) {
        float4_t tv;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const unsigned t = tb + 4 * x4 + e;
          const float x = sTT[s * FS + t]; // read always: the select below is branch-free
          tv[e] = t >= s ? x : 0.0f;
        }
        half4_t wh, wl, bh, bl;
        split4(tv * bw, wh, wl);
        split4(tv * bb, bh, bl);
        const unsigned o = s * CS + tb + 4 * x4;
        *reinterpret_cast<half4_t *>(sTwh + o) = wh;
        *reinterpret_cast<half4_t *>(sTwl + o) = wl;
        *reinterpret_cast<half4_t *>(sTbh + o) = bh;
        *reinterpret_cast<half4_t *>(sTbl + o) = bl;
      }
    }
    lds_sync();

    // N^T = T_w^T M^T (N = M T diag(beta e^g)); -N to LDS as [t][s] hi/lo.
    // Wave w: s rows [16 w, 16 w + 16), all four t tiles.
    {
      half8_t ah[2], al[2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        ah[ks] = load8(sTwh + (16 * wave + L) * CS + 32 * ks + 8 * g);
        al[ks] = load8(sTwl + (16 * wave + L) * CS + 32 * ks + 8 * g);
      }
      float4_t acc[4], crs[4];
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        acc[tt] = crs[tt] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const half8_t bh = load8(sMh + (16 * tt + L) * CS + 32 * ks + 8 * g);
          const half8_t bl = load8(sMl + (16 * tt + L) * CS + 32 * ks + 8 * g);
          acc[tt] = mfma16(ah[ks], bh, acc[tt]);
          crs[tt] = mfma16(ah[ks], bl, crs[tt]);
          crs[tt] = mfma16(al[ks], bh, crs[tt]);
        }
      }
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        half4_t nh, nl;
        split4(-(acc[tt] + crs[tt] * kSplitUnscale), nh, nl);
        const unsigned o = (16 * tt + L) * CS + 16 * wave + 4 * g;
        *reinterpret_cast<half4_t *>(sNh + o) = nh;
        *reinterpret_cast<half4_t *>(sNl + o) = nl;
      }
    }
    lds_sync();

    // Wn and Q' pieces: W^T = K^T T_w^T and Q'^T = e^g Q^T - K^T N^T share
    // the K^T operand. Wave w writes the blocks (m, kb = w): tiles d = 2w,
    // 2w + 1 of the transposed products against the four t tiles m.
    {
      half_t *const wp = reinterpret_cast<half_t *>(rec);
      half_t *const qp = reinterpret_cast<half_t *>(rec + kPieceBytes);
      half8_t kah[2][2], kal[2][2]; // [d tile][ks]
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          kah[hf][ks] = read_kcol(sKh, KS, 32 * ks, 16 * (2 * wave + hf), g, L);
          kal[hf][ks] = read_kcol(sKl, KS, 32 * ks, 16 * (2 * wave + hf), g, L);
        }
      // Two t tiles at a time: their B operands read first, then 48 MFMAs
      // over 16 independent accumulators.
#pragma unroll
      for (int mp = 0; mp < 2; ++mp) {
        half8_t b1h[2][2], b1l[2][2], b2h[2][2], b2l[2][2]; // [tile of the pair][ks]
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int mt = 2 * mp + u;
          const unsigned t = 16 * mt + L;
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) {
            b1h[u][ks] = read_kcol(sTwh, CS, 32 * ks, 16 * mt, g, L);
            b1l[u][ks] = read_kcol(sTwl, CS, 32 * ks, 16 * mt, g, L);
            b2h[u][ks] = load8(sNh + t * CS + 32 * ks + 8 * g);
            b2l[u][ks] = load8(sNl + t * CS + 32 * ks + 8 * g);
          }
        }
        float4_t wa[2][2], wx[2][2], qa[2][2], qx[2][2]; // [tile of the pair][d tile]
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int hf = 0; hf < 2; ++hf) {
            wa[u][hf] = wx[u][hf] = qx[u][hf] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
            qa[u][hf] = qinit[hf][2 * mp + u] * sEg[16 * (2 * mp + u) + L];
          }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
          for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
              wa[u][hf] = mfma16(kah[hf][ks], b1h[u][ks], wa[u][hf]);
              qa[u][hf] = mfma16(kah[hf][ks], b2h[u][ks], qa[u][hf]);
            }
#pragma unroll
          for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
              wx[u][hf] = mfma16(kah[hf][ks], b1l[u][ks], wx[u][hf]);
              qx[u][hf] = mfma16(kah[hf][ks], b2l[u][ks], qx[u][hf]);
            }
#pragma unroll
          for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
              wx[u][hf] = mfma16(kal[hf][ks], b1h[u][ks], wx[u][hf]);
              qx[u][hf] = mfma16(kal[hf][ks], b2h[u][ks], qx[u][hf]);
            }
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int mt = 2 * mp + u;
          const float ez = sEz[16 * mt + L];
          half8_t wh, wl, qh;
#pragma unroll
          for (int hf = 0; hf < 2; ++hf)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              half_t a, b;
              split_f16(-ez * (wa[u][hf][r] + wx[u][hf][r] * kSplitUnscale), a, b);
              wh[4 * hf + r] = a;
              wl[4 * hf + r] = b;
              qh[4 * hf + r] = (half_t)(qa[u][hf][r] + qx[u][hf][r] * kSplitUnscale);
            }
          const unsigned o = (4 * mt + wave) * kBlk + 8 * lane;
          *reinterpret_cast<half8_t *>(wp + o) = wh;
          *reinterpret_cast<half8_t *>(wp + kPieceBlocks * kBlk + o) = wl;
          *reinterpret_cast<half8_t *>(qp + o) = qh;
        }
      }
    }

    // U0 = T_b V per 16-column slice (wave w: slices w + 4 rep of each V
    // block), then Z0 = e^(g_C - g) U0 and Y0 = M U0 with U0 as the B
    // operand straight from its C-layout registers. The T_b and M operands
    // are read once per wave.
    {
      half8_t tbh[4][2], tbl[4][2], mah[4][2], mal[4][2];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          tbh[mt][ks] = read_kcol(sTbh, CS, 32 * ks, 16 * mt, g, L);
          tbl[mt][ks] = read_kcol(sTbl, CS, 32 * ks, 16 * mt, g, L);
          const unsigned o = (16 * mt + L) * CS + 32 * ks + 4 * g;
          mah[mt][ks] = cat8(load4(sMh + o), load4(sMh + o + 16));
          mal[mt][ks] = cat8(load4(sMl + o), load4(sMl + o + 16));
        }
      float ezr[4][4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          ezr[mt][r] = sEz[16 * mt + 4 * g + r];
      float4_t *const z0 = reinterpret_cast<float4_t *>(rec + rec_z0(DV));
      float4_t *const y0 = z0 + (size_t)C * DV / 4;
      for (unsigned jb = 0; jb < DV; jb += VB) {
        const unsigned w = min((unsigned)VB, DV - jb);
        if (jb > 0) {
          // Further dv blocks (DV > VB) are fetched here, in turn.
          fetch_v(h, jb, w);
          lds_sync();
          store_v(w);
          lds_sync();
        }
#pragma unroll 1
        for (unsigned jt = wave; jt < w / 16; jt += 4) {
          const unsigned js = jb / 16 + jt;
          half8_t bv[2];
#pragma unroll
          for (int ks = 0; ks < 2; ++ks)
            bv[ks] = read_kcol(sQV, KS, 32 * ks, 16 * jt, g, L);
          float4_t ua[4], ux[4];
#pragma unroll
          for (int mt = 0; mt < 4; ++mt) {
            ua[mt] = ux[mt] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
              ua[mt] = mfma16(tbh[mt][ks], bv[ks], ua[mt]);
              ux[mt] = mfma16(tbl[mt][ks], bv[ks], ux[mt]);
            }
          }
          float4_t u[4];
#pragma unroll
          for (int mt = 0; mt < 4; ++mt) {
            u[mt] = ua[mt] + ux[mt] * kSplitUnscale;
            float4_t zz;
#pragma unroll
            for (int r = 0; r < 4; ++r)
              zz[r] = ezr[mt][r] * u[mt][r];
            z0[(js * 4 + mt) * 64 + lane] = zz;
          }
          half8_t ubh[2], ubl[2];
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
            split8(u[2 * kb], u[2 * kb + 1], ubh[kb], ubl[kb]);
          float4_t ya[4], yx[4];
#pragma unroll
          for (int mt = 0; mt < 4; ++mt) {
            ya[mt] = yx[mt] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
              ya[mt] = mfma16(mah[mt][kb], ubh[kb], ya[mt]);
              yx[mt] = mfma16(mah[mt][kb], ubl[kb], yx[mt]);
              yx[mt] = mfma16(mal[mt][kb], ubh[kb], yx[mt]);
            }
          }
#pragma unroll
          for (int mt = 0; mt < 4; ++mt)
            y0[(js * 4 + mt) * 64 + lane] = ya[mt] + yx[mt] * kSplitUnscale;
        }
      }
    }
    if (hr + 1 < R && DV > VB)
      fetch_v(h + 1, 0, w0);
  }
}

// --------------------------------------------------------------- scan

// The scan workgroup: 4 waves, one per SIMD, for one (value head, 16-column
// dv slice). Wave w owns rows [32 w, 32 w + 32) of the slice's state (C
// tiles 2w and 2w + 1, in its registers for the whole call) and token tile
// w (rows [16 w, 16 w + 16)) of each chunk's Z and Y. Per chunk:
//   1. every wave splits its state rows into the hi/lo B operand of k block
//      w and puts it in LDS; barrier X1; every wave reads the whole split S;
//   2. Z_w = Z0_w + sum_kb Wn[w][kb] S[kb], Y_w = Y0_w + sum_kb Q'[w][kb] S[kb];
//   3. Z_w, split, to LDS; barrier X2; every wave reads the split Z;
//   4. S_w <- e^(g_C) S_w + sum_kb K^T[w][kb] Z[kb] (the two C tiles of w).
// The chain of a chunk is thus 12 + 12 MFMAs per wave instead of 48 + 48 on
// one wave. Each wave loads exactly the operand blocks it multiplies (a
// quarter of each piece, 88 KB per workgroup and chunk), one chunk ahead,
// straight into its registers. A fifth wave keeps those loads L2 hits: the
// pieces come from HBM / the MALL (the prep wrote them), ~3,500 cycles away
// under this load against ~1,900 cycles of work per chunk, so it reads one
// dword per 128-byte line of its workgroup's share of the record and K^T
// piece of chunk c + kWarmAhead (the slice workgroups of a value head share
// an XCD, and split the head's lines between them). Its loads count on its
// own vmcnt, so the compute waves' waits never cover them. No wave issues a global store inside the
// chunk loop -- the Y tiles go to an LDS stage that is written out every
// kStageChunks chunks and at the end -- so a wave's only outstanding
// vector-memory operations are those loads, which complete in order: the
// wait for one chunk's operands then never drains the next chunk's (with a
// store pending the compiler's wait would be vmcnt(0)).
constexpr int kStageChunks = 32;
constexpr int kAhead = 1;      // chunks of operands in flight in registers
constexpr int kWarmAhead = 3;  // chunks ahead that the warming wave reads
constexpr int kWarmSets = 8;   // its register sets (a touch is consumed kWarmSets chunks later)
constexpr int kScanThreads = 320;

// With NORM the kernel ends with gatedRmsNorm over the value head's output
// rows (Reference.metal:228-259): once every slice workgroup of the head has
// written its columns (a per-head arrival counter, zeroed by the prep; the
// host launches it only when the whole grid fits on the device at once, so
// every workgroup is resident and the wait ends; it is bounded regardless),
// workgroup js normalises rows [js p, js p + p) of the head, p = ceil(T /
// slices), in place: the sequential sum of squares of each row, then out =
// fp16(fp16(x * factor) * weight * silu(gate)) per element (gated_norm.hpp,
// the arithmetic of the standalone kernel).
// The wait polls at most `spin` times (delta_chunked_wait_limit(), 2^22 by
// default: ~0.3 s). A workgroup that gives up sets the fourth word of its
// head's counter record, which delta_chunked_wait_status() reads after the
// call: the rows it then normalises may not all have been written.
unsigned g_wait_limit = 1u << 22;
constexpr unsigned kNormMaxDv = 256; // dv the fused norm supports

template <bool NORM>
__global__ __launch_bounds__(kScanThreads, 1) void delta_scan_kernel(
    float *__restrict__ state, half_t *__restrict__ out, const void *__restrict__ ws,
    unsigned T, unsigned Hk, unsigned Hv, unsigned DV, const half_t *__restrict__ gate,
    const float *__restrict__ nweight, unsigned *cnt, float neps, unsigned spin) {
  // Workgroups are dealt to the 8 XCDs round-robin by block index. Give
  // each XCD a contiguous run of (value head, slice) pairs, so that the
  // workgroups reading one value head's pieces and one key head's K^T piece
  // share an L2.
  const unsigned slices = DV / 16, nb = gridDim.x;
  const unsigned Lb = nb % 8 == 0 ? (blockIdx.x % 8) * (nb / 8) + blockIdx.x / 8 : blockIdx.x;
  const unsigned h = Lb / slices, js = Lb % slices, kh = h / (Hv / Hk);
  const unsigned w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const unsigned lane = threadIdx.x & 63u, g = lane >> 4, L = lane & 15u;
  const unsigned chunks = (T + C - 1) / C, last = chunks - 1;
  const size_t recB = rec_bytes(DV), vStride = (size_t)Hv * DV;
  void *const wsp = const_cast<void *>(ws);

  __shared__ half8_t sSx[2][4][64]; // split S: [hi, lo][k block][lane]
  __shared__ half8_t sZx[2][2][64]; // split Z: [hi, lo][k block][lane], tile 2kb | 2kb + 1
  __shared__ __attribute__((aligned(16))) half_t sY[kStageChunks][C][16];

  // The operand blocks of wave w for one chunk.
  struct Ops {
    half8_t wn[2][4]; // Wn blocks (w, kb): [hi, lo][kb]
    half8_t kt[2][4]; // K^T blocks (tile 2w + i, kb) at 2i + kb: [hi, lo][.]
    half8_t qp[4];    // Q' blocks (w, kb)
    float4_t z0, y0;  // tile w of the slice's Z0 and Y0
    float eC;         // e^(g_C)
  };
  // The loads of one chunk's operands in three parts, which a step spreads
  // over its phases: issued in one burst, the 88 KB of a workgroup's loads
  // would hold each wave at its load instructions until the CU's memory
  // pipeline took them (~57 bytes per cycle per CU from L2, measured),
  // while its MFMAs wait behind them.
  auto load_wn = [&](unsigned c, Ops &d) {
    const char *r = rec_ptr(wsp, recB, Hv, c, h);
    const half8_t *pw = reinterpret_cast<const half8_t *>(r) + 4 * w * 64 + lane;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      d.wn[0][b] = pw[b * 64];
      d.wn[1][b] = pw[(kPieceBlocks + b) * 64];
    }
  };
  auto load_kt = [&](unsigned c, Ops &d) {
    const half8_t *pk =
        reinterpret_cast<const half8_t *>(kpiece_ptr(wsp, recB, chunks, Hv, Hk, c, kh)) +
        4 * w * 64 + lane;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      d.kt[0][b] = pk[b * 64];
      d.kt[1][b] = pk[(kPieceBlocks + b) * 64];
    }
  };
  auto load_qz = [&](unsigned c, Ops &d) {
    const char *r = rec_ptr(wsp, recB, Hv, c, h);
    const half8_t *pq = reinterpret_cast<const half8_t *>(r + kPieceBytes) + 4 * w * 64 + lane;
#pragma unroll
    for (int b = 0; b < 4; ++b)
      d.qp[b] = pq[b * 64];
    const float4_t *pz =
        reinterpret_cast<const float4_t *>(r + rec_z0(DV)) + (4 * js + w) * 64 + lane;
    d.z0 = pz[0];
    d.y0 = pz[(size_t)C * DV / 4];
    d.eC = *reinterpret_cast<const float *>(r + rec_scalars(DV));
  };
  auto load_ops = [&](unsigned c, Ops &d) {
    load_wn(c, d);
    load_kt(c, d);
    load_qz(c, d);
  };

  // Chunks [c0, c] of the stage to the output rows (two 16-byte stores per
  // 16-column row; rows past the end of the tokens are skipped).
  auto flush = [&](unsigned c) {
    const unsigned c0 = c - c % kStageChunks, rows = (c - c0 + 1) * C;
    for (unsigned i = threadIdx.x; i < 2 * rows; i += 256) { // waves 0-3
      const unsigned rr = i >> 1, hf = i & 1u, t = c0 * C + rr;
      if (t < T)
        *reinterpret_cast<uint4_t *>(out + (size_t)t * vStride + (size_t)h * DV + 16 * js +
                                     8 * hf) =
            *reinterpret_cast<const uint4_t *>(&sY[rr / C][rr % C][8 * hf]);
    }
  };

  if (w == 4) {
    // The warming wave: this workgroup's share of a chunk is recPart bytes
    // of each record (Wn, Q', Z0, Y0, scalars) and kPart bytes of the K^T
    // piece; it reads one dword per line of the first 16 KiB of the former
    // and 8 KiB of the latter (all of both at dv = 128). A touched value is
    // consumed kWarmSets chunks later (the loop is unrolled over the register
    // sets), long after it came, so the wave never waits on its loads.
    const unsigned R = Hv / Hk;
    const size_t recPart = (recB + slices - 1) / slices;
    const size_t kShare = (size_t)R * slices;
    const size_t kPart = ((size_t)kPieceBytes + kShare - 1) / kShare;
    const size_t kIdx = (size_t)(h % R) * slices + js;
    const size_t r0 = js * recPart, r1 = min(r0 + recPart, recB) - 4;
    const size_t k0 = kIdx * kPart, k1 = min(k0 + kPart, (size_t)kPieceBytes) - 4;
    // (The empty asm reading a register set is its consumption: the
    // compiler waits for those loads there, in program order, and cannot
    // hoist an arithmetic use of them ahead of the barriers.) Chunk x's
    // touch goes to register set x % kWarmSets.
    float4_t tv[kWarmSets];
#pragma unroll
    for (int u = 0; u < kWarmSets; ++u)
      tv[u] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
    auto touch = [&](unsigned c, float4_t &v) {
      asm volatile("" ::"v"(v[0]), "v"(v[1]), "v"(v[2]));
      const char *r = rec_ptr(wsp, recB, Hv, c, h);
      const char *k = kpiece_ptr(wsp, recB, chunks, Hv, Hk, c, kh);
      v[0] = *reinterpret_cast<const float *>(r + (min(r0 + 128 * lane, r1) & ~(size_t)3));
      v[1] = *reinterpret_cast<const float *>(r + (min(r0 + 8192 + 128 * lane, r1) & ~(size_t)3));
      v[2] = *reinterpret_cast<const float *>(k + (min(k0 + 128 * lane, k1) & ~(size_t)3));
    };
#pragma unroll
    for (int u = 1; u < kWarmAhead; ++u)
      touch(min((unsigned)u, last), tv[u % kWarmSets]);
    unsigned c = 0;
    for (; c + kWarmSets <= chunks; c += kWarmSets) {
#pragma unroll
      for (int u = 0; u < kWarmSets; ++u) {
        touch(min(c + u + kWarmAhead, last), tv[(u + kWarmAhead) % kWarmSets]);
        lds_sync(); // X1
        lds_sync(); // X2
      }
    }
    for (; c < chunks; ++c) {
      lds_sync(); // X1
      lds_sync(); // X2
    }
#pragma unroll
    for (int u = 0; u < kWarmSets; ++u)
      asm volatile("" ::"v"(tv[u][0]), "v"(tv[u][1]), "v"(tv[u][2]));
  } else {

  // State rows of wave w: register r of tile i holds S[32 w + 16 i + 4 g + r][j].
  const unsigned j = 16 * js + L;
  float *const scol = state + (size_t)h * DK * DV + j;
  float4_t S[2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      S[i][r] = scol[(size_t)(32 * w + 16 * i + 4 * g + r) * DV];

  // Chunk c multiplies `cur` and refills `dst` (the buffer of chunk c - 1)
  // with chunk c + kAhead.
  auto step = [&](unsigned c, const Ops &cur, Ops &dst) {
    const unsigned cn = min(c + kAhead, last);
    load_wn(cn, dst);
    __builtin_amdgcn_sched_barrier(0);
    // 1. The split S, through LDS.
    {
      half8_t hi, lo;
      split8(S[0], S[1], hi, lo);
      sSx[0][w][lane] = hi;
      sSx[1][w][lane] = lo;
    }
    lds_sync(); // X1
    half8_t bh[4], bl[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      bh[kb] = sSx[0][kb][lane];
      bl[kb] = sSx[1][kb][lane];
    }
    __builtin_amdgcn_sched_barrier(0);
    load_kt(cn, dst);
    __builtin_amdgcn_sched_barrier(0);
    // 2. Z_w and Y_w: five accumulators, each MFMA five issues after the
    // one it depends on (a dependent 16x16x32 MFMA waits ~44 cycles, an
    // independent one issues every ~18).
    float4_t za = cur.z0, zx{0.0f, 0.0f, 0.0f, 0.0f}, zy{0.0f, 0.0f, 0.0f, 0.0f};
    float4_t ya = cur.y0, yx{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      za = mfma16(cur.wn[0][kb], bh[kb], za);
      ya = mfma16(cur.qp[kb], bh[kb], ya);
      zx = mfma16(cur.wn[0][kb], bl[kb], zx);
      yx = mfma16(cur.qp[kb], bl[kb], yx);
      zy = mfma16(cur.wn[1][kb], bh[kb], zy);
    }
    // 3. The split Z tile w (halves 4 (w % 2) .. of k block w / 2), and the
    // output tile to the stage.
    {
      half4_t hi, lo;
      split4(za + (zx + zy) * kSplitUnscale, hi, lo);
      reinterpret_cast<half4_t *>(&sZx[0][w >> 1][lane])[w & 1u] = hi;
      reinterpret_cast<half4_t *>(&sZx[1][w >> 1][lane])[w & 1u] = lo;
      const float4_t y = ya + yx * kSplitUnscale;
      half_t *const sy = &sY[c % kStageChunks][16 * w + 4 * g][L];
#pragma unroll
      for (int r = 0; r < 4; ++r)
        sy[16 * r] = (half_t)y[r];
    }
    lds_sync(); // X2
    half8_t zh[2], zl[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      zh[kb] = sZx[0][kb][lane];
      zl[kb] = sZx[1][kb][lane];
    }
    __builtin_amdgcn_sched_barrier(0);
    load_qz(cn, dst);
    __builtin_amdgcn_sched_barrier(0);
    // 4. S_w <- e^(g_C) S_w + K^T Z.
    float4_t sa[2], sx[2], sy[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      sa[i] = S[i] * cur.eC;
      sx[i] = sy[i] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
    }
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        sa[i] = mfma16(cur.kt[0][2 * i + kb], zh[kb], sa[i]);
        sx[i] = mfma16(cur.kt[0][2 * i + kb], zl[kb], sx[i]);
        sy[i] = mfma16(cur.kt[1][2 * i + kb], zh[kb], sy[i]);
      }
#pragma unroll
    for (int i = 0; i < 2; ++i)
      S[i] = sa[i] + (sx[i] + sy[i]) * kSplitUnscale;
    // The stage's writes of this chunk were made before X2; its reads finish
    // before the next X1 (lds_sync waits for them), ahead of any rewrite.
    if (c % kStageChunks == kStageChunks - 1 || c == last)
      flush(c);
  };

  Ops oa, ob;
  load_ops(0, oa);
  unsigned c = 0;
  for (; c + 1 < chunks; c += 2) {
    step(c, oa, ob);
    step(c + 1, ob, oa);
  }
  if (c < chunks)
    step(c, oa, ob);

#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      scol[(size_t)(32 * w + 16 * i + 4 * g + r) * DV] = S[i][r];
  }

  if constexpr (NORM) {
    // Arrival. The head's 16-byte counter record holds a 64-bit arrival word
    // -- bits 0-7 the count, 7 bits per XCD at 8 + 7 x the arrivals from
    // that XCD -- and a second count. Every workgroup's output stores reach
    // L2 (each wave waits for its own), then it adds 1 + 2^(8 + 7 xcd) and
    // waits, with relaxed loads, for all slices. When they all ran on this
    // XCD they share its L2: dropping this CU's L1 makes their rows visible.
    // Otherwise their L2s are not coherent: every workgroup writes its L2
    // back (a device-scope release), counts again, and acquires device-wide.
    unsigned long long *const word = reinterpret_cast<unsigned long long *>(cnt + 4 * h);
    unsigned *const again = cnt + 4 * h + 2;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    __shared__ unsigned sDeviceWide;
    if (threadIdx.x == 0) {
      unsigned xcc;
      asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(xcc));
      __hip_atomic_fetch_add(word, 1ull + (1ull << (8 + 7 * (xcc & 7u))), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
      unsigned long long seen = 0;
      bool arrived = false;
      for (unsigned i = 0; i < spin && !arrived; ++i) {
        seen = __hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        arrived = (seen & 0xFFu) >= slices;
        if (!arrived)
          __builtin_amdgcn_s_sleep(2);
      }
      const unsigned here = (unsigned)(seen >> (8 + 7 * (xcc & 7u))) & 0x7Fu;
      sDeviceWide = here != slices;
      if (here != slices) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        __hip_atomic_fetch_add(again, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        arrived = false;
        for (unsigned i = 0; i < spin && !arrived; ++i) {
          arrived = __hip_atomic_load(again, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= slices;
          if (!arrived)
            __builtin_amdgcn_s_sleep(2);
        }
      }
      if (!arrived)
        __hip_atomic_store(cnt + 4 * h + 3, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (sDeviceWide)
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    else
      asm volatile("buffer_inv sc0" ::: "memory");
    const unsigned per = (T + slices - 1) / slices, r0 = min(T, js * per);
    const unsigned nrows = min(T, r0 + per) - r0, c8n = DV / 8;
    // The stage is free now: the weight, then the row factors.
    float *const sWn = reinterpret_cast<float *>(&sY[0][0][0]);
    float *const sF = sWn + DV;
    for (unsigned jj = threadIdx.x; jj < DV; jj += kScanThreads)
      sWn[jj] = nweight[jj];
    half_t *const ob = out + (size_t)r0 * vStride + (size_t)h * DV;
    const half_t *const gb = gate + (size_t)r0 * vStride + (size_t)h * DV;
    const unsigned kRowsPass = (unsigned)(sizeof(sY) / sizeof(float)) - DV;
    auto norm8 = [&](uint4_t x, uint4_t gv, float f, unsigned k8) {
      return gated_norm_out8(x, gv, f, sWn + 8 * k8);
    };
    for (unsigned rb = 0; rb < nrows; rb += kRowsPass) {
      const unsigned nr = min(kRowsPass, nrows - rb);
      for (unsigned r = threadIdx.x; r < nr; r += kScanThreads) {
        const uint4_t *row = reinterpret_cast<const uint4_t *>(ob + (size_t)(rb + r) * vStride);
        uint4_t xr[16];
        float sum = 0.0f;
        for (unsigned k0 = 0; k0 < c8n; k0 += 16) {
#pragma unroll
          for (unsigned k8 = 0; k8 < 16; ++k8)
            if (k0 + k8 < c8n)
              xr[k8] = row[k0 + k8];
#pragma unroll
          for (unsigned k8 = 0; k8 < 16; ++k8)
            if (k0 + k8 < c8n)
              sum = sumsq8(xr[k8], sum);
        }
        sF[r] = gated_norm_factor(sum, DV, neps);
      }
      __syncthreads();
      // Two 8-column pieces per thread and pass, both loaded before either
      // is computed.
      const unsigned items = nr * c8n;
      for (unsigned i = threadIdx.x; i < items; i += 2 * kScanThreads) {
        const unsigned i2 = i + kScanThreads;
        const unsigned ra = i / c8n, ka = i % c8n, rb2 = i2 / c8n, kb = i2 % c8n;
        uint4_t *const pa = reinterpret_cast<uint4_t *>(ob + (size_t)(rb + ra) * vStride) + ka;
        uint4_t *const pb = reinterpret_cast<uint4_t *>(ob + (size_t)(rb + rb2) * vStride) + kb;
        const uint4_t xa = *pa;
        const uint4_t ga =
            *(reinterpret_cast<const uint4_t *>(gb + (size_t)(rb + ra) * vStride) + ka);
        uint4_t xb{0, 0, 0, 0}, gbv{0, 0, 0, 0};
        if (i2 < items) {
          xb = *pb;
          gbv = *(reinterpret_cast<const uint4_t *>(gb + (size_t)(rb + rb2) * vStride) + kb);
        }
        *pa = norm8(xa, ga, sF[ra], ka);
        if (i2 < items)
          *pb = norm8(xb, gbv, sF[rb2], kb);
      }
      __syncthreads();
    }
  }
}

} // namespace

bool delta_chunked_supported(const DeltaShape &s) {
  return s.Dk == DK && s.Dv % 16 == 0 && s.Dv >= 16 && s.Hk >= 1 && s.Hv % s.Hk == 0 &&
         s.T >= 32;
}

// After the records and K^T pieces: the fused norm's 16-byte per-value-head
// arrival records (256-byte aligned).
static size_t counters_offset(const DeltaShape &s) {
  const size_t chunks = (s.T + C - 1) / C;
  return chunks * (s.Hv * rec_bytes(s.Dv) + s.Hk * (size_t)kPieceBytes);
}

size_t delta_chunked_workspace_bytes(const DeltaShape &s) {
  return counters_offset(s) + ((16 * (size_t)s.Hv + 255) / 256) * 256;
}

namespace {

template <bool QK16>
hipError_t launch_chunked(const void *q, const void *k, const uint16_t *v, const float *beta,
                          const float *decay, float *state, uint16_t *out, void *ws,
                          float eps, float qscale, const DeltaShape &s, hipStream_t stream,
                          const uint16_t *gate = nullptr, const float *nweight = nullptr,
                          float neps = 0.0f) {
  const unsigned chunks = (s.T + C - 1) / C;
  unsigned *cnt = gate ? reinterpret_cast<unsigned *>(static_cast<char *>(ws) +
                                                      counters_offset(s))
                       : nullptr;
  hipLaunchKernelGGL((delta_prep_kernel<QK16>), dim3(chunks, s.Hk), dim3(256), 0, stream, q, k,
                     reinterpret_cast<const half_t *>(v), beta, decay, ws, s.T, s.Hk, s.Hv,
                     s.Dv, eps, qscale, cnt);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return e;
  const dim3 grid(s.Hv * (s.Dv / 16));
  if (!gate) {
    hipLaunchKernelGGL(delta_scan_kernel<false>, grid, dim3(kScanThreads), 0, stream, state,
                       reinterpret_cast<half_t *>(out), ws, s.T, s.Hk, s.Hv, s.Dv,
                       (const half_t *)nullptr, (const float *)nullptr, (unsigned *)nullptr,
                       0.0f, 0u);
    return hipGetLastError();
  }
  // The norm's arrival wait needs every slice workgroup of a value head
  // resident at once: delta_chunked_norm_resident() checked that the whole
  // grid fits on the device together (a cooperative launch would guarantee
  // it too, but costs ~17 us more per call here, measured).
  hipLaunchKernelGGL(delta_scan_kernel<true>, grid, dim3(kScanThreads), 0, stream, state,
                     reinterpret_cast<half_t *>(out), ws, s.T, s.Hk, s.Hv, s.Dv,
                     reinterpret_cast<const half_t *>(gate), nweight, cnt, neps, g_wait_limit);
  return hipGetLastError();
}

} // namespace

bool delta_chunked_norm_resident(const DeltaShape &s) {
  static int capacity = -1; // workgroups of the norm scan resident at once
  if (capacity < 0) {
    int dev = 0, cus = 0, per = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &per, reinterpret_cast<const void *>(&delta_scan_kernel<true>), kScanThreads, 0) !=
            hipSuccess)
      return false;
    capacity = cus * per;
  }
  return s.Dv <= kNormMaxDv && (long)s.Hv * (s.Dv / 16) <= capacity;
}

hipError_t launch_delta_chunked(const float *q, const float *k, const uint16_t *v,
                                const float *beta, const float *decay, float *state,
                                uint16_t *out, void *ws, const DeltaShape &s,
                                hipStream_t stream) {
  return launch_chunked<false>(q, k, v, beta, decay, state, out, ws, 0.0f, 1.0f, s, stream);
}

hipError_t launch_delta_chunked_qk16(const uint16_t *q, const uint16_t *k, const uint16_t *v,
                                     const float *beta, const float *decay, float *state,
                                     uint16_t *out, void *ws, float eps, float qscale,
                                     const DeltaShape &s, hipStream_t stream) {
  return launch_chunked<true>(q, k, v, beta, decay, state, out, ws, eps, qscale, s, stream);
}

hipError_t launch_delta_chunked_gated_norm(const uint16_t *q, const uint16_t *k,
                                           const uint16_t *v, const float *beta,
                                           const float *decay, float *state, const uint16_t *gate,
                                           const float *nweight, uint16_t *out, void *ws,
                                           float eps, float qscale, float neps,
                                           const DeltaShape &s, hipStream_t stream) {
  return launch_chunked<true>(q, k, v, beta, decay, state, out, ws, eps, qscale, s, stream, gate,
                              nweight, neps);
}

unsigned delta_chunked_wait_limit(unsigned limit) {
  const unsigned old = g_wait_limit;
  g_wait_limit = limit;
  return old;
}

hipError_t delta_chunked_wait_status(const void *ws, const DeltaShape &s, hipStream_t stream,
                                     bool *gave_up) {
  *gave_up = false;
  std::vector<unsigned> rec(4 * (size_t)s.Hv);
  hipError_t e = hipMemcpyAsync(rec.data(), static_cast<const char *>(ws) + counters_offset(s),
                                rec.size() * sizeof(unsigned), hipMemcpyDeviceToHost, stream);
  if (e == hipSuccess)
    e = hipStreamSynchronize(stream);
  if (e != hipSuccess)
    return e;
  for (size_t h = 0; h < s.Hv; ++h)
    *gave_up = *gave_up || rec[4 * h + 3] != 0;
  return hipSuccess;
}

unsigned delta_chunked_dispatches() { return 2; }

const char *delta_chunked_kernel_name(unsigned index) {
  return index == 0 ? "deltaChunkPrep" : "deltaChunkScan";
}

} // namespace llmi
