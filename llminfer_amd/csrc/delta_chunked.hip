// Gated delta rule, chunk-wise (WY / UT-transform) form: the DeltaNet
// prefill.
//
// Same result as the token recurrence of graphDeltaUpdate / updateDeltaColumn
// (Graph.metal:146-170, Reference.metal:182-197), which walks the tokens one
// by one. The published chunk algorithm (Yang, Kautz, Hatamizadeh, "Gated
// Delta Networks", arXiv:2412.06464; Yang et al., "Parallelizing Linear
// Transformers with the Delta Rule over Sequence Length", arXiv:2406.06484)
// splits the tokens into chunks of C = 32. With g the cumulative log decay
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
//  * deltaChunkPrep, grid (chunk, key head), 256 threads, two workgroups a
//    CU (56 KB of LDS each): every chunk at once. The Gram matrices K K^T
//    and Q K^T on fp16 MFMA (kept in registers); per value head the decay
//    weighting, T by blocked substitution (the two 16x16 diagonal blocks in
//    fp32, the off-diagonal block on MFMA), and the products Wn and Q' on
//    fp16 MFMA in split form. The results (with T_b and M) go to the
//    workspace already in the register order of the scan's MFMA operands.
//
//  * deltaChunkScan, grid (value head, 16-column dv slice), 4 compute waves
//    and a fifth wave. Wave w keeps rows [32 w, 32 w + 32) of the state
//    slice S [dk x 16] in registers; waves 1 and 2 compute the two 16-token
//    tiles of each chunk's Z, waves 0 and 3 those of Y; S and Z pass
//    between the waves through LDS, two barriers per chunk. The fifth wave
//    forms the slice's Z0 and Y0 from T_b, M and V a chunk ahead and keeps
//    the other operands' lines in L2. Every
//    product runs on v_mfma_f32_16x16x32_f16, with the state (and Z) as the
//    B operand straight from the C-layout registers of the product that made
//    it: the k index of an operand block is permuted (sigma below) so that
//    the 8 halves a lane supplies are the 8 rows it holds in two consecutive
//    16-row C tiles; the A operands (Wn, Q', K^T) were written by the prep
//    with the same permutation. Each wave loads its own operand blocks one
//    chunk ahead into registers.
//
// Why 32: the prep's cost per chunk is dominated by its chain of dependent
// phases (the triangular solve, the products that follow it), which shrink
// with the chunk, and at 32 two workgroups share a CU and hide each other's
// latencies; the scan's chain per chunk (two barriers, two short MFMA runs)
// costs about as much at 32 as at 64 tokens.
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

constexpr int C = 32;       // chunk length
constexpr int DK = 128;     // key dimension handled by these kernels
constexpr int KS = DK + 8;  // fp16 stride of [token][dk] rows in LDS (and of V rows)
constexpr int CS = C + 8;   // fp16 stride of [*][token] rows in LDS
constexpr int FS = C + 1;   // fp32 stride of the prep's A and T^T rows
constexpr int TT = C / 16;  // 16-token tiles of a chunk
constexpr int KB = DK / 32; // 32-wide blocks of the key dimension
constexpr int DT = DK / 16; // 16-wide tiles of the key dimension

// MFMA operand blocks (v_mfma_f32_16x16x32_f16) in register order: lane l
// holds 8 halves at halves [8 l, 8 l + 8) of the block.
//
// Permuted k: in a 32-wide k block, element e of lane l (g = l / 16) stands
// for k = sigma(g, e) = 4g + e (e < 4) or 16 + 4g + (e - 4) (e >= 4) -- the
// rows a lane holds in the C layout of the two 16-row tiles of that block
// (register r of tile m holds row 16m + 4g + r). A product whose k is
// permuted the same way in both operands is unchanged.
//
// The operands of the scan's products for one chunk:
//  * Wn piece (per chunk and value head): block KB m + kb holds token rows t
//    of tile m against permuted k = d in block kb; TT x KB blocks of hi
//    halves, then as many of lo halves.
//  * Q' piece: the same blocks, hi halves only (Q' feeds the outputs alone).
//  * K^T piece (per chunk and key head): block i holds rows d of tile i
//    against permuted k = t (the chunk's one 32-token block); DT blocks of
//    hi halves, then DT of lo halves.
//  * T_b and M pieces (per chunk and value head), the operands of the
//    scan's U0 = T_b V and Y0 = M U0: block TT hl + m holds rows t of tile m
//    (hl 0: hi halves, 1: lo halves), against k = u in plain order for T_b
//    (V is its B operand) and permuted for M (U0 in C layout is its B
//    operand).
constexpr int kBlk = 64 * 8;
constexpr int kWnBlocks = TT * KB;
constexpr int kWnBytes = 2 * kWnBlocks * kBlk * 2; // 16 KiB
constexpr int kQpBytes = kWnBlocks * kBlk * 2;     // 8 KiB
constexpr int kKtBlocks = DT;
constexpr int kKtBytes = 2 * kKtBlocks * kBlk * 2; // 16 KiB
constexpr int kTbBytes = 2 * TT * kBlk * 2;        // 4 KiB
constexpr int kMBytes = 2 * TT * kBlk * 2;         // 4 KiB

// Workspace. Per (chunk, value head) a record: the Wn, Q', T_b and M
// pieces, then 64 floats of scalars: e^(g_C) at 0, e^(g_C - g_t) at 32 + t.
// After all records, per (chunk, key head) the K^T piece.
constexpr int kScalarBytes = 256;
constexpr size_t kRecTb = (size_t)kWnBytes + kQpBytes;
constexpr size_t kRecM = kRecTb + kTbBytes;
constexpr size_t kRecScalars = kRecM + kMBytes;
constexpr size_t kRecBytes = kRecScalars + kScalarBytes; // 32.25 KiB
__device__ __forceinline__ char *rec_ptr(void *ws, size_t recB, size_t Hv, size_t c,
                                         size_t h) {
  return static_cast<char *>(ws) + (c * Hv + h) * recB;
}
__device__ __forceinline__ char *kpiece_ptr(void *ws, size_t recB, size_t chunks, size_t Hv,
                                            size_t Hk, size_t c, size_t kh) {
  return static_cast<char *>(ws) + chunks * Hv * recB + (c * Hk + kh) * kKtBytes;
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

// One workgroup per (chunk, key head), four waves; the key head's value
// heads in turn.
//
// QK16: q and k arrive as fp16 rows and are L2-normalised here exactly as
// l2NormF32 (Graph.metal:96-109) would: one lane per (token, q or k) row of
// the chunk runs the reference's sequential sum of squares, and each fp32
// element is the single product x * factor -- the bits l2NormF32 writes.
template <bool QK16>
__global__ __launch_bounds__(256, 2) void delta_prep_kernel(
    const void *__restrict__ qp, const void *__restrict__ kp, const float *__restrict__ beta,
    const float *__restrict__ decay, void *__restrict__ ws,
    unsigned T, unsigned Hk, unsigned Hv, unsigned DV, float eps, float qscale, unsigned *cnt) {
  const float *q = static_cast<const float *>(qp), *k = static_cast<const float *>(kp);
  const half_t *q16 = static_cast<const half_t *>(qp), *k16 = static_cast<const half_t *>(kp);
  const unsigned c = blockIdx.x, kh = blockIdx.y;
  const unsigned R = Hv / Hk, chunks = (T + C - 1) / C;
  const unsigned t0 = c * C, n = min((unsigned)C, T - t0);
  const unsigned tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const unsigned g = lane >> 4, L = lane & 15u;
  const size_t recB = kRecBytes;
  const size_t qkStride = (size_t)Hk * DK;
  // The fused norm's per-value-head arrival records (4 words each), zeroed
  // here (the scan runs after this launch on the same stream).
  if (cnt && c == 0 && tid < 4 * R)
    cnt[4 * kh * R + tid] = 0;

  __shared__ __attribute__((aligned(16))) half_t sKh[C * KS], sKl[C * KS];
  __shared__ __attribute__((aligned(16))) half_t sQV[C * KS]; // Q hi
  __shared__ __attribute__((aligned(16))) float sATT[2 * C * FS]; // A, then T^T
  float *const sA = sATT, *const sTT = sATT + C * FS;
  // T_w^T, T_b^T, M and -N as hi/lo [*][token] rows; Q lo before them,
  // during the Gram products.
  __shared__ __attribute__((aligned(16))) half_t sTMN[8 * C * CS];
  half_t *const sTwh = sTMN, *const sTwl = sTMN + C * CS;
  half_t *const sTbh = sTMN + 2 * C * CS, *const sTbl = sTMN + 3 * C * CS;
  half_t *const sMh = sTMN + 4 * C * CS, *const sMl = sTMN + 5 * C * CS;
  half_t *const sNh = sTMN + 6 * C * CS, *const sNl = sTMN + 7 * C * CS;
  half_t *const sQl = sTMN;
  static_assert(C * KS <= 8 * C * CS, "Q lo fits");
  // Per value head, double-buffered by head parity: cumulative log decay,
  // beta, e^(g_t), e^(g_C - g_t).
  __shared__ double sG[2][C];
  __shared__ float sB[2][C], sEg[2][C], sEz[2][C];
  __shared__ float sFac[QK16 ? 2 * C : 1]; // QK16: L2 factors of the k rows, then the q rows

  // Loads that later phases need, issued up front so that their latency
  // hides behind the K/Q split and the Gram products: the fp32 queries of
  // the Q' initial values (wave w: d tiles 2w, 2w + 1, all t), the gates
  // of the first value head (wave 0) and its first block of V.
  float4_t qinit[2][TT];
  half4_t qraw[2][TT]; // QK16: the fp16 queries, normalised once the factors are known
#pragma unroll
  for (int hf = 0; hf < 2; ++hf)
#pragma unroll
    for (int mt = 0; mt < TT; ++mt) {
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
  // Wave 1 prepares each value head's gates one head ahead, off the chain of
  // dependent phases: the loads, then the cumulative log decay (double;
  // padding tokens: decay 1, beta 0), e^(g_t), e^(g_C - g_t) and e^(g_C).
  float gateA = 1.0f, gateB = 0.0f;
  auto load_gates = [&](unsigned h) {
    if (wave == 1 && lane < n) {
      gateA = decay[(size_t)(t0 + lane) * Hv + h];
      gateB = beta[(size_t)(t0 + lane) * Hv + h];
    }
  };
  auto gates = [&](unsigned hr) {
    if (wave == 1) {
      const unsigned t = lane, pb = hr & 1u;
      const float a = gateA, b = gateB;
      double gg = a > 0.0f ? (double)logf(a) : -1.0e4;
#pragma unroll
      for (int off = 1; off < C; off <<= 1) {
        const double up = __shfl_up(gg, off);
        if (lane >= (unsigned)off)
          gg += up;
      }
      const double gC = __shfl(gg, C - 1);
      if (t < C) {
        sG[pb][t] = gg;
        sB[pb][t] = b;
        sEg[pb][t] = expf((float)gg);
        sEz[pb][t] = expf((float)(gC - gg));
      }
      float *const sc = reinterpret_cast<float *>(rec_ptr(ws, recB, Hv, c, kh * R + hr) +
                                                   kRecScalars);
      if (t < C)
        sc[32 + t] = expf((float)(gC - gg));
      if (t == C - 1)
        sc[0] = expf((float)gg);
    }
  };
  load_gates(kh * R);

  // QK16: the L2 factors of the chunk's k rows (threads 0 .. C-1) and q
  // rows (C .. 2C-1), each the sequential sum over one row.
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
      for (int mt = 0; mt < TT; ++mt) {
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
  gates(0);
  if (R > 1)
    load_gates(kh * R + 1);
  lds_sync();

  // The K^T piece of this (chunk, key head): block i (wave w writes 2w and
  // 2w + 1), lane (g, L) element e = K[sigma(g, e)][16 i + L].
  {
    half_t *kt = reinterpret_cast<half_t *>(kpiece_ptr(ws, recB, chunks, Hv, Hk, c, kh));
#pragma unroll
    for (int bi = 0; bi < 2; ++bi) {
      const unsigned b = 2 * wave + bi;
      const unsigned off0 = ((4 * g + L / 4) * KS + 16 * b + 4 * (L % 4)) * 2;
      const unsigned off1 = off0 + 16 * KS * 2;
      *reinterpret_cast<half8_t *>(kt + b * kBlk + 8 * lane) =
          cat8(read_tr(sKh, off0), read_tr(sKh, off1));
      *reinterpret_cast<half8_t *>(kt + (kKtBlocks + b) * kBlk + 8 * lane) =
          cat8(read_tr(sKl, off0), read_tr(sKl, off1));
    }
  }

  // K K^T and Q K^T stay in registers: wave w holds the tile of rows t in
  // tile gm = w / 2 and columns s in tile gs = w % 2 (register r: t = 16 gm
  // + 4 g + r, s = 16 gs + L). Split form: both feed M, and through M the
  // outputs Y0 = M U0 and Q', where a row's output is often much smaller
  // than the terms that cancel in it, so a plain fp16 product (2^-11
  // relative per term) would show in rows of small RMS.
  const unsigned gm = wave >> 1, gs = wave & 1u;
  float4_t kk{0.0f, 0.0f, 0.0f, 0.0f}, qk{0.0f, 0.0f, 0.0f, 0.0f};
  {
    float4_t kx{0.0f, 0.0f, 0.0f, 0.0f}, qx{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int ks = 0; ks < KB; ++ks) {
      const unsigned bo = (16 * gs + L) * KS + 32 * ks + 8 * g;
      const unsigned ao = (16 * gm + L) * KS + 32 * ks + 8 * g;
      const half8_t bh = load8(sKh + bo), bl = load8(sKl + bo);
      const half8_t kah = load8(sKh + ao), kal = load8(sKl + ao);
      const half8_t qah = load8(sQV + ao), qal = load8(sQl + ao);
      kk = mfma16(kah, bh, kk);
      qk = mfma16(qah, bh, qk);
      kx = mfma16(kah, bl, kx);
      qx = mfma16(qah, bl, qx);
      kx = mfma16(kal, bh, kx);
      qx = mfma16(qal, bh, qx);
    }
    kk += kx * kSplitUnscale;
    qk += qx * kSplitUnscale;
  }

  for (unsigned hr = 0; hr < R; ++hr) {
    const unsigned h = kh * R + hr, pb = hr & 1u;
    char *const rec = rec_ptr(ws, recB, Hv, c, h);
    const double *const hG = sG[pb];
    const float *const hB = sB[pb], *const hEg = sEg[pb], *const hEz = sEz[pb];
    lds_sync(); // the previous head is done with every LDS buffer

    // A (fp32) and M (hi/lo) from the Gram registers:
    // A[t][s] = beta_t e^(g_t - g_s) k_t.k_s (s < t), M[t][s] = e^(g_t - g_s)
    // q_t.k_s (s <= t), zero above.
    // Branch-free: every operand is read, the masks are selects.
    {
      const unsigned s = 16 * gs + L;
      const double gsv = hG[s];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const unsigned t = 16 * gm + 4 * g + r;
        const float d = fminf((float)(hG[t] - gsv), 0.0f);
        const float e = s <= t ? __builtin_amdgcn_exp2f(d * kLog2e) : 0.0f;
        const float a = hB[t] * e * kk[r];
        sA[t * FS + s] = s < t ? a : 0.0f;
        split_f16(e * qk[r], sMh[t * CS + s], sMl[t * CS + s]);
      }
    }

    // T = (I + A)^-1 on 16x16 blocks. The diagonal blocks D_i = (I +
    // A_ii)^-1 by forward substitution on the waves that wrote A_ii (waves 0
    // and 3: they read only their own LDS writes, so no barrier), lane j <
    // 16 owning column j; D_i goes to sTT[s][t] = T[t][s] for the product
    // below, and straight into T_w^T[s][t] = beta_s e^(g_s) T[t][s] and
    // T_b^T[s][t] = beta_s T[t][s] (hi/lo), with the zeros of T_w^T / T_b^T
    // above the diagonal blocks (wave 3: s >= 16, t < 16).
    if ((wave == 0 || wave == 3) && lane < 16) {
      const unsigned j = lane, b0 = wave == 0 ? 0u : 16u;
      // Column-oriented: once col[u] is known it enters every later row's
      // sum. Each row's fma chain still runs over u in increasing order
      // (the bits of the row-by-row form), but the rows' chains are
      // independent, and the A values can be read well ahead of their use.
      float col[16], acc[16];
#pragma unroll
      for (int t = 0; t < 16; ++t)
        acc[t] = 0.0f;
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        col[u] = (unsigned)u == j ? 1.0f : ((unsigned)u > j ? -acc[u] : 0.0f);
#pragma unroll
        for (int t = u + 1; t < 16; ++t)
          acc[t] = fmaf(sA[(b0 + t) * FS + b0 + u], col[u], acc[t]);
      }
#pragma unroll
      for (int t = 0; t < 16; ++t)
        sTT[(b0 + j) * FS + b0 + t] = col[t];
      const unsigned s = b0 + j;
      const float bw = hB[s] * hEg[s], bb = hB[s];
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const float4_t tv{col[4 * q4], col[4 * q4 + 1], col[4 * q4 + 2], col[4 * q4 + 3]};
        half4_t wh, wl, bh, bl;
        split4(tv * bw, wh, wl);
        split4(tv * bb, bh, bl);
        const unsigned o = s * CS + b0 + 4 * q4;
        *reinterpret_cast<half4_t *>(sTwh + o) = wh;
        *reinterpret_cast<half4_t *>(sTwl + o) = wl;
        *reinterpret_cast<half4_t *>(sTbh + o) = bh;
        *reinterpret_cast<half4_t *>(sTbl + o) = bl;
        if (b0 == 16) {
          const half4_t z{0, 0, 0, 0};
          const unsigned oz = s * CS + 4 * q4;
          *reinterpret_cast<half4_t *>(sTwh + oz) = z;
          *reinterpret_cast<half4_t *>(sTwl + oz) = z;
          *reinterpret_cast<half4_t *>(sTbh + oz) = z;
          *reinterpret_cast<half4_t *>(sTbl + oz) = z;
        }
      }
    }
    lds_sync();
    // The block below the diagonal, T_10 = -D_1 A_10 D_0, on MFMA
    // (v_mfma_f32_16x16x16_f16, split form; its C layout is also its B
    // layout), on wave 0, into T_w^T / T_b^T directly. Meanwhile wave 1
    // prepares the next head's gates.
    if (wave == 0) {
      half4_t ah, al, bh, bl;
      // A_10[L][4g + e] and D_0[4g + e][L] = sTT[L][4g + e].
      load_split4(sA + (16 + L) * FS + 4 * g, 1, ah, al);
      load_split4(sTT + L * FS + 4 * g, 1, bh, bl);
      float4_t p{0.0f, 0.0f, 0.0f, 0.0f}, px{0.0f, 0.0f, 0.0f, 0.0f};
      p = mfma16k16(ah, bh, p);
      px = mfma16k16(ah, bl, px);
      px = mfma16k16(al, bh, px);
      half4_t ph, pl, dh, dl;
      split4(p + px * kSplitUnscale, ph, pl);
      // D_1[L][4g + e] = sTT[16 + 4g + e][16 + L].
      load_split4(sTT + (16 + 4 * g) * FS + 16 + L, FS, dh, dl);
      float4_t tt{0.0f, 0.0f, 0.0f, 0.0f}, tx{0.0f, 0.0f, 0.0f, 0.0f};
      tt = mfma16k16(dh, ph, tt);
      tx = mfma16k16(dh, pl, tx);
      tx = mfma16k16(dl, ph, tx);
      // Register r: T[16 + 4g + r][L], i.e. T_w^T / T_b^T row s = L at
      // columns 16 + 4g + r.
      const float4_t res = -(tt + tx * kSplitUnscale);
      const float bw = hB[L] * hEg[L], bb = hB[L];
      half4_t wh, wl, vh, vl;
      split4(res * bw, wh, wl);
      split4(res * bb, vh, vl);
      const unsigned o = L * CS + 16 + 4 * g;
      *reinterpret_cast<half4_t *>(sTwh + o) = wh;
      *reinterpret_cast<half4_t *>(sTwl + o) = wl;
      *reinterpret_cast<half4_t *>(sTbh + o) = vh;
      *reinterpret_cast<half4_t *>(sTbl + o) = vl;
    }
    if (hr + 1 < R) {
      gates(hr + 1);
      if (hr + 2 < R)
        load_gates(h + 2);
    }
    lds_sync();

    // N^T = T_w^T M^T (N = M T diag(beta e^g)); -N to LDS as [t][s] hi/lo.
    // Wave w: the tile of s rows 16 (w / 2) .. and t columns 16 (w % 2) ..
    {
      const unsigned st = wave >> 1, tt = wave & 1u;
      const half8_t ah = load8(sTwh + (16 * st + L) * CS + 8 * g);
      const half8_t al = load8(sTwl + (16 * st + L) * CS + 8 * g);
      const half8_t bh = load8(sMh + (16 * tt + L) * CS + 8 * g);
      const half8_t bl = load8(sMl + (16 * tt + L) * CS + 8 * g);
      float4_t acc{0.0f, 0.0f, 0.0f, 0.0f}, crs{0.0f, 0.0f, 0.0f, 0.0f};
      acc = mfma16(ah, bh, acc);
      crs = mfma16(ah, bl, crs);
      crs = mfma16(al, bh, crs);
      half4_t nh, nl;
      split4(-(acc + crs * kSplitUnscale), nh, nl);
      const unsigned o = (16 * tt + L) * CS + 16 * st + 4 * g;
      *reinterpret_cast<half4_t *>(sNh + o) = nh;
      *reinterpret_cast<half4_t *>(sNl + o) = nl;
    }
    lds_sync();

    // Wn and Q' pieces: W^T = K^T T_w^T and Q'^T = e^g Q^T - K^T N^T share
    // the K^T operand. Wave w writes the blocks (m, kb = w): tiles d = 2w,
    // 2w + 1 of the transposed products against the token tiles m.
    {
      half_t *const wp = reinterpret_cast<half_t *>(rec);
      half_t *const qp = reinterpret_cast<half_t *>(rec + kWnBytes);
      half8_t kah[2], kal[2]; // [d tile]
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        kah[hf] = read_kcol(sKh, KS, 0, 16 * (2 * wave + hf), g, L);
        kal[hf] = read_kcol(sKl, KS, 0, 16 * (2 * wave + hf), g, L);
      }
      half8_t b1h[TT], b1l[TT], b2h[TT], b2l[TT];
#pragma unroll
      for (int mt = 0; mt < TT; ++mt) {
        const unsigned t = 16 * mt + L;
        b1h[mt] = read_kcol(sTwh, CS, 0, 16 * mt, g, L);
        b1l[mt] = read_kcol(sTwl, CS, 0, 16 * mt, g, L);
        b2h[mt] = load8(sNh + t * CS + 8 * g);
        b2l[mt] = load8(sNl + t * CS + 8 * g);
      }
      float4_t wa[TT][2], wx[TT][2], qa[TT][2], qx[TT][2]; // [token tile][d tile]
#pragma unroll
      for (int mt = 0; mt < TT; ++mt)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          wa[mt][hf] = wx[mt][hf] = qx[mt][hf] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
          qa[mt][hf] = qinit[hf][mt] * hEg[16 * mt + L];
        }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int mt = 0; mt < TT; ++mt)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          wa[mt][hf] = mfma16(kah[hf], b1h[mt], wa[mt][hf]);
          qa[mt][hf] = mfma16(kah[hf], b2h[mt], qa[mt][hf]);
        }
#pragma unroll
      for (int mt = 0; mt < TT; ++mt)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          wx[mt][hf] = mfma16(kah[hf], b1l[mt], wx[mt][hf]);
          qx[mt][hf] = mfma16(kah[hf], b2l[mt], qx[mt][hf]);
        }
#pragma unroll
      for (int mt = 0; mt < TT; ++mt)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          wx[mt][hf] = mfma16(kal[hf], b1h[mt], wx[mt][hf]);
          qx[mt][hf] = mfma16(kal[hf], b2h[mt], qx[mt][hf]);
        }
#pragma unroll
      for (int mt = 0; mt < TT; ++mt) {
        const float ez = hEz[16 * mt + L];
        half8_t wh, wl, qh;
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            half_t a, b;
            split_f16(-ez * (wa[mt][hf][r] + wx[mt][hf][r] * kSplitUnscale), a, b);
            wh[4 * hf + r] = a;
            wl[4 * hf + r] = b;
            qh[4 * hf + r] = (half_t)(qa[mt][hf][r] + qx[mt][hf][r] * kSplitUnscale);
          }
        const unsigned o = (KB * mt + wave) * kBlk + 8 * lane;
        *reinterpret_cast<half8_t *>(wp + o) = wh;
        *reinterpret_cast<half8_t *>(wp + kWnBlocks * kBlk + o) = wl;
        *reinterpret_cast<half8_t *>(qp + o) = qh;
      }
    }

    // The T_b and M pieces: wave w writes T_b tile w (w < 2) or M tile w - 2,
    // hi and lo.
    {
      const unsigned mt = wave & 1u;
      half8_t hi, lo;
      if (wave < 2) {
        hi = read_kcol(sTbh, CS, 0, 16 * mt, g, L);
        lo = read_kcol(sTbl, CS, 0, 16 * mt, g, L);
      } else {
        const unsigned o = (16 * mt + L) * CS + 4 * g;
        hi = cat8(load4(sMh + o), load4(sMh + o + 16));
        lo = cat8(load4(sMl + o), load4(sMl + o + 16));
      }
      half8_t *const pc = reinterpret_cast<half8_t *>(rec + (wave < 2 ? kRecTb : kRecM));
      pc[mt * 64 + lane] = hi;
      pc[(TT + mt) * 64 + lane] = lo;
    }
  }
}

// --------------------------------------------------------------- scan

// The scan workgroup: 4 compute waves, one per SIMD, for one (value head,
// 16-column dv slice). Wave w owns rows [32 w, 32 w + 32) of the slice's
// state (C tiles 2w and 2w + 1, in its registers for the whole call).
// Per chunk:
//   1. every wave splits its state rows into the hi/lo B operand of k block
//      w and puts it in LDS; barrier X1; every wave reads the whole split S;
//   2. waves 1 and 2: Z_m = Z0_m + sum_kb Wn[m][kb] S[kb] for token tile
//      m = w / 2; waves 0 and 3: Y_m = Y0_m + sum_kb Q'[m][kb] S[kb];
//   3. Z_m, split, to LDS; barrier X2; every wave reads the split Z;
//   4. S_w <- e^(g_C) S_w + K^T[w] Z (the two C tiles of w).
// Z0 and Y0 come from LDS, where the fifth wave put them during the step
// before. Each compute wave loads exactly the operand blocks it multiplies
// (40 KB per workgroup and chunk in all), one chunk ahead, straight into
// its registers. The fifth wave also keeps those loads L2 hits: the pieces
// come from HBM / the MALL (the prep wrote them), so it reads one dword
// per 128-byte line of its workgroup's share of the record and K^T piece
// of chunk c + kWarmAhead (the slice workgroups of a value head share an
// XCD, and split the head's lines between them). Its loads count on its
// own vmcnt, so the compute waves' waits never cover them. No wave issues a global
// store inside the chunk loop -- the Y tiles go to an LDS stage that is
// written out every kStageChunks chunks and at the end -- so a wave's only
// outstanding vector-memory operations are those loads, which complete in
// order: the wait for one chunk's operands then never drains the next
// chunk's (with a store pending the compiler's wait would be vmcnt(0)).
constexpr int kStageChunks = 64;
constexpr int kAhead = 1;      // chunks of operands in flight in registers
constexpr int kWarmAhead = 4;  // chunks ahead that the warming wave reads
constexpr int kWarmSets = 8;   // its register sets (a touch is consumed kWarmSets chunks later)
constexpr int kScanThreads = 320;
static_assert(TT == 2, "two token tiles a chunk: two Z waves and two Y waves");

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
    const half_t *__restrict__ v, unsigned T, unsigned Hk, unsigned Hv, unsigned DV,
    const half_t *__restrict__ gate, const float *__restrict__ nweight, unsigned *cnt,
    float neps, unsigned spin) {
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
  const size_t recB = kRecBytes, vStride = (size_t)Hv * DV;
  void *const wsp = const_cast<void *>(ws);
  // Waves 1 and 2 compute the Z tiles 0 and 1, waves 0 and 3 the Y tiles
  // 0 and 1 (m is the token tile): wave 0 shares its SIMD with the fifth
  // wave, and a Y wave is off the chain.
  const bool zw = w == 1 || w == 2;
  const unsigned m = w >> 1;

  __shared__ half8_t sSx[2][KB][64]; // split S: [hi, lo][k block][lane]
  __shared__ half8_t sZx[2][64];     // split Z: [hi, lo][lane], tiles 0 | 1
  // Z0 and Y0 of the slice, from the fifth wave: [chunk parity][Z0 tile 0,
  // Z0 tile 1, Y0 tile 0, Y0 tile 1][lane], C layout.
  __shared__ float4_t sZY[2][2 * TT][64];
  __shared__ __attribute__((aligned(16))) half_t sVt[C * 24]; // its V rows, 24-half stride
  __shared__ __attribute__((aligned(16))) half_t sY[kStageChunks][C][16];

  // The operand blocks of wave w for one chunk.
  struct Ops {
    half8_t a[2][KB]; // Z waves: Wn blocks (m, kb) [hi, lo][kb]; Y waves: Q' blocks in a[0]
    half8_t kt[2][2]; // K^T blocks (tile 2w + i): [hi, lo][i]
    float eC;         // e^(g_C)
  };
  // The loads of one chunk's operands in three parts, which a step spreads
  // over its phases: issued in one burst, a workgroup's loads would hold
  // each wave at its load instructions until the CU's memory pipeline took
  // them (~57 bytes per cycle per CU from L2, measured), while its MFMAs
  // wait behind them.
  auto load_a = [&](unsigned c, Ops &d) __attribute__((always_inline)) {
    // The hi blocks (Wn or Q') through a selected pointer, the Wn lo blocks
    // under a branch: with stores to different fields in the two arms of one
    // branch, the optimiser merges them into a store through a selected
    // address, and the buffers then live in scratch memory.
    const char *r = rec_ptr(wsp, recB, Hv, c, h);
    const half8_t *p =
        reinterpret_cast<const half8_t *>(r + (zw ? 0 : kWnBytes)) + KB * m * 64 + lane;
#pragma unroll
    for (int b = 0; b < KB; ++b)
      d.a[0][b] = p[b * 64];
    if (zw) {
#pragma unroll
      for (int b = 0; b < KB; ++b)
        d.a[1][b] = p[(kWnBlocks + b) * 64];
    }
  };
  auto load_kt = [&](unsigned c, Ops &d) __attribute__((always_inline)) {
    const half8_t *pk =
        reinterpret_cast<const half8_t *>(kpiece_ptr(wsp, recB, chunks, Hv, Hk, c, kh)) +
        2 * w * 64 + lane;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      d.kt[0][i] = pk[i * 64];
      d.kt[1][i] = pk[(kKtBlocks + i) * 64];
    }
  };
  auto load_qz = [&](unsigned c, Ops &d) __attribute__((always_inline)) {
    d.eC = *reinterpret_cast<const float *>(rec_ptr(wsp, recB, Hv, c, h) + kRecScalars);
  };
  auto load_ops = [&](unsigned c, Ops &d) __attribute__((always_inline)) {
    load_a(c, d);
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
    // The fifth wave. (1) Z0 and Y0 of the slice, one chunk ahead of the
    // compute waves, into sZY: U0 = T_b V (V, 32 rows x 16 columns, staged
    // in LDS and read transposed as the B operand), Z0 = e^(g_C - g) U0, Y0
    // = M U0 with U0 as the B operand from its C-layout registers, in split
    // form as the other products. Chunk x's Z0/Y0 are written during step
    // x - 1, after that step's first barrier (the compute waves read parity
    // x % 2 of chunk x - 2 before that step's second barrier) and before
    // its own next barrier. (2) Warming: this workgroup's share of a chunk is
    // recPart bytes of each record and kPart bytes of the K^T piece; it
    // reads one dword per line of the first 16 KiB of the former and 8 KiB
    // of the latter (all of both at dv = 128). A touched value is consumed
    // kWarmSets chunks later (the loop is unrolled over the register sets),
    // long after it came, so the wave never waits on its loads.
    struct ZYOps {
      half8_t tb[2][TT], mm[2][TT]; // T_b and M blocks: [hi, lo][tile]
      uint4_t vr;                   // 8 halves of row lane / 2 of the slice's V
      float4_t ez[TT];              // e^(g_C - g_t) of the lane's C-layout rows
    };
    auto load_zy = [&](unsigned x, ZYOps &d) __attribute__((always_inline)) {
      const char *r = rec_ptr(wsp, recB, Hv, x, h);
      const half8_t *pt = reinterpret_cast<const half8_t *>(r + kRecTb) + lane;
      const half8_t *pm = reinterpret_cast<const half8_t *>(r + kRecM) + lane;
#pragma unroll
      for (int hl = 0; hl < 2; ++hl)
#pragma unroll
        for (int mt = 0; mt < TT; ++mt) {
          d.tb[hl][mt] = pt[(TT * hl + mt) * 64];
          d.mm[hl][mt] = pm[(TT * hl + mt) * 64];
        }
      const unsigned t = x * C + (lane >> 1);
      d.vr = t < T ? *reinterpret_cast<const uint4_t *>(v + (size_t)t * vStride + (size_t)h * DV +
                                                         16 * js + 8 * (lane & 1u))
                   : uint4_t{0, 0, 0, 0};
      const float4_t *pe = reinterpret_cast<const float4_t *>(r + kRecScalars) + 8 + g;
#pragma unroll
      for (int mt = 0; mt < TT; ++mt)
        d.ez[mt] = pe[4 * mt];
    };
    // In two parts, one per barrier interval of the step before chunk x:
    // U0 and Z0, then Y0 (U0 kept in registers between them).
    float4_t u[TT];
    auto compute_z0 = [&](unsigned x, const ZYOps &d) __attribute__((always_inline)) {
      *reinterpret_cast<uint4_t *>(sVt + (lane >> 1) * 24 + 8 * (lane & 1u)) = d.vr;
      const half8_t vb = read_kcol(sVt, 24, 0, 0, g, L); // V[8g + e][L]
#pragma unroll
      for (int mt = 0; mt < TT; ++mt) {
        float4_t ua{0.0f, 0.0f, 0.0f, 0.0f}, ux{0.0f, 0.0f, 0.0f, 0.0f};
        ua = mfma16(d.tb[0][mt], vb, ua);
        ux = mfma16(d.tb[1][mt], vb, ux);
        u[mt] = ua + ux * kSplitUnscale;
        sZY[x & 1u][mt][lane] = u[mt] * d.ez[mt];
      }
    };
    auto compute_y0 = [&](unsigned x, const ZYOps &d) __attribute__((always_inline)) {
      half8_t ubh, ubl;
      split8(u[0], u[1], ubh, ubl);
#pragma unroll
      for (int mt = 0; mt < TT; ++mt) {
        float4_t ya{0.0f, 0.0f, 0.0f, 0.0f}, yx{0.0f, 0.0f, 0.0f, 0.0f};
        ya = mfma16(d.mm[0][mt], ubh, ya);
        yx = mfma16(d.mm[0][mt], ubl, yx);
        yx = mfma16(d.mm[1][mt], ubh, yx);
        sZY[x & 1u][TT + mt][lane] = ya + yx * kSplitUnscale;
      }
    };
    ZYOps z0s, z1s; // chunk x's operands in set x % 2
    load_zy(0, z0s);
    load_zy(min(1u, last), z1s);
    compute_z0(0, z0s);
    compute_y0(0, z0s);
    load_zy(min(2u, last), z0s);
    const unsigned R = Hv / Hk;
    const size_t recPart = (recB + slices - 1) / slices;
    const size_t kShare = (size_t)R * slices;
    const size_t kPart = ((size_t)kKtBytes + kShare - 1) / kShare;
    const size_t kIdx = (size_t)(h % R) * slices + js;
    const size_t r0 = js * recPart, r1 = min(r0 + recPart, recB) - 4;
    const size_t k0 = kIdx * kPart, k1 = min(k0 + kPart, (size_t)kKtBytes) - 4;
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
    // Step x, between its two barriers: chunk x + 1's U0 and Z0 from set
    // (x + 1) % 2; after the second: its Y0, and the set then takes chunk
    // x + 3.
    auto next_z0 = [&](unsigned x, ZYOps &d) __attribute__((always_inline)) {
      if (x + 1 < chunks)
        compute_z0(x + 1, d);
    };
    auto next_y0 = [&](unsigned x, ZYOps &d) __attribute__((always_inline)) {
      if (x + 1 < chunks) {
        compute_y0(x + 1, d);
        load_zy(min(x + 3, last), d);
      }
    };
    static_assert(kWarmSets % 2 == 0, "the Z0/Y0 sets alternate inside the unrolled loop");
    unsigned c = 0;
    for (; c + kWarmSets <= chunks; c += kWarmSets) {
#pragma unroll
      for (int u = 0; u < kWarmSets; u += 2) {
        touch(min(c + u + kWarmAhead, last), tv[(u + kWarmAhead) % kWarmSets]);
        lds_sync(); // X1
        next_z0(c + u, z1s);
        lds_sync(); // X2
        next_y0(c + u, z1s);
        touch(min(c + u + 1 + kWarmAhead, last), tv[(u + 1 + kWarmAhead) % kWarmSets]);
        lds_sync(); // X1
        next_z0(c + u + 1, z0s);
        lds_sync(); // X2
        next_y0(c + u + 1, z0s);
      }
    }
    for (; c + 2 <= chunks; c += 2) {
      lds_sync(); // X1
      next_z0(c, z1s);
      lds_sync(); // X2
      next_y0(c, z1s);
      lds_sync(); // X1
      next_z0(c + 1, z0s);
      lds_sync(); // X2
      next_y0(c + 1, z0s);
    }
    if (c < chunks) {
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
  auto step = [&](unsigned c, const Ops &cur, Ops &dst) __attribute__((always_inline)) {
    const unsigned cn = min(c + kAhead, last);
    load_a(cn, dst);
    __builtin_amdgcn_sched_barrier(0);
    // 1. The split S, through LDS.
    {
      half8_t hi, lo;
      split8(S[0], S[1], hi, lo);
      sSx[0][w][lane] = hi;
      sSx[1][w][lane] = lo;
    }
    lds_sync(); // X1
    half8_t bh[KB], bl[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      bh[kb] = sSx[0][kb][lane];
      bl[kb] = sSx[1][kb][lane];
    }
    __builtin_amdgcn_sched_barrier(0);
    load_kt(cn, dst);
    __builtin_amdgcn_sched_barrier(0);
    // 2. Z or Y of token tile m (each MFMA issued two or three after the
    // one it depends on: a dependent 16x16x32 MFMA waits ~44 cycles, an
    // independent one issues every ~18). 3. The split Z tile (halves
    // 4 m .. 4 m + 3 of the k block), or the output tile to the stage.
    if (zw) {
      float4_t za = sZY[c & 1u][m][lane], zx{0.0f, 0.0f, 0.0f, 0.0f};
      float4_t zy{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        za = mfma16(cur.a[0][kb], bh[kb], za);
        zx = mfma16(cur.a[0][kb], bl[kb], zx);
        zy = mfma16(cur.a[1][kb], bh[kb], zy);
      }
      half4_t hi, lo;
      split4(za + (zx + zy) * kSplitUnscale, hi, lo);
      reinterpret_cast<half4_t *>(&sZx[0][lane])[m] = hi;
      reinterpret_cast<half4_t *>(&sZx[1][lane])[m] = lo;
    } else {
      float4_t ya = sZY[c & 1u][TT + m][lane], yb{0.0f, 0.0f, 0.0f, 0.0f};
      float4_t yx{0.0f, 0.0f, 0.0f, 0.0f}, yz{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int kb = 0; kb < KB; kb += 2) {
        ya = mfma16(cur.a[0][kb], bh[kb], ya);
        yb = mfma16(cur.a[0][kb + 1], bh[kb + 1], yb);
        yx = mfma16(cur.a[0][kb], bl[kb], yx);
        yz = mfma16(cur.a[0][kb + 1], bl[kb + 1], yz);
      }
      const float4_t y = (ya + yb) + (yx + yz) * kSplitUnscale;
      half_t *const sy = &sY[c % kStageChunks][16 * m + 4 * g][L];
#pragma unroll
      for (int r = 0; r < 4; ++r)
        sy[16 * r] = (half_t)y[r];
    }
    lds_sync(); // X2
    const half8_t zh = sZx[0][lane], zl = sZx[1][lane];
    __builtin_amdgcn_sched_barrier(0);
    load_qz(cn, dst);
    __builtin_amdgcn_sched_barrier(0);
    // 4. S_w <- e^(g_C) S_w + K^T Z (both cross terms in one accumulator).
    float4_t sa[2], sx[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      sa[i] = mfma16(cur.kt[0][i], zh, S[i] * cur.eC);
      sx[i] = mfma16(cur.kt[0][i], zl, float4_t{0.0f, 0.0f, 0.0f, 0.0f});
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
      sx[i] = mfma16(cur.kt[1][i], zh, sx[i]);
#pragma unroll
    for (int i = 0; i < 2; ++i)
      S[i] = sa[i] + sx[i] * kSplitUnscale;
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
  return chunks * (s.Hv * kRecBytes + s.Hk * (size_t)kKtBytes);
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
                     beta, decay, ws, s.T, s.Hk, s.Hv, s.Dv, eps, qscale, cnt);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return e;
  const dim3 grid(s.Hv * (s.Dv / 16));
  if (!gate) {
    hipLaunchKernelGGL(delta_scan_kernel<false>, grid, dim3(kScanThreads), 0, stream, state,
                       reinterpret_cast<half_t *>(out), ws, reinterpret_cast<const half_t *>(v),
                       s.T, s.Hk, s.Hv, s.Dv,
                       (const half_t *)nullptr, (const float *)nullptr, (unsigned *)nullptr,
                       0.0f, 0u);
    return hipGetLastError();
  }
  // The norm's arrival wait needs every slice workgroup of a value head
  // resident at once: delta_chunked_norm_resident() checked that the whole
  // grid fits on the device together (a cooperative launch would guarantee
  // it too, but costs ~17 us more per call here, measured).
  hipLaunchKernelGGL(delta_scan_kernel<true>, grid, dim3(kScanThreads), 0, stream, state,
                     reinterpret_cast<half_t *>(out), ws, reinterpret_cast<const half_t *>(v),
                     s.T, s.Hk, s.Hv, s.Dv,
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
