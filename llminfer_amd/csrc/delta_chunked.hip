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
//  * deltaChunkScan, grid (value head, 16-column dv slice), 4 waves: one
//    walks the chunks in order with its state slice S [dk x 16] in
//    registers, one computes the outputs, two load. Every product runs on
//    v_mfma_f32_16x16x32_f16, with the state (and Z) as the B operand
//    straight from the C-layout registers of the product that made it: the k
//    index of an operand block is permuted (sigma below) so that the 8 halves
//    a lane supplies are the 8 rows it holds in two consecutive 16-row C
//    tiles; the A operands (Wn, Q', K^T) were written by the prep with the
//    same permutation. No LDS round trip and no shuffle on the chain. The
//    next chunk's Wn and K^T stream HBM/L2 -> LDS (buffer_load ... lds) while
//    the current chunk computes; the chain wave reads them from LDS with one
//    16-byte read per lane and block.
//
// Split form: x = hi + lo 2^-11 with hi = fp16(x), lo = fp16((x - hi) 2^11),
// a.b ~ ah.bh + (ah.bl + al.bh) 2^-11, the cross terms in a second fp32
// accumulator -- 22 significant bits per operand. A plain fp16 product
// leaves the fp32 state ~8e-4 relative off the recurrence after 1024 tokens;
// the split form ~1e-5, well inside the 1e-3 bound. The Gram matrices only
// feed T and M and stay plain fp16.
//
// Decays are linear at the op boundary (Graph.metal:143). The cumulative
// log decay is summed, and differenced, in double: log(0) is clamped to -1e4
// (e^-1e4 = 0), and in fp32 a difference of two sums near -1e4 would keep
// only ~1e-3 absolute precision. Only non-positive differences are
// exponentiated.
#include "exact_fp.hpp"
#include "hip_common.hpp"
#include "kernels.hpp"

#include "capi_internal.hpp"

#include <math.h>

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
constexpr int kPieceLoads = kPieceBytes / 1024;    // 16-byte-per-lane loads of a piece
constexpr int kBufferWord3 = 0x00020000;           // gfx9 raw buffer descriptor, dword 3
typedef __attribute__((address_space(3))) void lds_void_t;

// Workspace. Per (chunk, value head) a record: the Wn piece, the Q' piece,
// then Z0 and Y0 as fp32 in C-layout register order, per 16-column slice js
// and 16-row tile m a 64-lane block of float4 (block 4 js + m), then 64
// floats of scalars (e^(g_C) first). After all records, per (chunk, key
// head) the K^T piece.
constexpr int kScalarBytes = 256;
__host__ __device__ inline size_t rec_bytes(unsigned DV) {
  return 2 * (size_t)kPieceBytes + 2 * (size_t)C * DV * sizeof(float) + kScalarBytes;
}
__host__ __device__ inline size_t rec_scalars(unsigned DV) {
  return 2 * (size_t)kPieceBytes + 2 * (size_t)C * DV * sizeof(float);
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
    unsigned T, unsigned Hk, unsigned Hv, unsigned DV, float eps, float qscale) {
  const float *q = static_cast<const float *>(qp), *k = static_cast<const float *>(kp);
  const half_t *q16 = static_cast<const half_t *>(qp), *k16 = static_cast<const half_t *>(kp);
  const unsigned c = blockIdx.x, kh = blockIdx.y;
  const unsigned R = Hv / Hk, chunks = (T + C - 1) / C;
  const unsigned t0 = c * C, n = min((unsigned)C, T - t0);
  const unsigned tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const unsigned g = lane >> 4, L = lane & 15u;
  const size_t recB = rec_bytes(DV);
  const size_t qkStride = (size_t)Hk * DK, vStride = (size_t)Hv * DV;

  __shared__ __attribute__((aligned(16))) half_t sKh[C * KS], sKl[C * KS];
  __shared__ __attribute__((aligned(16))) half_t sQV[C * KS]; // Q hi, later a V block
  __shared__ float sA[C * FS], sTT[C * FS];                   // A and T^T (fp32)
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
    __syncthreads();
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
    }
  }
  __syncthreads();

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

  // K K^T and Q K^T (fp16 hi) stay in registers: wave w holds the tiles of
  // key columns s in [16 w, 16 w + 16) for the four row tiles (register r
  // of tile mt: t = 16 mt + 4 g + r, s = 16 w + L).
  float4_t kk[4], qk[4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    kk[mt] = qk[mt] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int ks = 0; ks < DK / 32; ++ks) {
      const half8_t b = load8(sKh + (16 * wave + L) * KS + 32 * ks + 8 * g);
      kk[mt] = mfma16(load8(sKh + (16 * mt + L) * KS + 32 * ks + 8 * g), b, kk[mt]);
      qk[mt] = mfma16(load8(sQV + (16 * mt + L) * KS + 32 * ks + 8 * g), b, qk[mt]);
    }
  }

  for (unsigned hr = 0; hr < R; ++hr) {
    const unsigned h = kh * R + hr;
    char *const rec = rec_ptr(ws, recB, Hv, c, h);
    __syncthreads(); // the previous head is done with every LDS buffer

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
    __syncthreads();

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
    __syncthreads();

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
    __syncthreads();
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
      __syncthreads();
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
    __syncthreads();

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
    __syncthreads();

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
          half8_t wh, wl, qh, ql;
#pragma unroll
          for (int hf = 0; hf < 2; ++hf)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              half_t a, b;
              split_f16(-ez * (wa[u][hf][r] + wx[u][hf][r] * kSplitUnscale), a, b);
              wh[4 * hf + r] = a;
              wl[4 * hf + r] = b;
              split_f16(qa[u][hf][r] + qx[u][hf][r] * kSplitUnscale, a, b);
              qh[4 * hf + r] = a;
              ql[4 * hf + r] = b;
            }
          const unsigned o = (4 * mt + wave) * kBlk + 8 * lane;
          *reinterpret_cast<half8_t *>(wp + o) = wh;
          *reinterpret_cast<half8_t *>(wp + kPieceBlocks * kBlk + o) = wl;
          *reinterpret_cast<half8_t *>(qp + o) = qh;
          *reinterpret_cast<half8_t *>(qp + kPieceBlocks * kBlk + o) = ql;
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
      float4_t *const z0 = reinterpret_cast<float4_t *>(rec + 2 * kPieceBytes);
      float4_t *const y0 = z0 + (size_t)C * DV / 4;
      for (unsigned jb = 0; jb < DV; jb += VB) {
        const unsigned w = min((unsigned)VB, DV - jb);
        if (jb > 0) {
          // Further dv blocks (DV > VB) are fetched here, in turn.
          fetch_v(h, jb, w);
          __syncthreads();
          store_v(w);
          __syncthreads();
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

// Direct HBM/L2 -> LDS loads (buffer_load_dwordx4 ... lds), issued from
// inline assembly so that the compiler neither waits for them nor reorders
// LDS accesses across them ("memory" clobber): the scan orders them itself.
// Each load moves 16 bytes per lane, lane i's bytes landing at M0 + 16 i.
typedef __attribute__((address_space(3))) char lds_char_t;
typedef int int4v_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int4v_t buffer_rsrc(const void *base, unsigned bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  return int4v_t{__builtin_amdgcn_readfirstlane((int)(uint32_t)a),
                 __builtin_amdgcn_readfirstlane((int)((uint32_t)(a >> 32) & 0xFFFFu)),
                 (int)bytes, kBufferWord3};
}
__device__ __forceinline__ unsigned lds_addr(const void *p) {
  return (unsigned)(uintptr_t)(const lds_char_t *)p;
}
// M0 is reserved to the compiler; it keeps nothing in it across these
// statements in this file, and the clobber tells it M0 changes.
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void load_lds_1k(int4v_t rsrc, unsigned ldsDst, unsigned voff,
                                            unsigned soff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(__builtin_amdgcn_readfirstlane(ldsDst)), "v"(voff), "s"(rsrc),
                 "s"(__builtin_amdgcn_readfirstlane(soff))
               : "memory", "m0");
}
__device__ __forceinline__ void load_lds_256(int4v_t rsrc, unsigned ldsDst, unsigned voff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, 0 offen lds"
               :
               : "s"(__builtin_amdgcn_readfirstlane(ldsDst)), "v"(voff), "s"(rsrc)
               : "memory", "m0");
}
// Wait until this wave's LDS reads have returned (before a barrier after
// which their buffer is reloaded).
__device__ __forceinline__ void wait_lds_reads() { __builtin_amdgcn_s_waitcnt(0xC07F); }
// Wait until at most N of this wave's vector-memory operations are
// outstanding (they complete in order).
template <int N> __device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}
// Workgroup barrier that the compiler moves no memory access across; no
// wait attached (each wave waits for exactly what it must beforehand).
__device__ __forceinline__ void barrier() { asm volatile("s_barrier" ::: "memory"); }

// The scan workgroup, 4 waves on the 4 SIMDs of one CU:
//   wave 0 (chain): the state recursion Z = Z0 + Wn S, S <- e^(g_C) S + K^T Z;
//   wave 1 (output): Y = Y0 + Q' S from the split S that wave 0 leaves in
//           LDS, with Q' and Y0 loaded straight into its registers;
//   waves 2-3 (loaders): the Wn, K^T pieces and Z0 (+ scalars) of the next
//           chunk, direct to LDS, double-buffered.
// A wave moves at most ~16 bytes per cycle through direct-to-LDS loads
// (measured: ~38 GB/s per wave whether the data sits in L2 or in HBM,
// scaling with the number of waves), so the chain wave issues none.
constexpr int kLoaders = 2;
constexpr int kPartLoads = kPieceLoads / kLoaders;  // 16 KiB of a piece per loader
constexpr int kZLoads = 4 / kLoaders + 1;            // Z0 blocks + the scalars
constexpr int kWLoads = kPartLoads + kZLoads;

__global__ __launch_bounds__(256, 1) void delta_scan_kernel(
    float *__restrict__ state, half_t *__restrict__ out, const void *__restrict__ ws,
    unsigned T, unsigned Hk, unsigned Hv, unsigned DV) {
  // Workgroups are dealt to the 8 XCDs round-robin by block index. Give
  // each XCD a contiguous run of (value head, slice) pairs, so that the
  // workgroups reading one value head's pieces and one key head's K^T piece
  // share an L2.
  const unsigned slices = DV / 16, nb = gridDim.x;
  const unsigned Lb = nb % 8 == 0 ? (blockIdx.x % 8) * (nb / 8) + blockIdx.x / 8 : blockIdx.x;
  const unsigned h = Lb / slices, js = Lb % slices, kh = h / (Hv / Hk);
  const unsigned wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const unsigned lane = threadIdx.x & 63u, g = lane >> 4;
  const unsigned chunks = (T + C - 1) / C, last = chunks - 1;
  const size_t recB = rec_bytes(DV), vStride = (size_t)Hv * DV;
  void *const wsp = const_cast<void *>(ws);

  // Chunk c uses buffer c % 2 of Wn, K^T and Z0; sS holds the split S of
  // the current chunk for wave 1.
  constexpr int PB = 2 * kPieceBlocks * 64; // half8s per piece
  __shared__ half8_t sW0[PB], sW1[PB], sK0[PB], sK1[PB];
  __shared__ float4_t sZ0[4 * 64 + 16], sZ1[4 * 64 + 16]; // Z0 blocks, scalars
  __shared__ half8_t sS[8 * 64];                           // bh[4], bl[4]

  auto rec = [&](unsigned c) { return rec_ptr(wsp, recB, Hv, c, h); };
  auto kp = [&](unsigned c) { return kpiece_ptr(wsp, recB, chunks, Hv, Hk, c, kh); };
  const unsigned j = 16 * js + (lane & 15u);

  // Per chunk c, barriers A(c) then B(c):
  //   A(c): Wn, Z0 of c landed (buffer c % 2); wave 1 has read the previous
  //         split S; the buffers of chunk c - 1 are free.
  //   B(c): K^T of c landed; wave 0 has written this chunk's split S.
  if (wave >= 2) {
    const unsigned l = wave - 2;
    auto load_part = [&](const char *src, const half8_t *dst) {
      const int4v_t rsrc = buffer_rsrc(src, kPieceBytes);
#pragma unroll
      for (int it = 0; it < kPartLoads; ++it) {
        const unsigned kib = kPartLoads * l + it;
        load_lds_1k(rsrc, lds_addr(dst) + 1024 * kib, 16 * lane, 1024 * kib);
      }
    };
    auto load_w = [&](unsigned c, const half8_t *dW, const float4_t *dZ) {
      const char *r = rec(c);
      load_part(r, dW);
      const char *z = r + 2 * kPieceBytes + (size_t)js * 4 * 64 * sizeof(float4_t);
      const int4v_t rz = buffer_rsrc(z, 4 * 1024);
#pragma unroll
      for (int i = 0; i < kZLoads - 1; ++i) {
        const unsigned blk = (kZLoads - 1) * l + i;
        load_lds_1k(rz, lds_addr(dZ + 64 * blk), 16 * lane, 1024 * blk);
      }
      load_lds_256(buffer_rsrc(r + rec_scalars(DV), kScalarBytes), lds_addr(dZ + 4 * 64),
                   4 * lane);
    };
    load_w(0, sW0, sZ0);
    load_part(kp(0), sK0);
    wait_vm<kPartLoads>(); // Wn, Z0 of 0
    for (unsigned c = 0; c < chunks; ++c) {
      barrier(); // A(c)
      const unsigned cn = min(c + 1, last);
      if (c % 2 == 0) {
        load_w(cn, sW1, sZ1);
        load_part(kp(cn), sK1);
      } else {
        load_w(cn, sW0, sZ0);
        load_part(kp(cn), sK0);
      }
      wait_vm<kWLoads + kPartLoads>(); // K^T of c
      barrier(); // B(c)
      wait_vm<kPartLoads>(); // Wn, Z0 of c + 1
    }
    wait_vm<0>();
    return;
  }

  if (wave == 1) {
    // Q' (32 blocks) and Y0 (4 blocks) of a chunk, into registers.
    struct QY {
      half8_t q[2][kPieceBlocks];
      float4_t y[4];
    };
    auto load_qy = [&](unsigned c, QY &d) {
      const char *r = rec(c);
      const half8_t *qp = reinterpret_cast<const half8_t *>(r + kPieceBytes) + lane;
#pragma unroll
      for (int b = 0; b < kPieceBlocks; ++b) {
        d.q[0][b] = qp[b * 64];
        d.q[1][b] = qp[(kPieceBlocks + b) * 64];
      }
      const float4_t *yp = reinterpret_cast<const float4_t *>(r + 2 * kPieceBytes) +
                           (size_t)C * DV / 4 + js * 4 * 64 + lane;
#pragma unroll
      for (int m = 0; m < 4; ++m)
        d.y[m] = yp[m * 64];
    };
    auto ystep = [&](unsigned c, const QY &cur, QY &nxt) {
      const unsigned t0 = c * C, n = min((unsigned)C, T - t0);
      barrier(); // A(c)
      barrier(); // B(c)
      half8_t bh[4], bl[4];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        bh[kb] = sS[kb * 64 + lane];
        bl[kb] = sS[(4 + kb) * 64 + lane];
      }
      wait_lds_reads();
      load_qy(min(c + 1, last), nxt);
      float4_t ya[4], yx[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        ya[m] = cur.y[m];
        yx[m] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
      }
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
        for (int m = 0; m < 4; ++m)
          ya[m] = mfma16(cur.q[0][4 * m + kb], bh[kb], ya[m]);
#pragma unroll
        for (int m = 0; m < 4; ++m)
          yx[m] = mfma16(cur.q[0][4 * m + kb], bl[kb], yx[m]);
#pragma unroll
        for (int m = 0; m < 4; ++m)
          yx[m] = mfma16(cur.q[1][4 * m + kb], bh[kb], yx[m]);
      }
      // Rows past the end of the tokens fall outside the descriptor and
      // are dropped by the buffer stores.
      const auto ro = __builtin_amdgcn_make_buffer_rsrc(
          (void *)(out + (size_t)t0 * vStride + (size_t)h * DV), (short)0,
          (int)(((n - 1) * vStride + DV) * sizeof(half_t)), kBufferWord3);
#pragma unroll
      for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const unsigned t = 16 * m + 4 * g + r;
          const half_t y = (half_t)(ya[m][r] + yx[m][r] * kSplitUnscale);
          __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, y), ro,
                                                (unsigned)((t * vStride + j) * sizeof(half_t)),
                                                0, 0);
        }
    };
    QY qa, qb;
    load_qy(0, qa);
    unsigned c = 0;
    for (; c + 1 < chunks; c += 2) {
      ystep(c, qa, qb);
      ystep(c + 1, qb, qa);
    }
    if (c < chunks)
      ystep(c, qa, qb);
    return;
  }

  // Wave 0: the state slice, register r of tile i holding S[16 i + 4 g + r][j].
  float4_t S[8];
  float *const scol = state + (size_t)h * DK * DV + j;
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      S[i][r] = scol[(size_t)(16 * i + 4 * g + r) * DV];

  auto step = [&](unsigned c, const half8_t *rW, const float4_t *rZ, const half8_t *rK) {
    barrier(); // A(c)
    // All of a product's A blocks are read before its first MFMA (the
    // scheduler is kept from sinking the reads next to their uses, where
    // each would expose the LDS latency), and the MFMAs of one k block go
    // accumulator by accumulator so that no MFMA waits on the one before
    // (a dependent 16x16x32 MFMA waits ~44 cycles, an independent one
    // issues every ~18).
    half8_t A[2][kPieceBlocks];
#pragma unroll
    for (int b = 0; b < kPieceBlocks; ++b) {
      A[0][b] = rW[b * 64 + lane];
      A[1][b] = rW[(kPieceBlocks + b) * 64 + lane];
    }
    const float eC = rZ[4 * 64][0];
    float4_t za[4], zx[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      za[m] = rZ[m * 64 + lane];
      zx[m] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
    }
    // S as the B operand of its four 32-row k blocks, also left for wave 1.
    half8_t bh[4], bl[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      split8(S[2 * kb], S[2 * kb + 1], bh[kb], bl[kb]);
      sS[kb * 64 + lane] = bh[kb];
      sS[(4 + kb) * 64 + lane] = bl[kb];
    }
    __builtin_amdgcn_sched_barrier(0);
    // Z = Z0 + Wn S.
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
      for (int m = 0; m < 4; ++m)
        za[m] = mfma16(A[0][4 * m + kb], bh[kb], za[m]);
#pragma unroll
      for (int m = 0; m < 4; ++m)
        zx[m] = mfma16(A[0][4 * m + kb], bl[kb], zx[m]);
#pragma unroll
      for (int m = 0; m < 4; ++m)
        zx[m] = mfma16(A[1][4 * m + kb], bh[kb], zx[m]);
    }
    wait_lds_reads();
    barrier(); // B(c)

    // S <- e^(g_C) S + K^T Z, Z as the B operand of its two k blocks.
#pragma unroll
    for (int b = 0; b < kPieceBlocks; ++b) {
      A[0][b] = rK[b * 64 + lane];
      A[1][b] = rK[(kPieceBlocks + b) * 64 + lane];
    }
    half8_t zbh[2], zbl[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
      split8(za[2 * kb] + zx[2 * kb] * kSplitUnscale,
             za[2 * kb + 1] + zx[2 * kb + 1] * kSplitUnscale, zbh[kb], zbl[kb]);
    float4_t sa[8], sx[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      sa[i] = S[i] * eC;
      sx[i] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        sa[i] = mfma16(A[0][2 * i + kb], zbh[kb], sa[i]);
#pragma unroll
      for (int i = 0; i < 8; ++i)
        sx[i] = mfma16(A[0][2 * i + kb], zbl[kb], sx[i]);
#pragma unroll
      for (int i = 0; i < 8; ++i)
        sx[i] = mfma16(A[1][2 * i + kb], zbh[kb], sx[i]);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
      S[i] = sa[i] + sx[i] * kSplitUnscale;
    wait_lds_reads();
  };

  unsigned c = 0;
  for (; c + 1 < chunks; c += 2) {
    step(c, sW0, sZ0, sK0);
    step(c + 1, sW1, sZ1, sK1);
  }
  if (c < chunks)
    step(c, sW0, sZ0, sK0);

#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      scol[(size_t)(16 * i + 4 * g + r) * DV] = S[i][r];
}

} // namespace

bool delta_chunked_supported(const DeltaShape &s) {
  return s.Dk == DK && s.Dv % 16 == 0 && s.Dv >= 16 && s.Hk >= 1 && s.Hv % s.Hk == 0 &&
         s.T >= 32;
}

size_t delta_chunked_workspace_bytes(const DeltaShape &s) {
  const size_t chunks = (s.T + C - 1) / C;
  return chunks * (s.Hv * rec_bytes(s.Dv) + s.Hk * (size_t)kPieceBytes);
}

namespace {

template <bool QK16>
hipError_t launch_chunked(const void *q, const void *k, const uint16_t *v, const float *beta,
                          const float *decay, float *state, uint16_t *out, void *ws,
                          float eps, float qscale, const DeltaShape &s, hipStream_t stream) {
  const unsigned chunks = (s.T + C - 1) / C;
  hipLaunchKernelGGL((delta_prep_kernel<QK16>), dim3(chunks, s.Hk), dim3(256), 0, stream, q, k,
                     reinterpret_cast<const half_t *>(v), beta, decay, ws, s.T, s.Hk, s.Hv,
                     s.Dv, eps, qscale);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return e;
  hipLaunchKernelGGL(delta_scan_kernel, dim3(s.Hv * (s.Dv / 16)), dim3(256), 0, stream, state,
                     reinterpret_cast<half_t *>(out), ws, s.T, s.Hk, s.Hv, s.Dv);
  return hipGetLastError();
}

} // namespace

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

unsigned delta_chunked_dispatches() { return 2; }

const char *delta_chunked_kernel_name(unsigned index) {
  return index == 0 ? "deltaChunkPrep" : "deltaChunkScan";
}

} // namespace llmi
