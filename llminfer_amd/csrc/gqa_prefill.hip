// Causal GQA prefill (flash attention) on fp16 MFMA for gfx950.
//
// Replaces gqaFlashAttention (FlashAttention.metal:1-83), which runs one query
// per SIMD group with a scalar per-key reduction. Here:
//
//  * one workgroup = (block of 32 query tokens, KV head, HW query heads of
//    that head's group); wave w computes query head kvh*G + grp*HW + w for the
//    32 tokens, so the waves share every K/V tile staged in LDS.
//  * K/V tiles of 64 keys go HBM -> LDS with buffer loads that write LDS
//    directly (no register staging), double-buffered: tile i+1 is in flight
//    while tile i is consumed. The buffer descriptor's range ends at the
//    block's last visible key, so rows past it read as zero without any
//    per-lane clamping.
//  * LDS rows are XOR-swizzled in 16-byte chunks so the MFMA operand reads
//    are free of bank conflicts: K chunk c of row j sits at c ^ (j % 8), V
//    chunk c of row j at c ^ 2(j % 4).
//  * scores are computed transposed, S^T = K Q^T, with
//    v_mfma_f32_32x32x16_f16: each lane owns one query row (lane % 32) and 32
//    of the tile's keys; the row max needs one exchange with lane ^ 32.
//  * O^T += V^T P^T on the same MFMA; its V^T operand comes straight from
//    the row-major V tile through ds_read_b64_tr_b16 (transposing LDS read),
//    and P^T is the probability tile converted to fp16 in registers.
//  * softmax with a lazily moved reference: probabilities are
//    exp2(s*c - m) with m only raised when a row's maximum would push a
//    probability past 2^15 (then m = max - 7). O and l are rescaled only on
//    such a raise, which after the first tiles is rare; probabilities stay
//    <= 2^15 (fp16-safe) and at least 2^-14 down to 21 binades below the
//    row maximum, so the MFMA sees no fp16 subnormals where they matter.
//  * PV of tile i-1 is issued after the scores of tile i, so its MFMAs
//    overlap the softmax arithmetic of tile i.
//
// At head_dim 256 with four query heads per KV head, grids of 64 workgroups
// or more run gqa_prefill_halves_kernel instead: the single-wave kernel
// needs ~500 registers per lane, one wave per SIMD, and a lone wave cannot
// hide its LDS operand reads behind its MFMAs (measured on gfx950: 55-60
// cycles per 32x32x16 MFMA with a 1 KB operand read each, against 38 with a
// second wave on the SIMD and the reads two MFMAs ahead). The key-split
// kernel gives each head a wave pair that splits the keys, at 248 registers.
#include "hip_common.hpp"
#include "kernels.hpp"
#include "rope_gate.hpp"

#include <math.h>
#include <stdlib.h>
#include <type_traits>

namespace llmi {
namespace {

constexpr int BM = 32;            // query tokens per wave (= MFMA N)
constexpr int BN = 64;            // keys per tile
constexpr int kBufferWord3 = 0x00020000; // gfx9 raw buffer descriptor, dword 3
constexpr float kRaise = 15.0f;   // raise m when a probability would exceed 2^15
constexpr float kHeadroom = 7.0f; // after a raise the largest probability is 2^7

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __fp16 fp16x4_t __attribute__((__vector_size__(4 * sizeof(__fp16))));
typedef __attribute__((address_space(3))) fp16x4_t lds_fp16x4_t;

// Direct HBM -> LDS load of 16 bytes per lane: lane i's bytes land at
// dst + 16 i (dst is wave-uniform).
__device__ __forceinline__ void load_lds16(__amdgpu_buffer_rsrc_t rsrc, char *dst,
                                           unsigned voffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void_t *)dst, 16, voffset, 0, 0, 0);
}

// Hides a value's known bit range from the compiler, so that adding a
// constant to it stays an add (folded into the LDS instruction's offset
// field) instead of becoming an OR of disjoint bits computed on the VALU.
__device__ __forceinline__ void opaque(unsigned &x) { asm volatile("" : "+v"(x)); }

__device__ __forceinline__ void wait_loads() {
  __builtin_amdgcn_s_waitcnt(0x0F70); // vmcnt(0)
}

// ds_read_b64_tr_b16: in each 16-lane group, lane j receives element j % 4 of
// the 8-byte chunks addressed by lanes j/4, 4 + j/4, 8 + j/4, 12 + j/4.
__device__ __forceinline__ half4_t read_tr(const char *base, unsigned off) {
  typedef __attribute__((address_space(3))) char lds_char_t;
  return __builtin_bit_cast(half4_t, __builtin_amdgcn_ds_read_tr16_b64_v4f16(
                                         (lds_fp16x4_t *)((lds_char_t *)base + off)));
}

// The sigmoid gate of one lane's 16 outputs of a 32-channel tile (the
// four half4 groups at g + 8 i): the fast logistic first, then the exact one
// for the few that miss the margin test, one per pass of the wave (as the
// standalone gate kernel does). activated: the gate values are already
// fp16(logistic(.)), and the output is their plain product (multiplyF16).
__device__ __forceinline__ void gate_tile(half4_t (&v)[4], const half_t *g4p, bool activated) {
  float g[16], sg[16];
  unsigned need = 0;
#pragma unroll
  for (int g4 = 0; g4 < 4; ++g4) {
    const half4_t gv = *reinterpret_cast<const half4_t *>(g4p + 8 * g4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      g[4 * g4 + e] = (float)gv[e];
      sg[4 * g4 + e] = activated ? g[4 * g4 + e] : logistic_estimate(g[4 * g4 + e]);
      need |= activated || f16_settled(sg[4 * g4 + e]) ? 0u : 1u << (4 * g4 + e);
    }
  }
  while (need) {
    const unsigned k = __builtin_ctz(need);
    need &= need - 1;
    float gk = g[0];
#pragma unroll
    for (int e = 1; e < 16; ++e)
      gk = k == (unsigned)e ? g[e] : gk;
    const float sk = logistic_exact(gk);
#pragma unroll
    for (int e = 0; e < 16; ++e)
      sg[e] = k == (unsigned)e ? sk : sg[e];
  }
#pragma unroll
  for (int g4 = 0; g4 < 4; ++g4)
#pragma unroll
    for (int e = 0; e < 4; ++e)
      v[g4][e] = __builtin_bit_cast(half_t, f2h(mul32(round16(sg[4 * g4 + e]), (float)v[g4][e])));
}

struct NoRows {}; // the ungated kernel's (empty) row argument

// GATED: the query rows come from the projected q (per head D query values,
// then D gate values) through normRope, staged in the K/V buffers before
// the keys need them, and the output goes through the sigmoid gate: the
// bits of the standalone normRope and sigmoidMul (rope_gate.hpp) around the
// same attention.
template <int D, int HW, bool GATED>
__global__ __attribute__((amdgpu_flat_work_group_size(64 * HW, 64 * HW),
                          amdgpu_waves_per_eu(HW > 4 ? 2 : 1, HW > 4 ? 2 : 1)))
void gqa_prefill_kernel(const half_t *__restrict__ q, const half_t *__restrict__ kc,
                        const half_t *__restrict__ vc, half_t *__restrict__ out,
                        unsigned T, unsigned Hq, unsigned Hkv, unsigned P,
                        unsigned groups, unsigned nb, float c,
                        typename std::conditional<GATED, GatedRows, NoRows>::type ga) {
  constexpr int KS = D / 16;         // k-steps of S^T over channels
  constexpr int DT = D / 32;         // 32-channel output tiles
  constexpr int ROWB = 2 * D;        // bytes per K/V row
  constexpr int TILEB = BN * ROWB;   // bytes per K or V tile
  constexpr int NIW = TILEB / 1024 / HW; // 1-KB LDS loads per wave per tile
  constexpr int CPR = D / 8;         // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;      // rows per 1-KB load
  static_assert(NIW >= 1 && TILEB % (1024 * HW) == 0, "tile/waves");
  // V is staged transposed (V^T rows of BN keys, padded) when one pass of
  // the workgroup's threads covers the tile in (8-key run, 8-channel) units;
  // smaller workgroups read V with the transposing LDS read instead.
  constexpr int VUNITS = (BN / 8) * (D / 8);
  constexpr bool kStagedV = VUNITS <= 64 * HW;
  constexpr int VTROW = 2 * BN;       // bytes per V^T row (8 chunks of 16 B)
  constexpr int VBUF = kStagedV ? D * VTROW : TILEB;

  __shared__ __attribute__((aligned(1024))) char sK0[TILEB], sK1[TILEB];
  __shared__ __attribute__((aligned(1024))) char sV0[VBUF], sV1[VBUF];

  // Workgroup -> (head group, token block). Each XCD (workgroups are dealt
  // round-robin over 8) serves as few head groups as possible, so its L2
  // holds their K/V; token blocks go longest (most keys) first.
  const unsigned NH = Hkv * groups;
  const unsigned id = blockIdx.x, xcd = id % 8, j8 = id / 8;
  unsigned hg, tbr;
  if (8 % NH == 0 && nb % (8 / NH) == 0) {
    const unsigned X = 8 / NH;
    hg = xcd / X;
    tbr = j8 * X + xcd % X;
  } else if (NH % 8 == 0) {
    const unsigned per = NH / 8;
    hg = xcd * per + j8 % per;
    tbr = j8 / per;
  } else {
    hg = id % NH;
    tbr = id / NH;
  }
  const unsigned tb = nb - 1 - tbr;
  const unsigned kvh = hg / groups, grp = hg % groups;
  const unsigned wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
  const unsigned lane = threadIdx.x % 64, r = lane % 32, hi = lane / 32;
  const unsigned h = (kvh * groups + grp) * HW + wave;
  const unsigned t0 = tb * BM, tq = t0 + r;
  const bool rowValid = tq < T;
  const unsigned tLast = min(t0 + BM, T) - 1;
  const unsigned kend = P + tLast + 1; // keys [0, kend) can be visible
  const unsigned tiles = (kend + BN - 1) / BN;
  const size_t rowBytes = (size_t)Hkv * D * 2;
  const char *kbase = reinterpret_cast<const char *>(kc) + (size_t)kvh * D * 2;
  const char *vbase = reinterpret_cast<const char *>(vc) + (size_t)kvh * D * 2;

  // Load i of this wave writes tile rows (wave + HW i) RPI + [0, RPI). The
  // swizzle repeats every 8 rows (K) or 4 rows (V), so the lane offsets
  // repeat every PK / PV loads up to a uniform row shift, added per load.
  constexpr int STEP = HW * RPI;
  constexpr int PK = STEP >= 8 ? 1 : 8 / STEP, PV = STEP >= 4 ? 1 : 4 / STEP;
  unsigned koff[PK], voff[PV];
#pragma unroll
  for (int p = 0; p < PK; ++p) {
    const unsigned row = wave * RPI + lane / CPR + STEP * p, slot = lane % CPR;
    koff[p] = row * (unsigned)rowBytes + 16 * (slot ^ (row & 7));
  }
#pragma unroll
  for (int p = 0; p < PV; ++p) {
    const unsigned row = wave * RPI + lane / CPR + STEP * p, slot = lane % CPR;
    voff[p] = row * (unsigned)rowBytes + 16 * (slot ^ ((row & 3) << 1));
  }
  // One descriptor per tile over its rows below kend (none for a tile past
  // the end, whose loads then do nothing).
  auto tile_rsrc = [&](const char *base, unsigned tile) {
    const unsigned first = tile * BN;
    const unsigned rows = kend > first ? min((unsigned)BN, kend - first) : 0u;
    return __builtin_amdgcn_make_buffer_rsrc((void *)(base + (size_t)first * rowBytes),
                                             (short)0, (int)(rows * rowBytes), kBufferWord3);
  };
  // A tile's loads go out in NPART parts spread over the score MFMAs, so the
  // vector memory pipeline takes them while the matrix cores work.
  constexpr int NPART = 4;
  auto issue = [&](__amdgpu_buffer_rsrc_t rs, const unsigned *off, int period, char *dst,
                   int part) {
#pragma unroll
    for (int i = 0; i < NIW; ++i)
      if (i * NPART / NIW == part)
        load_lds16(rs, dst + 1024 * (wave + HW * i),
                   off[i % period] + (unsigned)(STEP * (i - i % period)) * (unsigned)rowBytes);
  };
  auto issue_k = [&](unsigned tile, char *dst) {
    const __amdgpu_buffer_rsrc_t rs = tile_rsrc(kbase, tile);
#pragma unroll
    for (int part = 0; part < NPART; ++part)
      issue(rs, koff, PK, dst, part);
  };
  auto issue_v = [&](unsigned tile, char *dst) {
    const __amdgpu_buffer_rsrc_t rs = tile_rsrc(vbase, tile);
#pragma unroll
    for (int part = 0; part < NPART; ++part)
      issue(rs, voff, PV, dst, part);
  };

  // Staged V: thread t owns unit t = (run, 8-channel block cb). A run is the
  // 8 keys 16G + 4hh + {0..3} and 16G + 8 + 4hh + {0..3} of a 16-key group
  // G; V^T stores them at key positions 16G + 8hh + [0, 8), i.e. bits 2 and
  // 3 of the key index swapped within each group, which is exactly the key
  // order the probability operand holds (lane half hi, slots e: key
  // 16G + 8(e/4) + 4hi + e%4). So one 16-byte read gives an MFMA operand.
  // The 16-byte chunk c of V^T row j sits at c ^ ((j / 8) % 8): the eight
  // threads writing rows 8 cb + ch for consecutive cb hit distinct banks.
  const unsigned vunit = threadIdx.x, vcb = vunit % (D / 8), vrun = vunit / (D / 8);
  const unsigned vG = vrun / 2, vhh = vrun % 2;
  const bool vowner = VUNITS == 64 * HW || vunit < (unsigned)VUNITS;
  const unsigned vsrc = (16 * vG + 4 * vhh) * (unsigned)rowBytes + 16 * vcb;
  const unsigned vdst = (8 * vcb) * VTROW + 16 * ((2 * vG + vhh) ^ (vcb % 8));
  half8_t vst[8];
  auto load_v_part = [&](__amdgpu_buffer_rsrc_t rs, int part) {
    if (vowner) {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (e * NPART / 8 == part)
          vst[e] = __builtin_bit_cast(
              half8_t,
              __builtin_amdgcn_raw_buffer_load_b128(
                  rs, vsrc, (unsigned)((e % 4) + 8 * (e / 4)) * (unsigned)rowBytes, 0));
    }
  };
  auto load_v = [&](unsigned tile) {
    const __amdgpu_buffer_rsrc_t rs = tile_rsrc(vbase, tile);
#pragma unroll
    for (int part = 0; part < NPART; ++part)
      load_v_part(rs, part);
  };
  auto store_vt = [&](char *dst) {
    if (vowner) {
#pragma unroll
      for (int ch = 0; ch < 8; ++ch)
        *reinterpret_cast<half8_t *>(dst + vdst + ch * VTROW) =
            half8_t{vst[0][ch], vst[1][ch], vst[2][ch], vst[3][ch],
                    vst[4][ch], vst[5][ch], vst[6][ch], vst[7][ch]};
    }
  };

  // Operand read offsets. K (A of S^T, row 32kt + r, chunk 2s + hi): the
  // swizzle only touches the low 3 chunk bits, so s = 4a + b reads
  // kread[b] + 128a. V^T via the transposing read: lane j of a 16-lane group
  // addresses row k0 + j/4, channels 16g + 4(j%4) .. +3 of an output tile.
  unsigned kread[4];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    kread[b] = r * ROWB + 16 * ((2 * b + hi) ^ (r & 7));
    opaque(kread[b]);
  }
  const unsigned j16 = lane % 16, g = (lane / 16) % 2;
  const unsigned vx = 2 * (j16 / 4), vb = (j16 % 4) / 2;
  const unsigned vrow = (4 * hi + j16 / 4) * ROWB + 8 * (j16 % 2);
  const unsigned vread[2] = {vrow + 16 * ((2 * g + vb) ^ vx),
                             vrow + 16 * ((4 + 2 * g + vb) ^ vx)};
  // Staged V^T: lane reads row 32 dt + r, key positions 16 G + 8 hi + [0, 8),
  // i.e. chunk (2G + hi) ^ ((4 dt + r / 8) % 8): one offset per (dt % 2, G).
  unsigned vtread[2][4];
#pragma unroll
  for (int dp = 0; dp < 2; ++dp)
#pragma unroll
    for (int G = 0; G < 4; ++G) {
      vtread[dp][G] = r * VTROW + 16 * ((2 * G + hi) ^ ((4 * dp + r / 8) % 8));
      opaque(vtread[dp][G]);
    }
  // PV operand of a tile: output tile dt, 16-key group G = 2 kt + m.
  auto vop = [&](const char *sv, int dt, int kt, int m) {
    if constexpr (kStagedV) {
      return load8(reinterpret_cast<const half_t *>(sv + vtread[dt % 2][2 * kt + m] +
                                                    32 * dt * VTROW));
    } else {
      const unsigned o = vread[dt % 2] + 128 * (dt / 2) + ROWB * (32 * kt + 16 * m);
      const half4_t lo = read_tr(sv, o), up = read_tr(sv, o + 8 * ROWB);
      return half8_t{lo[0], lo[1], lo[2], lo[3], up[0], up[1], up[2], up[3]};
    }
  };

  // Q^T as the MFMA B operand: lane holds query row r, channels
  // 16 s + 8 hi + [0, 8). Rows past T use zeros (their output is dropped).
  half8_t qb[KS];
  if constexpr (GATED) {
    // Each wave's 32 query rows through normRope in its own K/V buffer
    // (rows of D + 8 halves, then their scales). The (1 + w) weights and the
    // (token, pair) table of fp16 cos/sin, the same for every head of the
    // block, are made once per workgroup after wave 0's rows. The buffers
    // are cleared for the keys afterwards.
    static_assert(HW <= 4, "one K/V buffer per wave");
    constexpr unsigned PITCH = D + 8, CPR = D / 8;
    char *buf = wave == 0 ? sK0 : wave == 1 ? sK1 : wave == 2 ? sV0 : sV1;
    uint16_t *rows = reinterpret_cast<uint16_t *>(buf);
    float *scl = reinterpret_cast<float *>(rows + BM * PITCH);
    float *w1 = reinterpret_cast<float *>(sK0 + BM * PITCH * 2 + BM * 4);
    half2_t *cs = reinterpret_cast<half2_t *>(w1 + D); // fp16 values, stored exactly
    const unsigned half = ga.rot / 2, nrow = min((unsigned)BM, T - t0);
    const half_t *qp = reinterpret_cast<const half_t *>(ga.qproj);
    for (unsigned i = lane; i < nrow * CPR; i += 64) {
      const unsigned rr = i / CPR, cc = i % CPR;
      *reinterpret_cast<uint4_t *>(rows + rr * PITCH + 8 * cc) =
          *reinterpret_cast<const uint4_t *>(qp + ((size_t)(t0 + rr) * Hq + h) * 2 * D + 8 * cc);
    }
    for (unsigned i = threadIdx.x; i < (unsigned)D; i += 64 * HW)
      w1[i] = 1.0f + ga.qw[i];
    for (unsigned e = threadIdx.x; e < nrow * half; e += 64 * HW) {
      const unsigned tt = e / half, i = e % half;
      const float2 v2 = rope_cos_sin(__fdiv_rn((float)(P + t0 + tt), ga.freqs[i]));
      cs[e] = half2_t{(half_t)v2.x, (half_t)v2.y};
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (lane < nrow) {
      // The sequential chain; its row is read eight chunks ahead.
      const uint4_t *row = reinterpret_cast<const uint4_t *>(rows + lane * PITCH);
      float sum = 0.0f;
      for (unsigned c8 = 0; c8 < CPR; c8 += 8) {
        uint4_t x[8];
#pragma unroll
        for (int u = 0; u < 8; ++u)
          x[u] = row[c8 + u];
#pragma unroll
        for (int u = 0; u < 8; ++u)
          sum = sumsq8(x[u], sum);
      }
      scl[lane] = rms_scale_of(sum, D, ga.eps);
    }
    __syncthreads(); // the shared tables and every row's scale are in place
    const unsigned pchunks = half / 8, rest = CPR - 2 * pchunks;
    for (unsigned it = lane; it < nrow * pchunks; it += 64) {
      const unsigned rr = it / pchunks, j0 = 8 * (it % pchunks), j1 = j0 + half;
      uint16_t *row = rows + rr * PITCH;
      const float scale = scl[rr];
      const uint4_t qx = *reinterpret_cast<const uint4_t *>(row + j0);
      const uint4_t qy = *reinterpret_cast<const uint4_t *>(row + j1);
      uint4_t sx, sy;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint16_t bx = (uint16_t)(qx[e / 2] >> (16 * (e & 1)));
        const uint16_t by = (uint16_t)(qy[e / 2] >> (16 * (e & 1)));
        const float x = normed(bx, scale, w1[j0 + e]);
        const float y = normed(by, scale, w1[j1 + e]);
        const half2_t c2 = cs[rr * half + j0 + e];
        const float2 t2 = make_float2((float)c2[0], (float)c2[1]);
        const uint32_t ox = rotate_x(x, y, t2), oy = rotate_y(x, y, t2);
        if (e & 1) {
          sx[e / 2] |= ox << 16;
          sy[e / 2] |= oy << 16;
        } else {
          sx[e / 2] = ox;
          sy[e / 2] = oy;
        }
      }
      *reinterpret_cast<uint4_t *>(row + j0) = sx;
      *reinterpret_cast<uint4_t *>(row + j1) = sy;
    }
    for (unsigned it = lane; it < nrow * rest; it += 64) {
      const unsigned rr = it / rest, j0 = 8 * (2 * pchunks + it % rest);
      uint16_t *row = rows + rr * PITCH;
      const float scale = scl[rr];
      const uint4_t qx = *reinterpret_cast<const uint4_t *>(row + j0);
      uint4_t sx;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t lo = f2h(normed((uint16_t)(qx[e] & 0xFFFFu), scale, w1[j0 + 2 * e]));
        const uint32_t hi = f2h(normed((uint16_t)(qx[e] >> 16), scale, w1[j0 + 2 * e + 1]));
        sx[e] = lo | (hi << 16);
      }
      *reinterpret_cast<uint4_t *>(row + j0) = sx;
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int s = 0; s < KS; ++s)
      qb[s] = rowValid ? *reinterpret_cast<const half8_t *>(rows + r * PITCH + 16 * s + 8 * hi)
                       : half8_t{0, 0, 0, 0, 0, 0, 0, 0};
    __syncthreads(); // every wave is done with its buffer before they are cleared
  } else {
#pragma unroll
    for (int s = 0; s < KS; ++s)
      qb[s] = rowValid ? load8(q + ((size_t)tq * Hq + h) * D + 16 * s + 8 * hi)
                       : half8_t{0, 0, 0, 0, 0, 0, 0, 0};
  }

  float16_t oacc[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i)
    oacc[i] = float16_t{0};
  // l (the softmax denominator) is accumulated by the MFMA as ones x P^T,
  // from the same fp16 probabilities that multiply V: every register of
  // lacc holds the row sum of the lane's query.
  float mRef = -INFINITY;
  float16_t lacc = float16_t{0};
  const half8_t ones{1, 1, 1, 1, 1, 1, 1, 1};
  half8_t pb[2][2]; // P^T B operands, [32-key half][16-key step]

  auto pv = [&](const char *svl) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int m = 0; m < 2; ++m) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
          oacc[dt] = mfma32x32x16(vop(svl, dt, kt, m), pb[kt][m], oacc[dt]);
        lacc = mfma32x32x16(ones, pb[kt][m], lacc);
      }
  };
  // Causal mask as the scores' initial accumulator: -inf where key > P + tq
  // (a finite K row plus -inf stays -inf), 0 elsewhere.
  auto mask_init = [&](unsigned base, float16_t (&init)[2]) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int v = 0; v < 16; ++v)
        init[kt][v] = base + 32 * kt + mfma_c_row(v, hi) > P + tq ? -INFINITY : 0.0f;
  };
  // Softmax, first half: the tile's row maximum decides whether the
  // reference moves (then O must be rescaled by the returned factor, which
  // the caller does when any row of the wave moved); l follows at once.
  auto reference = [&](float mx, bool &raised) {
    const LanePair pr = pair32(mx);
    const float tm = fmaxf(pr.a, pr.b) * c;
    const bool need = tm - mRef > kRaise;
    const float mNew = need ? tm - kHeadroom : mRef;
    const float alpha = fast_exp2(mRef - mNew);
    mRef = mNew;
    raised = __builtin_amdgcn_ballot_w64(need) != 0;
    return alpha;
  };
  // Softmax, second half: the fp16 probabilities of scores sp against the
  // current reference, as PV operand pb, and their sum into l.
  auto prob = [&](const float (&sp)[32], int j, float negm) {
    const int kt = j / 16, m = (j / 8) % 2, e = j % 8;
    pb[kt][m][e] = (half_t)fast_exp2(fmaf(sp[16 * kt + 8 * m + e], c, negm));
  };

  // Phase A of step i: the score MFMAs of tile i, each K operand read three
  // k-steps ahead, with the probabilities of tile i-1 (scores sp) computed
  // on the VALU in between.
  auto phase_a = [&](const char *sk, const float16_t *init, const float (&sp)[32],
                     float16_t (&sacc)[2], auto &&feed) {
    constexpr int PER = 32 / KS; // probabilities per k-step
    auto kld = [&](int st, int kt) {
      return load8(reinterpret_cast<const half_t *>(sk + kread[st % 4] + 128 * (st / 4) +
                                                    32 * ROWB * kt));
    };
    const float negm = -mRef;
    constexpr int AHEAD = 3;
    half8_t ka[AHEAD + 1][2];
#pragma unroll
    for (int st = 0; st < AHEAD; ++st) {
      ka[st][0] = kld(st, 0);
      ka[st][1] = kld(st, 1);
    }
    sacc[0] = init ? init[0] : float16_t{0};
    sacc[1] = init ? init[1] : float16_t{0};
#pragma unroll
    for (int st = 0; st < KS; ++st) {
      if (st + AHEAD < KS) {
        ka[(st + AHEAD) % (AHEAD + 1)][0] = kld(st + AHEAD, 0);
        ka[(st + AHEAD) % (AHEAD + 1)][1] = kld(st + AHEAD, 1);
      }
      sacc[0] = mfma32x32x16(ka[st % (AHEAD + 1)][0], qb[st], sacc[0]);
      sacc[1] = mfma32x32x16(ka[st % (AHEAD + 1)][1], qb[st], sacc[1]);
#pragma unroll
      for (int u = 0; u < PER; ++u)
        prob(sp, st * PER + u, negm);
      if (st % (KS / NPART) == 0)
        feed(st / (KS / NPART));
    }
  };
  // Phase B of step i: the PV MFMAs of tile i-1, each V^T operand read two
  // MFMAs ahead, with the row maximum of tile i taken in between.
  auto phase_b = [&](const char *svl, const float16_t (&sacc)[2], float (&sv)[32],
                     bool &raised) {
    constexpr int NPV = 4 * DT, PER = 32 / NPV;
    // Consecutive MFMAs go to different output tiles (independent chains).
    auto vld = [&](int n) { return vop(svl, n % DT, n / (2 * DT), (n / DT) % 2); };
    half8_t va[3];
    va[0] = vld(0);
    va[1] = vld(1);
    float mx = -INFINITY;
#pragma unroll
    for (int n = 0; n < NPV; ++n) {
      if (n + 2 < NPV)
        va[(n + 2) % 3] = vld(n + 2);
      const int dt = n % DT, kt = n / (2 * DT), m = (n / DT) % 2;
      oacc[dt] = mfma32x32x16(va[n % 3], pb[kt][m], oacc[dt]);
      if (dt == DT - 1)
        lacc = mfma32x32x16(ones, pb[kt][m], lacc);
#pragma unroll
      for (int u = 0; u < PER; ++u) {
        const int j = n * PER + u;
        sv[j] = sacc[j / 16][j % 16];
        mx = fmaxf(mx, sv[j]);
      }
    }
    return reference(mx, raised);
  };

  // Buffers start zeroed: rows past the block's last key may keep what was
  // there before, which must be finite (a probability of 0 times V, and the
  // -inf mask plus a K dot product, must stay exact).
  {
    const uint4_t z{0, 0, 0, 0};
    for (unsigned i = threadIdx.x * 16; i < (unsigned)TILEB; i += 64 * HW * 16) {
      *reinterpret_cast<uint4_t *>(sK0 + i) = z;
      *reinterpret_cast<uint4_t *>(sK1 + i) = z;
    }
    for (unsigned i = threadIdx.x * 16; i < (unsigned)VBUF; i += 64 * HW * 16) {
      *reinterpret_cast<uint4_t *>(sV0 + i) = z;
      *reinterpret_cast<uint4_t *>(sV1 + i) = z;
    }
  }
  __syncthreads();
  issue_k(0, sK0);
  if constexpr (kStagedV)
    load_v(0);
  else
    issue_v(0, sV0);
  wait_loads();
  __syncthreads();
  if (tiles > 1)
    issue_k(1, sK1);

  // Tile 0: scores and reference only (O is still zero).
  float sv[32]; // scores of the last tile, raw (masked keys -inf)
  {
    float16_t init[2], sacc[2];
    const bool masked = BN > P + t0 + 1;
    if (masked)
      mask_init(0, init);
    const float zero[32] = {};
    phase_a(sK0, masked ? init : nullptr, zero, sacc, [](int) {});
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      sv[j] = sacc[j / 16][j % 16];
      mx = fmaxf(mx, sv[j]);
    }
    bool raised;
    reference(mx, raised);
  }

  // Step i: phase A (scores of tile i, probabilities of tile i-1), phase B
  // (PV of tile i-1, row maximum of tile i), with the loads of K(i+1) and
  // V(i) in flight. Buffers are named statically so the compiler can tell
  // the loads in flight from the LDS reads and need not wait for them;
  // tiles below the block's first query (the steady state, run in pairs)
  // skip the mask.
  auto step = [&](unsigned i, bool masked, const char *kcur, char *vprev, char *knext,
                  char *vdst) {
    wait_loads();
    if constexpr (kStagedV)
      store_vt(vprev); // V(i-1), loaded during the previous step
    __syncthreads();
    // K(i+1) (none past the last tile) and V(i), spread over phase A.
    const __amdgpu_buffer_rsrc_t krs = tile_rsrc(kbase, i + 1), vrs = tile_rsrc(vbase, i);
    auto feed = [&](int part) {
      issue(krs, koff, PK, knext, part);
      if constexpr (kStagedV)
        load_v_part(vrs, part);
      else
        issue(vrs, voff, PV, vdst, part);
    };
    float16_t init[2], sacc[2];
    if (masked)
      mask_init(i * BN, init);
    bool raised;
    phase_a(kcur, masked ? init : nullptr, sv, sacc, feed);
    const float alpha = phase_b(vprev, sacc, sv, raised);
    if (raised) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
        oacc[dt] *= alpha;
      lacc *= alpha;
    }
  };
  // Tiles [1, iu) lie wholly below the block's first query.
  const unsigned iu = max(1u, min(tiles, (P + t0 + 1) / BN));
  unsigned i = 1;
  for (; i + 1 < iu; i += 2) {
    step(i, false, sK1, sV0, sK0, sV1);
    step(i + 1, false, sK0, sV1, sK1, sV0);
  }
  // The rest (at most three tiles) with the mask, which is all-pass on an
  // unmasked tile.
  for (; i < tiles; i += 2) {
    step(i, true, sK1, sV0, sK0, sV1);
    if (i + 1 < tiles)
      step(i + 1, true, sK0, sV1, sK1, sV0);
  }
  {
    const float negm = -mRef;
#pragma unroll
    for (int j = 0; j < 32; ++j)
      prob(sv, j, negm);
  }
  wait_loads();
  if constexpr (kStagedV)
    store_vt((tiles - 1) % 2 == 0 ? sV0 : sV1);
  __syncthreads();
  if ((tiles - 1) % 2 == 0)
    pv(sV0);
  else
    pv(sV1);

  if (!rowValid)
    return;
  const float inv = 1.0f / lacc[0];
  half_t *orow = out + ((size_t)tq * Hq + h) * D;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    half4_t v[4];
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4)
      v[g4] = half4_t{f16_of(oacc[dt][4 * g4 + 0] * inv), f16_of(oacc[dt][4 * g4 + 1] * inv),
                      f16_of(oacc[dt][4 * g4 + 2] * inv), f16_of(oacc[dt][4 * g4 + 3] * inv)};
    if constexpr (GATED)
      gate_tile(v, reinterpret_cast<const half_t *>(ga.qproj) + ((size_t)tq * Hq + h) * 2 * D +
                       D + 32 * dt + 4 * hi, ga.activated);
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4)
      *reinterpret_cast<half4_t *>(orow + 32 * dt + 8 * g4 + 4 * hi) = v[g4];
  }
}

// d = 256 with an even number of query heads per KV head: eight waves, two
// per SIMD, over a pair of token blocks (nb - 1 - p and p: their key counts
// add up to the same total for every pair, which balances the causal
// triangle across workgroups) and two query heads. Wave w serves block
// w / 4 (the long one first), head (w / 2) % 2 and key half w % 2: each
// (block, head) has a wave pair that splits the keys by 32-key tiles, the
// even tiles to one wave, the odd ones to the other, each with its own
// (m, l, O). SIMD j (a workgroup's waves are dealt to the SIMDs in turn)
// runs wave j of the long block and wave j of the short one: while one
// waits on LDS operands or runs its softmax the other keeps the matrix core
// busy, and once the short block is done the long block's wave has the
// SIMD to itself. A lane holds O^T (128 registers), Q^T (64) and one 32x32
// score block; the row sums are fp32 sums of the fp16 probabilities that
// multiply V (v_dot2). At the end each odd-tile wave hands its (m, l, O) to
// its partner through LDS. One step = one barrier: the four tiles of the
// next step (K and V of tiles 2s + 2 and 2s + 3, shared by both blocks) go
// HBM -> LDS as the step begins. GATED as in gqa_prefill_kernel: the query
// rows go through normRope in LDS before the loop (the workgroup's 512
// threads share the rows, the scales and one cos/sin table per block), the
// output through the sigmoid gate.
template <bool GATED>
__global__ __attribute__((amdgpu_flat_work_group_size(512, 512), amdgpu_waves_per_eu(2, 2)))
void gqa_prefill_halves_kernel(const half_t *__restrict__ q, const half_t *__restrict__ kc,
                               const half_t *__restrict__ vc, half_t *__restrict__ out,
                               unsigned T, unsigned Hq, unsigned Hkv, unsigned P,
                               unsigned hpairs, unsigned nb, float c,
                               typename std::conditional<GATED, GatedRows, NoRows>::type ga) {
  constexpr int D = 256, KS = D / 16, DT = D / 32;
  constexpr int BK = 32;           // keys per tile
  constexpr int ROWB = 2 * D;      // bytes per K/V row
  constexpr int TILEB = BK * ROWB; // 16 KB per K or V tile
  // [set][half]: set s % 2 holds what step s reads. Named one by one so the
  // compiler can tell the loads in flight from the LDS reads.
  __shared__ __attribute__((aligned(1024))) char sK00[TILEB], sK01[TILEB], sK10[TILEB],
      sK11[TILEB];
  __shared__ __attribute__((aligned(1024))) char sV00[TILEB], sV01[TILEB], sV10[TILEB],
      sV11[TILEB];
  __shared__ float sML[4][2][64];
  // GATED: the (1 + w) weights, then the (token, pair) table of fp16 cos/sin.
  __shared__ float sTab[GATED ? D + BM * (D / 2) : 1];

  // Workgroup -> (block pair, KV head, head pair): each XCD (workgroups are
  // dealt round-robin over 8) serves as few KV heads as possible, so its L2
  // holds their K/V.
  const unsigned NH = Hkv * hpairs, npairs = (nb + 1) / 2;
  const unsigned id = blockIdx.x, xcd = id % 8, j8 = id / 8;
  unsigned hg, pr;
  if (8 % NH == 0 && npairs % (8 / NH) == 0) {
    const unsigned X = 8 / NH;
    hg = xcd / X;
    pr = j8 * X + xcd % X;
  } else if (NH % 8 == 0) {
    const unsigned per = NH / 8;
    hg = xcd * per + j8 % per;
    pr = j8 / per;
  } else {
    hg = id % NH;
    pr = id / NH;
  }
  const unsigned kvh = hg / hpairs, hp = hg % hpairs;
  const unsigned bL = nb - 1 - pr, bS = pr;
  const unsigned wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
  const unsigned blk = wave / 4, hs = (wave / 2) % 2, half = wave % 2;
  const unsigned pi = 2 * blk + hs; // (block, head) of this wave
  const bool idle = blk == 1 && bS == bL; // nb odd: the middle block pairs with itself
  const unsigned lane = threadIdx.x % 64, r = lane % 32, hi = lane / 32;
  const unsigned h = (kvh * hpairs + hp) * 2 + hs;
  const unsigned t0 = (blk ? bS : bL) * BM, tq = t0 + r;
  const bool rowValid = tq < T && !idle;
  // Keys [0, kend) can be visible to the long block; this wave's block needs
  // its first `mine` tiles.
  const unsigned kend = P + min(bL * BM + BM, T);
  const unsigned ntiles = (kend + BK - 1) / BK, steps = (ntiles + 1) / 2;
  const unsigned mine = idle ? 0u : (P + min(t0 + BM, T) + BK - 1) / BK;
  const unsigned ju = (P + t0 + 1) / BK; // tiles [0, ju) need no mask
  const size_t rowBytes = (size_t)Hkv * D * 2;
  const char *kbase = reinterpret_cast<const char *>(kc) + (size_t)kvh * D * 2;
  const char *vbase = reinterpret_cast<const char *>(vc) + (size_t)kvh * D * 2;

  // Wave w moves the 1-KB pieces w and w + 8 (tile rows 2p, 2p + 1) of each
  // tile; the XOR swizzles (K chunk c of row j at c ^ (j % 8), V chunk c at
  // c ^ 2(j % 4)) repeat every 16 rows, so piece w + 8 is piece w 16 rows on.
  const unsigned prow = 2 * wave + lane / 32, slot = lane % 32;
  const unsigned koff = prow * (unsigned)rowBytes + 16 * (slot ^ (prow & 7));
  const unsigned voff = prow * (unsigned)rowBytes + 16 * (slot ^ ((prow & 3) << 1));
  const unsigned pstep = 16 * (unsigned)rowBytes;
  auto tile_rsrc = [&](const char *base, unsigned tile) {
    const unsigned first = tile * BK;
    const unsigned rows = kend > first ? min((unsigned)BK, kend - first) : 0u;
    return __builtin_amdgcn_make_buffer_rsrc((void *)(base + (size_t)first * rowBytes),
                                             (short)0, (int)(rows * rowBytes), kBufferWord3);
  };
  auto load_tile = [&](const char *base, unsigned tile, unsigned off, char *dst) {
    const __amdgpu_buffer_rsrc_t rs = tile_rsrc(base, tile);
    load_lds16(rs, dst + 1024 * wave, off);
    load_lds16(rs, dst + 1024 * (wave + 8), off + pstep);
  };

  // Operand reads. K (A of S^T, row r, chunk 2s + hi): kread[s % 4] +
  // 128 (s / 4). V^T through the transposing read: lane j of a 16-lane
  // group addresses row k0 + j / 4, channels 16 g + 4 (j % 4) .. +3.
  unsigned kread[4];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    kread[b] = r * ROWB + 16 * ((2 * b + hi) ^ (r & 7));
    opaque(kread[b]);
  }
  const unsigned j16 = lane % 16, g = (lane / 16) % 2;
  const unsigned vx = 2 * (j16 / 4), vb = (j16 % 4) / 2;
  const unsigned vrow = (4 * hi + j16 / 4) * ROWB + 8 * (j16 % 2);
  unsigned vread[2] = {vrow + 16 * ((2 * g + vb) ^ vx), vrow + 16 * ((4 + 2 * g + vb) ^ vx)};
  opaque(vread[0]);
  opaque(vread[1]);

  half8_t qb[KS];
  if constexpr (GATED) {
    // (block, head) pair pp's row rr sits in buffer 2 pp + rr / 16 at
    // (rr % 16) * PITCH (rows of D + 8 halves keep the per-row chains off
    // one bank).
    constexpr unsigned PITCH = D + 8, CPR = D / 8;
    auto rowp = [&](unsigned pp, unsigned rr) {
      const unsigned bsel = 2 * pp + rr / 16;
      char *b = bsel == 0   ? sK00
                : bsel == 1 ? sK01
                : bsel == 2 ? sK10
                : bsel == 3 ? sK11
                : bsel == 4 ? sV00
                : bsel == 5 ? sV01
                : bsel == 6 ? sV10
                            : sV11;
      return reinterpret_cast<uint16_t *>(b) + (rr % 16) * PITCH;
    };
    const unsigned halfrot = ga.rot / 2;
    const unsigned nrL = min((unsigned)BM, T - bL * BM), nrS = min((unsigned)BM, T - bS * BM);
    auto nrow = [&](unsigned pp) { return pp < 2 ? nrL : nrS; };
    auto first_tok = [&](unsigned pp) { return (pp < 2 ? bL : bS) * BM; };
    const half_t *qp = reinterpret_cast<const half_t *>(ga.qproj);
    for (unsigned i = threadIdx.x; i < 4 * BM * CPR; i += 512) {
      const unsigned pp = i / (BM * CPR), rem = i % (BM * CPR);
      const unsigned rr = rem / CPR, cc = rem % CPR;
      if (rr < nrow(pp))
        *reinterpret_cast<uint4_t *>(rowp(pp, rr) + 8 * cc) =
            *reinterpret_cast<const uint4_t *>(
                qp + ((size_t)(first_tok(pp) + rr) * Hq + (kvh * hpairs + hp) * 2 + pp % 2) *
                         2 * D +
                8 * cc);
    }
    float *w1 = sTab;
    half2_t *cs = reinterpret_cast<half2_t *>(sTab + D); // fp16 values, stored exactly
    for (unsigned i = threadIdx.x; i < (unsigned)D; i += 512)
      w1[i] = 1.0f + ga.qw[i];
    __syncthreads();
    if (threadIdx.x < 4 * BM) {
      // The sequential chain of one row; its chunks are read eight ahead.
      const unsigned pp = threadIdx.x / BM, rr = threadIdx.x % BM;
      if (rr < nrow(pp)) {
        const uint4_t *row = reinterpret_cast<const uint4_t *>(rowp(pp, rr));
        float sum = 0.0f;
        for (unsigned c8 = 0; c8 < CPR; c8 += 8) {
          uint4_t x[8];
#pragma unroll
          for (int u = 0; u < 8; ++u)
            x[u] = row[c8 + u];
#pragma unroll
          for (int u = 0; u < 8; ++u)
            sum = sumsq8(x[u], sum);
        }
        sML[pp][0][rr] = rms_scale_of(sum, D, ga.eps);
      }
    }
    const unsigned pchunks = halfrot / 8, rest = CPR - 2 * pchunks;
    for (unsigned bb = 0; bb < 2; ++bb) {
      // The cos/sin table of this block's tokens, then its two heads' rows.
      const unsigned tok0 = bb ? bS * BM : bL * BM, nr = bb ? nrS : nrL;
      for (unsigned e = threadIdx.x; e < nr * halfrot; e += 512) {
        const unsigned tt = e / halfrot, i = e % halfrot;
        const float2 v2 = rope_cos_sin(__fdiv_rn((float)(P + tok0 + tt), ga.freqs[i]));
        cs[e] = half2_t{(half_t)v2.x, (half_t)v2.y};
      }
      __syncthreads(); // the table (and, the first time, every scale)
      for (unsigned it = threadIdx.x; it < 2 * nr * pchunks; it += 512) {
        const unsigned pp = 2 * bb + it / (nr * pchunks), rem = it % (nr * pchunks);
        const unsigned rr = rem / pchunks, j0 = 8 * (rem % pchunks), j1 = j0 + halfrot;
        uint16_t *row = rowp(pp, rr);
        const float scale = sML[pp][0][rr];
        const uint4_t qx = *reinterpret_cast<const uint4_t *>(row + j0);
        const uint4_t qy = *reinterpret_cast<const uint4_t *>(row + j1);
        uint4_t sx, sy;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint16_t bx = (uint16_t)(qx[e / 2] >> (16 * (e & 1)));
          const uint16_t by = (uint16_t)(qy[e / 2] >> (16 * (e & 1)));
          const float x = normed(bx, scale, w1[j0 + e]);
          const float y = normed(by, scale, w1[j1 + e]);
          const half2_t c2 = cs[rr * halfrot + j0 + e];
          const float2 t2 = make_float2((float)c2[0], (float)c2[1]);
          const uint32_t ox = rotate_x(x, y, t2), oy = rotate_y(x, y, t2);
          if (e & 1) {
            sx[e / 2] |= ox << 16;
            sy[e / 2] |= oy << 16;
          } else {
            sx[e / 2] = ox;
            sy[e / 2] = oy;
          }
        }
        *reinterpret_cast<uint4_t *>(row + j0) = sx;
        *reinterpret_cast<uint4_t *>(row + j1) = sy;
      }
      for (unsigned it = threadIdx.x; it < 2 * nr * rest; it += 512) {
        const unsigned pp = 2 * bb + it / (nr * rest), rem = it % (nr * rest);
        const unsigned rr = rem / rest, j0 = 8 * (2 * pchunks + rem % rest);
        uint16_t *row = rowp(pp, rr);
        const float scale = sML[pp][0][rr];
        const uint4_t qx = *reinterpret_cast<const uint4_t *>(row + j0);
        uint4_t sx;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t lo = f2h(normed((uint16_t)(qx[e] & 0xFFFFu), scale, w1[j0 + 2 * e]));
          const uint32_t hi2 = f2h(normed((uint16_t)(qx[e] >> 16), scale, w1[j0 + 2 * e + 1]));
          sx[e] = lo | (hi2 << 16);
        }
        *reinterpret_cast<uint4_t *>(row + j0) = sx;
      }
      __syncthreads(); // the table is free again
    }
    const uint16_t *myrow = rowp(pi, r);
#pragma unroll
    for (int s = 0; s < KS; ++s)
      qb[s] = rowValid ? *reinterpret_cast<const half8_t *>(myrow + 16 * s + 8 * hi)
                       : half8_t{0, 0, 0, 0, 0, 0, 0, 0};
    __syncthreads(); // every wave has its rows before the buffers are cleared
  } else {
#pragma unroll
    for (int s = 0; s < KS; ++s)
      qb[s] = rowValid ? load8(q + ((size_t)tq * Hq + h) * D + 16 * s + 8 * hi)
                       : half8_t{0, 0, 0, 0, 0, 0, 0, 0};
  }

  float16_t oacc[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i)
    oacc[i] = float16_t{0};
  float mRef = -INFINITY, lsum = 0.0f;
  float16_t sacc = float16_t{0};
  half8_t pb[2]; // P^T B operands, [16-key step]

  // Scores of one tile into sacc (the causal mask as the initial
  // accumulator where the tile reaches past the block's first query).
  auto scores = [&](const char *kb, unsigned tile) {
    auto kld = [&](int st) {
      return load8(reinterpret_cast<const half_t *>(kb + kread[st % 4] + 128 * (st / 4)));
    };
    constexpr int KA = 2; // operand reads run KA MFMAs ahead
    half8_t ka[KA + 1];
#pragma unroll
    for (int st = 0; st < KA; ++st)
      ka[st] = kld(st);
    if (tile >= ju) {
#pragma unroll
      for (int v = 0; v < 16; ++v)
        sacc[v] = tile * BK + mfma_c_row(v, hi) > P + tq ? -INFINITY : 0.0f;
    } else {
      sacc = float16_t{0};
    }
#pragma unroll
    for (int st = 0; st < KS; ++st) {
      if (st + KA < KS)
        ka[(st + KA) % (KA + 1)] = kld(st + KA);
      sacc = mfma32x32x16(ka[st % (KA + 1)], qb[st], sacc);
      __builtin_amdgcn_sched_barrier(0); // operand reads stay KA ahead, no further
    }
  };
  // Softmax of sacc against the lazily moved reference (raised only when a
  // probability would pass 2^15; O and l rescaled then), the fp16
  // probabilities into pb, their sum into l.
  auto softmax = [&]() {
    float mx = sacc[0];
#pragma unroll
    for (int v = 1; v < 16; ++v)
      mx = fmaxf(mx, sacc[v]);
    const LanePair pr = pair32(mx);
    const float tm = fmaxf(pr.a, pr.b) * c;
    const bool need = tm - mRef > kRaise; // false while every key so far is masked
    const float mNew = need ? tm - kHeadroom : mRef;
    const float alpha = need ? fast_exp2(mRef - mNew) : 1.0f;
    mRef = mNew;
    if (__builtin_amdgcn_ballot_w64(need) != 0) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
        oacc[dt] *= alpha;
      lsum *= alpha;
    }
    const float negm = mRef == -INFINITY ? 0.0f : -mRef;
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int e = 0; e < 8; ++e)
        pb[m][e] = (half_t)fast_exp2(fmaf(sacc[8 * m + e], c, negm));
    const half2_t one2{1, 1};
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int e = 0; e < 8; e += 2)
        lsum = __builtin_amdgcn_fdot2(half2_t{pb[m][e], pb[m][e + 1]}, one2, lsum, false);
  };
  // O^T += V^T P^T for one tile: output tile dt, 16-key step m.
  auto pv = [&](const char *vbuf) {
    auto vld = [&](int n) {
      const int dt = n % DT, m = n / DT;
      const unsigned o = vread[dt % 2] + 128 * (dt / 2) + ROWB * 16 * m;
      const half4_t lo = read_tr(vbuf, o), up = read_tr(vbuf, o + 8 * ROWB);
      return half8_t{lo[0], lo[1], lo[2], lo[3], up[0], up[1], up[2], up[3]};
    };
    constexpr int VA = 2;
    half8_t va[VA + 1];
#pragma unroll
    for (int n = 0; n < VA; ++n)
      va[n] = vld(n);
#pragma unroll
    for (int n = 0; n < 2 * DT; ++n) {
      if (n + VA < 2 * DT)
        va[(n + VA) % (VA + 1)] = vld(n + VA);
      oacc[n % DT] = mfma32x32x16(va[n % (VA + 1)], pb[n / DT], oacc[n % DT]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // LDS starts zeroed: rows past the block's last key keep whatever an
  // earlier tile left there, which must be finite.
  {
    const uint4_t z{0, 0, 0, 0};
    for (unsigned i = threadIdx.x * 16; i < (unsigned)TILEB; i += 512 * 16) {
      *reinterpret_cast<uint4_t *>(sK00 + i) = z;
      *reinterpret_cast<uint4_t *>(sK01 + i) = z;
      *reinterpret_cast<uint4_t *>(sK10 + i) = z;
      *reinterpret_cast<uint4_t *>(sK11 + i) = z;
      *reinterpret_cast<uint4_t *>(sV00 + i) = z;
      *reinterpret_cast<uint4_t *>(sV01 + i) = z;
      *reinterpret_cast<uint4_t *>(sV10 + i) = z;
      *reinterpret_cast<uint4_t *>(sV11 + i) = z;
    }
  }
  __syncthreads();
  load_tile(kbase, 0, koff, sK00);
  load_tile(kbase, 1, koff, sK01);
  load_tile(vbase, 0, voff, sV00);
  load_tile(vbase, 1, voff, sV01);

  // Step s: set s % 2 holds K and V of tiles 2s and 2s + 1; the other set
  // receives those of 2s + 2 and 2s + 3, requested as the step begins. Each
  // half runs its own loop (one barrier per step in both) over its
  // statically named buffers.
  auto loads = [&](unsigned s, char *nkA, char *nkB, char *nvA, char *nvB) {
    load_tile(kbase, 2 * s + 2, koff, nkA);
    load_tile(kbase, 2 * s + 3, koff, nkB);
    load_tile(vbase, 2 * s + 2, voff, nvA);
    load_tile(vbase, 2 * s + 3, voff, nvB);
  };
  auto run = [&](unsigned first, const char *k0, const char *v0, const char *k1,
                 const char *v1) {
    auto step = [&](unsigned s, const char *kc_, const char *vc_, char *nkA, char *nkB,
                    char *nvA, char *nvB) {
      wait_loads();
      __syncthreads();
      loads(s, nkA, nkB, nvA, nvB);
      if (2 * s + first < mine) {
        scores(kc_, 2 * s + first);
        softmax();
        pv(vc_);
      }
    };
    unsigned s = 0;
    for (; s + 1 < steps; s += 2) {
      step(s, k0, v0, sK10, sK11, sV10, sV11);
      step(s + 1, k1, v1, sK00, sK01, sV00, sV01);
    }
    if (s < steps)
      step(s, k0, v0, sK10, sK11, sV10, sV11);
  };
  if (half == 0)
    run(0, sK00, sV00, sK10, sV10);
  else
    run(1, sK01, sV01, sK11, sV11);
  wait_loads();
  __syncthreads(); // every wave is done with the K/V buffers

  // The odd half's (m, l, O^T) to LDS, lane-major (conflict-free): pair pi
  // uses two 16 KB buffers, output tiles 0-3 in the first.
  char *ma = pi == 0 ? sK00 : pi == 1 ? sK10 : pi == 2 ? sV00 : sV10;
  char *mb = pi == 0 ? sK01 : pi == 1 ? sK11 : pi == 2 ? sV01 : sV11;
  if (half == 1) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int v = 0; v < 16; ++v)
        reinterpret_cast<float *>(dt < 4 ? ma : mb)[((dt % 4) * 16 + v) * 64 + lane] =
            oacc[dt][v];
    sML[pi][0][lane] = mRef;
    sML[pi][1][lane] = lsum;
  }
  __syncthreads();
  if (half == 1 || !rowValid)
    return;
  const float m1 = sML[pi][0][lane], l1 = sML[pi][1][lane];
  const float M = fmaxf(mRef, m1); // mRef is finite: key 0 is visible to every row
  const float a0 = fast_exp2(mRef - M), a1 = fast_exp2(m1 - M);
  const LanePair lp = pair32(lsum * a0 + l1 * a1);
  const float inv = 1.0f / (lp.a + lp.b);
  half_t *orow = out + ((size_t)tq * Hq + h) * D;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    const float *o1 = reinterpret_cast<const float *>(dt < 4 ? ma : mb) + (dt % 4) * 16 * 64;
    half4_t v[4];
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = 4 * g4 + e;
        v[g4][e] = f16_of((oacc[dt][i] * a0 + o1[i * 64 + lane] * a1) * inv);
      }
    if constexpr (GATED)
      gate_tile(v, reinterpret_cast<const half_t *>(ga.qproj) + ((size_t)tq * Hq + h) * 2 * D +
                       D + 32 * dt + 4 * hi, ga.activated);
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4)
      *reinterpret_cast<half4_t *>(orow + 32 * dt + 8 * g4 + 4 * hi) = v[g4];
  }
}

template <int D> constexpr unsigned heads_per_wg(unsigned G) {
  return G < (D == 256 ? 4u : 8u) ? G : (D == 256 ? 4u : 8u);
}

template <int D, int HW, bool GATED = false, typename Rows = NoRows>
hipError_t launch_dw(const GqaShape &s, const uint16_t *q, const uint16_t *k,
                     const uint16_t *v, uint16_t *out, hipStream_t stream,
                     const Rows &rows = Rows{}) {
  const float c = kLog2e / sqrtf((float)D);
  const unsigned G = s.Hq / s.Hkv, groups = G / HW, nb = (s.T + BM - 1) / BM;
  hipLaunchKernelGGL((gqa_prefill_kernel<D, HW, GATED>), dim3(nb * s.Hkv * groups),
                     dim3(64 * HW), 0, stream, reinterpret_cast<const half_t *>(q),
                     reinterpret_cast<const half_t *>(k), reinterpret_cast<const half_t *>(v),
                     reinterpret_cast<half_t *>(out), s.T, s.Hq, s.Hkv, s.P, groups, nb, c,
                     rows);
  return hipGetLastError();
}

template <bool GATED, typename Rows>
hipError_t launch_halves(const GqaShape &s, const uint16_t *q, const uint16_t *k,
                         const uint16_t *v, uint16_t *out, hipStream_t stream,
                         const Rows &rows) {
  const float c = kLog2e / sqrtf(256.0f);
  const unsigned G = s.Hq / s.Hkv, hpairs = G / 2, nb = (s.T + BM - 1) / BM;
  hipLaunchKernelGGL((gqa_prefill_halves_kernel<GATED>), dim3((nb + 1) / 2 * s.Hkv * hpairs),
                     dim3(512), 0, stream, reinterpret_cast<const half_t *>(q),
                     reinterpret_cast<const half_t *>(k), reinterpret_cast<const half_t *>(v),
                     reinterpret_cast<half_t *>(out), s.T, s.Hq, s.Hkv, s.P, hpairs, nb, c,
                     rows);
  return hipGetLastError();
}

// The key-split kernel once the grid has at least 64 workgroups (below
// that, as at 128 tokens, the single-wave kernel's shorter prologue wins by
// ~1 us). LLMI_PREFILL_HALVES=0 selects the single-wave kernel always, =1
// the key-split one always (for A/B timing). The plain and gated launches
// take the same choice, so the two stay bit-identical.
bool use_halves(const GqaShape &s) {
  static const int forced = [] {
    const char *e = getenv("LLMI_PREFILL_HALVES");
    return e && *e ? (*e == '0' ? 0 : 1) : -1;
  }();
  if (forced >= 0)
    return forced == 1;
  const unsigned nb = (s.T + BM - 1) / BM, hpairs = s.Hq / s.Hkv / 2;
  return (nb + 1) / 2 * s.Hkv * hpairs >= 64;
}

// Query heads a single-wave-kernel workgroup serves: four share each K/V
// tile, but a grid of fewer than 32 such workgroups (a short prefill, e.g.
// 128 tokens at 16 / 4 heads: 16 workgroups) leaves most CUs idle, and two
// heads a workgroup twice as many workgroups ran faster (measured at 128
// tokens: 13.2 us with four, 10.9 with two, 12.3 with one). Every head's
// arithmetic is its own, so the choice changes no bits.
template <int D> unsigned prefill_heads(const GqaShape &s) {
  const unsigned G = s.Hq / s.Hkv, hw = heads_per_wg<D>(G);
  const unsigned nb = (s.T + BM - 1) / BM;
  return hw == 4 && nb * s.Hkv * (G / hw) < 32 ? 2u : hw;
}

template <int D>
hipError_t launch_gated_d(const GqaShape &s, const uint16_t *k, const uint16_t *v,
                          uint16_t *out, const GatedRows &ga, hipStream_t stream) {
  switch (prefill_heads<D>(s)) {
  case 1:
    return launch_dw<D, 1, true>(s, nullptr, k, v, out, stream, ga);
  case 2:
    return launch_dw<D, 2, true>(s, nullptr, k, v, out, stream, ga);
  case 4:
    if (D == 256 && use_halves(s))
      return launch_halves<true>(s, nullptr, k, v, out, stream, ga);
    return launch_dw<D, 4, true>(s, nullptr, k, v, out, stream, ga);
  }
  return hipErrorInvalidValue;
}

template <int D>
hipError_t launch_d(const GqaShape &s, const uint16_t *q, const uint16_t *k,
                    const uint16_t *v, uint16_t *out, hipStream_t stream) {
  switch (prefill_heads<D>(s)) {
  case 1:
    return launch_dw<D, 1>(s, q, k, v, out, stream);
  case 2:
    return launch_dw<D, 2>(s, q, k, v, out, stream);
  case 4:
    if (D == 256 && use_halves(s))
      return launch_halves<false>(s, q, k, v, out, stream, NoRows{});
    return launch_dw<D, 4>(s, q, k, v, out, stream);
  case 8:
    if constexpr (D == 128)
      return launch_dw<D, 8>(s, q, k, v, out, stream);
  }
  return hipErrorInvalidValue;
}

} // namespace

bool prefill_supported(const GqaShape &s) {
  const unsigned G = s.Hkv ? s.Hq / s.Hkv : 0;
  // A 64-key slice of one cache must stay within a buffer descriptor's
  // 32-bit range.
  const uint64_t sliceBytes = (uint64_t)BN * s.Hkv * s.D * 2;
  return (s.D == 128 || s.D == 256) && (G == 1 || G == 2 || G == 4 || G == 8) &&
         s.T >= 1 && sliceBytes < (1ull << 31);
}

bool prefill_gated_supported(const GqaShape &s, unsigned rot) {
  // One K/V buffer per wave holds the wave's rows, their scales and the
  // cos/sin table of its 32 tokens.
  const unsigned HW = s.D == 256 ? heads_per_wg<256>(s.Hkv ? s.Hq / s.Hkv : 0)
                                 : heads_per_wg<128>(s.Hkv ? s.Hq / s.Hkv : 0);
  // wave 0's buffer also holds the (1 + w) weights and the cos/sin table
  const size_t need = (size_t)BM * (s.D + 8) * 2 + BM * 4 + (size_t)s.D * 4 +
                      (size_t)BM * (rot / 2) * 4;
  return prefill_supported(s) && HW <= 4 && need <= (size_t)BN * 2 * s.D &&
         rot % 16 == 0 && rot <= s.D;
}

hipError_t launch_gqa_prefill_gated(const uint16_t *k, const uint16_t *v, uint16_t *out,
                                    const GqaShape &s, const GatedRows &ga,
                                    hipStream_t stream) {
  if (s.D == 128)
    return launch_gated_d<128>(s, k, v, out, ga, stream);
  return launch_gated_d<256>(s, k, v, out, ga, stream);
}

hipError_t launch_gqa_prefill(const uint16_t *q, const uint16_t *k,
                              const uint16_t *v, uint16_t *out,
                              const GqaShape &s, hipStream_t stream) {
  if (s.D == 128)
    return launch_d<128>(s, q, k, v, out, stream);
  return launch_d<256>(s, q, k, v, out, stream);
}

} // namespace llmi
