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
#include "hip_common.hpp"
#include "kernels.hpp"

#include <math.h>

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

__device__ __forceinline__ void wait_loads() {
  __builtin_amdgcn_s_waitcnt(0x0F70); // vmcnt(0)
}

// ds_read_b64_tr_b16: in each 16-lane group, lane j receives element j % 4 of
// the 8-byte chunks addressed by lanes j/4, 4 + j/4, 8 + j/4, 12 + j/4.
__device__ __forceinline__ half4_t read_tr(const char *p) {
  return __builtin_bit_cast(half4_t, __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_fp16x4_t *)p));
}

template <int D, int HW>
__global__ __attribute__((amdgpu_flat_work_group_size(64 * HW, 64 * HW),
                          amdgpu_waves_per_eu(D == 128 ? 2 : 1, D == 128 ? 2 : 1)))
void gqa_prefill_kernel(const half_t *__restrict__ q, const half_t *__restrict__ kc,
                        const half_t *__restrict__ vc, half_t *__restrict__ out,
                        unsigned T, unsigned Hq, unsigned Hkv, unsigned P,
                        unsigned groups, unsigned nb, float c) {
  constexpr int KS = D / 16;         // k-steps of S^T over channels
  constexpr int DT = D / 32;         // 32-channel output tiles
  constexpr int ROWB = 2 * D;        // bytes per K/V row
  constexpr int TILEB = BN * ROWB;   // bytes per K or V tile
  constexpr int NIW = TILEB / 1024 / HW; // 1-KB LDS loads per wave per tile
  constexpr int CPR = D / 8;         // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;      // rows per 1-KB load
  static_assert(NIW >= 1 && TILEB % (1024 * HW) == 0, "tile/waves");

  __shared__ __attribute__((aligned(1024))) char sK0[TILEB], sK1[TILEB];
  __shared__ __attribute__((aligned(1024))) char sV0[TILEB], sV1[TILEB];

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

  // Per-lane source offsets of this wave's loads (constant over tiles):
  // load n writes rows [n*RPI, n*RPI + RPI) of the tile.
  unsigned koff[NIW], voff[NIW];
#pragma unroll
  for (int i = 0; i < NIW; ++i) {
    const unsigned row = (wave + HW * i) * RPI + lane / CPR, slot = lane % CPR;
    koff[i] = row * (unsigned)rowBytes + 16 * (slot ^ (row & 7));
    voff[i] = row * (unsigned)rowBytes + 16 * (slot ^ ((row & 3) << 1));
  }
  auto rsrc = [&](const char *base, unsigned tile) {
    const unsigned first = tile * BN;
    const unsigned rows = min((unsigned)BN, kend - first);
    return __builtin_amdgcn_make_buffer_rsrc((void *)(base + (size_t)first * rowBytes),
                                             (short)0, (int)(rows * rowBytes), kBufferWord3);
  };
  auto issue_k = [&](unsigned tile, char *dst) {
    const __amdgpu_buffer_rsrc_t rs = rsrc(kbase, tile);
#pragma unroll
    for (int i = 0; i < NIW; ++i)
      load_lds16(rs, dst + 1024 * (wave + HW * i), koff[i]);
  };
  auto issue_v = [&](unsigned tile, char *dst) {
    const __amdgpu_buffer_rsrc_t rs = rsrc(vbase, tile);
#pragma unroll
    for (int i = 0; i < NIW; ++i)
      load_lds16(rs, dst + 1024 * (wave + HW * i), voff[i]);
  };

  // Operand read offsets. K (A of S^T, row 32kt + r, chunk 2s + hi): the
  // swizzle only touches the low 3 chunk bits, so s = 4a + b reads
  // kread[b] + 128a. V^T via the transposing read: lane j of a 16-lane group
  // addresses row k0 + j/4, channels 16g + 4(j%4) .. +3 of an output tile.
  unsigned kread[4];
#pragma unroll
  for (int b = 0; b < 4; ++b)
    kread[b] = r * ROWB + 16 * ((2 * b + hi) ^ (r & 7));
  const unsigned j16 = lane % 16, g = (lane / 16) % 2;
  const unsigned vx = 2 * (j16 / 4), vb = (j16 % 4) / 2;
  const unsigned vrow = (4 * hi + j16 / 4) * ROWB + 8 * (j16 % 2);
  const unsigned vread[2] = {vrow + 16 * ((2 * g + vb) ^ vx),
                             vrow + 16 * ((4 + 2 * g + vb) ^ vx)};

  // Q^T as the MFMA B operand: lane holds query row r, channels
  // 16 s + 8 hi + [0, 8). Rows past T use zeros (their output is dropped).
  half8_t qb[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s)
    qb[s] = rowValid ? load8(q + ((size_t)tq * Hq + h) * D + 16 * s + 8 * hi)
                     : half8_t{0, 0, 0, 0, 0, 0, 0, 0};

  float16_t oacc[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i)
    oacc[i] = float16_t{0};
  float mRef = -INFINITY, lRun = 0.0f;
  half8_t pb[2][2]; // P^T B operands of the previous tile, [32-key half][16-key step]

  // The two 32-key halves are independent accumulation chains; alternating
  // them keeps the MFMA pipe full.
  auto scores = [&](const char *sk, float16_t (&sacc)[2]) {
    sacc[0] = float16_t{0};
    sacc[1] = float16_t{0};
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
        sacc[kt] = mfma32x32x16(load8(reinterpret_cast<const half_t *>(
                                    sk + kread[s % 4] + 128 * (s / 4) + 32 * ROWB * kt)),
                                qb[s], sacc[kt]);
  };
  auto pv = [&](const char *sv) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int m = 0; m < 2; ++m) {
          const char *p = sv + vread[dt % 2] + 128 * (dt / 2) + ROWB * (32 * kt + 16 * m);
          half4_t lo = read_tr(p), up = read_tr(p + 8 * ROWB);
          half8_t a{lo[0], lo[1], lo[2], lo[3], up[0], up[1], up[2], up[3]};
          oacc[dt] = mfma32x32x16(a, pb[kt][m], oacc[dt]);
        }
  };
  // Softmax of one tile: masks, moves the reference if needed, writes the
  // fp16 probabilities into pb and returns the rescale factor of O.
  auto softmax = [&](const float16_t (&sacc)[2], unsigned base, bool masked, bool &raised) {
    float sv[2][16];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int v = 0; v < 16; ++v)
        sv[kt][v] = sacc[kt][v];
    if (masked) {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const unsigned key = base + 32 * kt + mfma_c_row(v, hi);
          if (key > P + tq)
            sv[kt][v] = -INFINITY;
        }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int v = 0; v < 16; ++v)
        mx = fmaxf(mx, sv[kt][v]);
    const LanePair pr = pair32(mx);
    const float tm = fmaxf(pr.a, pr.b) * c;
    const bool need = tm - mRef > kRaise;
    const float mNew = need ? tm - kHeadroom : mRef;
    const float alpha = fast_exp2(mRef - mNew);
    const float negm = -mNew;
    float psum = 0.0f;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float p = fast_exp2(fmaf(sv[kt][8 * m + e], c, negm));
          psum += p;
          pb[kt][m][e] = (half_t)p;
        }
    lRun = lRun * alpha + psum;
    mRef = mNew;
    raised = __builtin_amdgcn_ballot_w64(need) != 0;
    return alpha;
  };

  // V buffers start zeroed: rows past the block's last key are never
  // written by the range-checked loads, and a probability of 0 must not
  // meet a non-finite leftover.
  {
    const uint4_t z{0, 0, 0, 0};
    for (unsigned i = threadIdx.x * 16; i < (unsigned)TILEB; i += 64 * HW * 16) {
      *reinterpret_cast<uint4_t *>(sV0 + i) = z;
      *reinterpret_cast<uint4_t *>(sV1 + i) = z;
    }
  }
  __syncthreads();
  issue_k(0, sK0);
  issue_v(0, sV0);
  wait_loads();
  __syncthreads();
  if (tiles > 1)
    issue_k(1, sK1);
  {
    float16_t sacc[2];
    bool raised;
    scores(sK0, sacc);
    softmax(sacc, 0, BN > P + t0 + 1, raised); // O is still zero: nothing to rescale
  }

  // Step i: scores of tile i, PV of tile i-1, softmax of tile i, with the
  // loads of K(i+1) and V(i) in flight. Buffers are named statically (the
  // steady-state loop runs in pairs) so the compiler can tell the loads in
  // flight from the LDS reads and need not wait for them.
  auto step = [&](unsigned i, const char *kcur, const char *vprev, char *knext, char *vdst) {
    wait_loads();
    __syncthreads();
    if (i + 1 < tiles)
      issue_k(i + 1, knext);
    issue_v(i, vdst);
    float16_t sacc[2];
    bool raised;
    scores(kcur, sacc);
    pv(vprev);
    const float alpha = softmax(sacc, i * BN, i * BN + BN > P + t0 + 1, raised);
    if (raised) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
        oacc[dt] *= alpha;
    }
  };
  unsigned i = 1;
  for (; i + 1 < tiles; i += 2) {
    step(i, sK1, sV0, sK0, sV1);
    step(i + 1, sK0, sV1, sK1, sV0);
  }
  if (i < tiles) // i == tiles - 1, odd
    step(i, sK1, sV0, sK0, sV1);
  wait_loads();
  __syncthreads();
  if ((tiles - 1) % 2 == 0)
    pv(sV0);
  else
    pv(sV1);

  const LanePair lp = pair32(lRun);
  if (!rowValid)
    return;
  const float inv = 1.0f / (lp.a + lp.b);
  half_t *orow = out + ((size_t)tq * Hq + h) * D;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      half4_t v{(half_t)(oacc[dt][4 * g4 + 0] * inv), (half_t)(oacc[dt][4 * g4 + 1] * inv),
                (half_t)(oacc[dt][4 * g4 + 2] * inv), (half_t)(oacc[dt][4 * g4 + 3] * inv)};
      *reinterpret_cast<half4_t *>(orow + 32 * dt + 8 * g4 + 4 * hi) = v;
    }
}

template <int D> constexpr unsigned heads_per_wg(unsigned G) {
  return G < (D == 256 ? 4u : 8u) ? G : (D == 256 ? 4u : 8u);
}

template <int D, int HW>
hipError_t launch_dw(const GqaShape &s, const uint16_t *q, const uint16_t *k,
                     const uint16_t *v, uint16_t *out, hipStream_t stream) {
  const float c = kLog2e / sqrtf((float)D);
  const unsigned G = s.Hq / s.Hkv, groups = G / HW, nb = (s.T + BM - 1) / BM;
  hipLaunchKernelGGL((gqa_prefill_kernel<D, HW>), dim3(nb * s.Hkv * groups), dim3(64 * HW), 0,
                     stream, reinterpret_cast<const half_t *>(q),
                     reinterpret_cast<const half_t *>(k), reinterpret_cast<const half_t *>(v),
                     reinterpret_cast<half_t *>(out), s.T, s.Hq, s.Hkv, s.P, groups, nb, c);
  return hipGetLastError();
}

template <int D>
hipError_t launch_d(const GqaShape &s, const uint16_t *q, const uint16_t *k,
                    const uint16_t *v, uint16_t *out, hipStream_t stream) {
  switch (heads_per_wg<D>(s.Hq / s.Hkv)) {
  case 1:
    return launch_dw<D, 1>(s, q, k, v, out, stream);
  case 2:
    return launch_dw<D, 2>(s, q, k, v, out, stream);
  case 4:
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

hipError_t launch_gqa_prefill(const uint16_t *q, const uint16_t *k,
                              const uint16_t *v, uint16_t *out,
                              const GqaShape &s, hipStream_t stream) {
  if (s.D == 128)
    return launch_d<128>(s, q, k, v, out, stream);
  return launch_d<256>(s, q, k, v, out, stream);
}

} // namespace llmi
