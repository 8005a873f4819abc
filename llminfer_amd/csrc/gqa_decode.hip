// Causal GQA decode: split-K over the KV cache.
//
// Replaces the reference's three decode dispatches gqaScores -> gqaSoftmax ->
// gqaValue (Reference.metal:303-323, Graph.metal:172-230) with one pass over
// K and V. It is an HBM-bandwidth problem (4 FLOP/byte), so no MFMA:
//
//  * grid = (split, kv head, token). A workgroup of 4 waves streams one key
//    range of one KV head and serves all G = Hq/Hkv query heads of the
//    group, so each K/V byte leaves HBM once.
//  * D/16 lanes share one key row: each lane holds 16 channels as two 16-byte
//    loads, so one wave instruction reads whole 256-byte row segments.
//  * q.k is v_dot2_f32_f16 on packed fp16 pairs, reduced over the lanes of a
//    key with DPP row permutes; softmax state (reference, sum) and the
//    output accumulator are fp32, with exp2 on log2e-prescaled scores.
//  * On MI355X this loop is VALU-bound before it is HBM-bound: a wave64 VALU
//    instruction occupies its 16-lane SIMD for 4 cycles, and with G = 4 every
//    key costs ~30 wave instructions (measured: with the K/V reads served
//    from L2 the loop alone takes 16 us at 32K). So the per-key arithmetic
//    is trimmed: the probabilities are packed to fp16 pairs and P.V is
//    v_dot2_f32_f16 over two keys at once (the sum l is taken from the same
//    rounded values, so numerator and denominator agree), and the softmax
//    reference is lazy -- it moves only when a score exceeds it by more than
//    2^8, so the rescale of the accumulators is almost never executed.
//  * One wave per SIMD (4-wave workgroups, ~256 VGPRs) with the K/V loads of
//    the next three sets in flight while one set is scored. (With two waves
//    per SIMD the older wave wins most VALU issue slots: per-wave timestamps
//    showed the second wave of every SIMD finishing ~8 us after the first.)
//  * each lane group runs its own online softmax over its keys; groups,
//    waves and finally splits are merged with the usual (m, l, o) rescale.
//  * a one-split launch writes the output directly. Otherwise every
//    workgroup writes its (m, l, o) partial to the workspace and a second,
//    small launch merges them: one 64-thread workgroup per 16 output channels
//    of a query head, four lanes per channel taking every fourth split, all
//    of the partial loads in flight at once. (Merging
//    inside the split kernel's last-arriving workgroup was measured slower on
//    MI355X: the partial stores then need agent-scope release -- a whole-L2
//    writeback per workgroup, which serialises -- and the single merging
//    workgroup reads all partials through one CU.)
//  * optionally (k_new/v_new non-null) the launch also performs the step's
//    KvAppend: keys [P, P+T) are read from the new rows rather than the
//    cache, and the workgroups of the last token write them into the cache
//    rows [P, P+T) -- the same bytes cacheAppend (Reference.metal:295-301)
//    writes, without a second launch.
#include "hip_common.hpp"
#include "kernels.hpp"
#include "rope_gate.hpp"

#include <algorithm>
#include <math.h>
#include <stdlib.h>
#include <type_traits>

namespace llmi {
namespace {

constexpr int kSlots = 2;         // keys per lane group in one loaded set
constexpr int kWaves = 4;         // waves per workgroup, one per SIMD
constexpr unsigned kMaxSplits = 128;
constexpr float kHeadroom = 8.0f; // log2 units a score may exceed the reference

// Sets in flight per wave: the loads of kRing - 1 sets overlap the scoring of
// one. Eight query heads per KV head need twice the accumulators, so less.
template <int G> constexpr int ring_depth() { return G <= 4 ? 4 : 2; }

template <int D> struct DecodeGeom {
  static constexpr int LPK = D / 16;            // lanes per key row
  static constexpr int KPR = 64 / LPK;          // key rows per wave instruction
  static constexpr int WaveTile = KPR * kSlots; // keys per wave and set
};

struct Plan {
  unsigned splits, keysPerSplit;
};

unsigned wave_tile(unsigned D) {
  switch (D) {
  case 64:
    return DecodeGeom<64>::WaveTile;
  case 128:
    return DecodeGeom<128>::WaveTile;
  default:
    return DecodeGeom<256>::WaveTile;
  }
}

// Tuning knob, read once. LLMI_DECODE_TARGET_WGS: resident workgroups to
// plan for (default 256: one per CU of MI355X).
unsigned env_or(const char *name, unsigned dflt) {
  const char *v = getenv(name);
  if (!v || !*v)
    return dflt;
  long x = strtol(v, nullptr, 10);
  return x > 0 ? (unsigned)x : dflt;
}

unsigned target_wgs() {
  static const unsigned v = env_or("LLMI_DECODE_TARGET_WGS", 256);
  return v;
}

// The kernel holds ~256 VGPRs, so a CU keeps one 4-wave workgroup resident.
// The plan gives every wave the fewest sets for which the whole grid is
// resident in one round.
Plan plan_for(const GqaShape &s) {
  const unsigned wt = wave_tile(s.D);
  const unsigned visible = s.P + s.T;
  const unsigned rows = s.T * s.Hkv;
  const unsigned budget = target_wgs() * kWaves; // resident waves to fill
  const uint64_t waveTiles = (uint64_t)rows * ((visible + wt - 1) / wt);
  const unsigned iters =
      (unsigned)std::max<uint64_t>(1, (waveTiles + budget - 1) / budget);
  unsigned kps = wt * kWaves * iters;
  unsigned splits = (visible + kps - 1) / kps;
  if (splits > kMaxSplits) { // very long contexts: more sets per wave
    kps = (visible + kMaxSplits - 1) / kMaxSplits;
    kps = (kps + wt * kWaves - 1) / (wt * kWaves) * (wt * kWaves);
    splits = (visible + kps - 1) / kps;
  }
  return {splits, kps};
}

struct WsLayout {
  size_t ml, o, total;
};

// Partials of a multi-split launch: (m, l) pairs, then o vectors.
WsLayout layout_for(const GqaShape &s, const Plan &p) {
  unsigned G = s.Hq / s.Hkv;
  size_t rows = (size_t)s.T * s.Hkv;
  WsLayout w;
  w.ml = 0;
  w.o = ((rows * p.splits * G * 2 * 4 + 255) / 256) * 256;
  w.total = p.splits > 1 ? w.o + rows * p.splits * G * s.D * 4 : 0;
  return w;
}

__device__ __forceinline__ float rescale(float m, float M) {
  return m == -INFINITY ? 0.0f : fast_exp2(m - M);
}

// Max / sum over the 64 lanes of a wave, the result in every lane.
__device__ __forceinline__ float wave_max(float x) {
  x = fmaxf(x, row_ror<1>(x));
  x = fmaxf(x, row_ror<2>(x));
  x = fmaxf(x, row_ror<4>(x));
  x = fmaxf(x, row_ror<8>(x));
  LanePair p = pair16(x);
  x = fmaxf(p.a, p.b);
  p = pair32(x);
  return fmaxf(p.a, p.b);
}

__device__ __forceinline__ float wave_sum(float x) {
  x += row_ror<1>(x);
  x += row_ror<2>(x);
  x += row_ror<4>(x);
  x += row_ror<8>(x);
  LanePair p = pair16(x);
  x = p.a + p.b;
  p = pair32(x);
  return p.a + p.b;
}

struct NoRows {}; // the ungated kernels' (empty) row argument


// The gated decode's row work for one workgroup (kv head kvh, token 0):
// its G query rows through normRope into qv, and -- for the owner of the
// new key row P -- that key through normRope into the cache row P and the
// new V row into the value cache row P, both stores complete on return.
// Staged through LDS so that one lane per row runs the reference's
// sequential sum of squares (rmsScale, Reference.metal:98-103).
template <int D, int G> struct GatedStage {
  uint4_t row, vrow; // one 16-byte chunk of a q or k row, of the v row
};

template <int D, int G>
__device__ __forceinline__ void gated_fetch(const GatedRows &ga, unsigned P, unsigned kvh,
                                            unsigned Hq, unsigned Hkv, bool owner,
                                            unsigned tid, GatedStage<D, G> &st) {
  constexpr unsigned CPR = D / 8;
  const unsigned r = tid / CPR, col = tid % CPR;
  if (r < (unsigned)G)
    st.row = *reinterpret_cast<const uint4_t *>(ga.qproj + (size_t)(kvh * G + r) * 2 * D +
                                                8 * col);
  else if (r == (unsigned)G && owner)
    st.row = *reinterpret_cast<const uint4_t *>(ga.kproj + (size_t)kvh * D + 8 * col);
  if (owner && tid < CPR)
    st.vrow = *reinterpret_cast<const uint4_t *>(ga.vnew + (size_t)kvh * D + 8 * col);
  (void)P;
  (void)Hq;
  (void)Hkv;
}

template <int D, int G>
__device__ __forceinline__ void gated_finish(const GatedRows &ga, half_t *kc, half_t *vc,
                                             unsigned P, unsigned kvh, unsigned Hkv,
                                             bool owner, const GatedStage<D, G> &st,
                                             half8_t (&qv)[G][2], unsigned tid,
                                             unsigned slice) {
  constexpr unsigned CPR = D / 8, PITCH = D + 8;
  __shared__ __attribute__((aligned(16))) uint16_t sRow[(G + 1) * PITCH];
  __shared__ float sScale[G + 1];
  __shared__ float2 sCs[D / 2];
  const unsigned rows = owner ? G + 1 : G;
  const size_t prow = ((size_t)P * Hkv + kvh) * D; // cache row P of this kv head
  {
    const unsigned r = tid / CPR, col = tid % CPR;
    if (r < rows)
      *reinterpret_cast<uint4_t *>(sRow + r * PITCH + 8 * col) = st.row;
    if (owner && tid < CPR)
      *reinterpret_cast<uint4_t *>(vc + prow + 8 * tid) = st.vrow;
  }
  lds_sync();
  const unsigned half = ga.rot / 2;
  if (tid < rows) {
    // The sequential fma chain over the row, in index order.
    const uint4_t *row = reinterpret_cast<const uint4_t *>(sRow + tid * PITCH);
    float sum = 0.0f;
    for (unsigned c8 = 0; c8 < CPR; ++c8)
      sum = sumsq8(row[c8], sum);
    sScale[tid] = rms_scale_of(sum, D, ga.eps);
  }
  if (tid >= 64 && tid - 64 < half)
    sCs[tid - 64] = rope_cos_sin(__fdiv_rn((float)P, ga.freqs[tid - 64]));
  lds_sync();
  // Rotary items (a row and 8 pairs: chunks j0 and j0 + rot/2), then the
  // copied chunks, normalised with (1 + w) and written back in place (q) or
  // to the cache row P (the new key).
  const unsigned pchunks = half / 8, rest = CPR - 2 * pchunks;
  for (unsigned it = tid; it < rows * pchunks; it += 64 * kWaves) {
    const unsigned r = it / pchunks, j0 = 8 * (it % pchunks), j1 = j0 + half;
    uint16_t *row = sRow + r * PITCH;
    const float *w = r < (unsigned)G ? ga.qw : ga.kw;
    const float scale = sScale[r];
    const uint4_t qx = *reinterpret_cast<const uint4_t *>(row + j0);
    const uint4_t qy = *reinterpret_cast<const uint4_t *>(row + j1);
    uint4_t sx, sy;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint16_t bx = (uint16_t)(qx[e / 2] >> (16 * (e & 1)));
      const uint16_t by = (uint16_t)(qy[e / 2] >> (16 * (e & 1)));
      const float x = normed(bx, scale, 1.0f + w[j0 + e]);
      const float y = normed(by, scale, 1.0f + w[j1 + e]);
      const float2 cs = sCs[j0 + e];
      const uint32_t ox = rotate_x(x, y, cs), oy = rotate_y(x, y, cs);
      if (e & 1) {
        sx[e / 2] |= ox << 16;
        sy[e / 2] |= oy << 16;
      } else {
        sx[e / 2] = ox;
        sy[e / 2] = oy;
      }
    }
    if (r < (unsigned)G) {
      *reinterpret_cast<uint4_t *>(row + j0) = sx;
      *reinterpret_cast<uint4_t *>(row + j1) = sy;
    } else {
      *reinterpret_cast<uint4_t *>(kc + prow + j0) = sx;
      *reinterpret_cast<uint4_t *>(kc + prow + j1) = sy;
    }
  }
  for (unsigned it = tid; it < rows * rest; it += 64 * kWaves) {
    const unsigned r = it / rest, j0 = 8 * (2 * pchunks + it % rest);
    uint16_t *row = sRow + r * PITCH;
    const float *w = r < (unsigned)G ? ga.qw : ga.kw;
    const float scale = sScale[r];
    const uint4_t qx = *reinterpret_cast<const uint4_t *>(row + j0);
    uint4_t sx;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t lo = f2h(normed((uint16_t)(qx[e] & 0xFFFFu), scale, 1.0f + w[j0 + 2 * e]));
      const uint32_t hi =
          f2h(normed((uint16_t)(qx[e] >> 16), scale, 1.0f + w[j0 + 2 * e + 1]));
      sx[e] = lo | (hi << 16);
    }
    if (r < (unsigned)G)
      *reinterpret_cast<uint4_t *>(row + j0) = sx;
    else
      *reinterpret_cast<uint4_t *>(kc + prow + j0) = sx;
  }
  if (owner)
    __builtin_amdgcn_s_waitcnt(0); // the cache row P is written before any key load
  lds_sync();
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int j = 0; j < 2; ++j)
      qv[g][j] = *reinterpret_cast<const half8_t *>(sRow + g * PITCH + j * (D / 2) + slice * 8);
}

// GATED (one token): the attention block's row work around the decode --
// q and the new key through normRope, the new V row appended, the output
// through the sigmoid gate -- with every result the standalone row kernels'
// bits (rope_gate.hpp).
template <int D, int G, bool GATED>
__global__ __launch_bounds__(64 * kWaves) void gqa_decode_kernel(
    const half_t *__restrict__ q, half_t *kc, half_t *vc,
    const half_t *__restrict__ knew, const half_t *__restrict__ vnew,
    half_t *__restrict__ out, float *__restrict__ wml,
    float *__restrict__ wo, unsigned Hq, unsigned Hkv, unsigned P,
    unsigned T, unsigned keysPerSplit, unsigned splits, float scoreScale,
    typename std::conditional<GATED, GatedRows, NoRows>::type ga) {
  using Geo = DecodeGeom<D>;
  constexpr int LPK = Geo::LPK, KPR = Geo::KPR;
  constexpr int W = kWaves, NT = 64 * W;
  constexpr int Tile = Geo::WaveTile * W;
  constexpr int F4 = G * D / 4; // float4 columns of one (m, l, o) partial
  const unsigned split = blockIdx.x, kvh = blockIdx.y, t = blockIdx.z;
  const unsigned tid = threadIdx.x;
  const unsigned lane = tid & 63u, wave = tid >> 6;
  const unsigned slice = lane % LPK, kg = lane / LPK;
  const unsigned visible = P + t + 1;
  const unsigned begin = split * keysPerSplit;
  const unsigned end = min(begin + keysPerSplit, visible);
  const size_t rowStride = (size_t)Hkv * D;
  const bool fused = knew != nullptr;

  // Fused KvAppend: the last token's workgroups own the new rows of their
  // key range and copy them into the cache (nothing in this launch reads
  // those cache rows: new keys are taken from k_new/v_new below).
  if (fused && t == T - 1) {
    const unsigned r0 = max(begin, P), r1 = end;
    for (unsigned i = tid; i < (r1 > r0 ? r1 - r0 : 0u) * (D / 8); i += NT) {
      const unsigned r = r0 + i / (D / 8), c = (i % (D / 8)) * 8;
      const size_t src = (size_t)(r - P) * rowStride + (size_t)kvh * D + c;
      const size_t dst = (size_t)r * rowStride + (size_t)kvh * D + c;
      *reinterpret_cast<half8_t *>(kc + dst) = load8(knew + src);
      *reinterpret_cast<half8_t *>(vc + dst) = load8(vnew + src);
    }
  }

  // Channels of this lane: [j*D/2 + slice*8, +8) for j = 0, 1.
  half8_t qv[G][2];
  if constexpr (!GATED) {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        qv[g][j] = load8(q + ((size_t)t * Hq + kvh * G + g) * D + j * (D / 2) + slice * 8);
  }

  float m[G], l[G], o[G][16];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.0f;
#pragma unroll
    for (int x = 0; x < 16; ++x)
      o[g][x] = 0.0f;
  }

  const size_t chan = (size_t)kvh * D + slice * 8;

  // One set: kSlots keys of each lane group (KPR * kSlots keys per wave,
  // Tile per workgroup). Keys past the range are clamped to the last key
  // of the range (an L2 hit) and masked out of the softmax. The cache is
  // read once per step, so the loads are non-temporal (measured on a cold
  // 134 MB stream: 6.2 TB/s against 5.8 with default caching).
  struct KvSet {
    half8_t k[kSlots][2], v[kSlots][2];
  };
  auto load_set = [&](KvSet &st, unsigned base) {
    const unsigned first = base + wave * Geo::WaveTile + kg;
#pragma unroll
    for (int n = 0; n < kSlots; ++n) {
      const unsigned key = min(first + n * KPR, end - 1);
      const bool isNew = fused && key >= P;
      const half_t *kp = (isNew ? knew + (size_t)(key - P) * rowStride
                                : kc + (size_t)key * rowStride) + chan;
      const half_t *vp = (isNew ? vnew + (size_t)(key - P) * rowStride
                                : vc + (size_t)key * rowStride) + chan;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        st.k[n][j] = load8_stream(kp + j * (D / 2));
        st.v[n][j] = load8_stream(vp + j * (D / 2));
      }
    }
  };

  // Score one set and fold it into (m, l, o). m is a lazy reference, the
  // same in every lane of the wave: the probabilities are 2^(s - m), at most
  // 2^kHeadroom, and m (with l and o) is raised only when some score exceeds
  // it by more than that -- a wave-uniform branch taken a handful of times
  // per wave.
  auto consume_set = [&](const KvSet &st, unsigned base) {
    const unsigned first = base + wave * Geo::WaveTile + kg;
    float sc[kSlots][G];
#pragma unroll
    for (int n = 0; n < kSlots; ++n) {
      const bool ok = first + n * KPR < end;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float acc = dot8(qv[g][0], st.k[n][0], 0.0f);
        acc = dot8(qv[g][1], st.k[n][1], acc);
        acc = group_sum<LPK>(acc);
        sc[n][g] = ok ? acc * scoreScale : -INFINITY;
      }
    }
    float tmax[G];
    bool raise = false;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      tmax[g] = sc[0][g];
#pragma unroll
      for (int n = 1; n < kSlots; ++n)
        tmax[g] = fmaxf(tmax[g], sc[n][g]);
      raise |= tmax[g] > m[g] + kHeadroom;
    }
    if (__builtin_amdgcn_ballot_w64(raise)) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float mNew = wave_max(fmaxf(m[g], tmax[g])); // one m per wave
        const float alpha = rescale(m[g], mNew);
        l[g] *= alpha;
#pragma unroll
        for (int x = 0; x < 16; ++x)
          o[g][x] *= alpha;
        m[g] = mNew;
      }
    }
    // P.V two keys at a time: p of keys (2i, 2i+1) as an fp16 pair against
    // the two keys' values of one channel, gathered by a byte permute.
    const half2_t ones{(half_t)1.0f, (half_t)1.0f};
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float negm = m[g] == -INFINITY ? 0.0f : -m[g]; // nothing seen yet: p = 0
#pragma unroll
      for (int i = 0; i < kSlots / 2; ++i) {
        const half2_t pp = __builtin_bit_cast(
            half2_t, __builtin_amdgcn_cvt_pkrtz(fast_exp2(sc[2 * i][g] + negm),
                                                fast_exp2(sc[2 * i + 1][g] + negm)));
        l[g] = __builtin_amdgcn_fdot2(pp, ones, l[g], false);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const uint4_t a = __builtin_bit_cast(uint4_t, st.v[2 * i][j]);
          const uint4_t b = __builtin_bit_cast(uint4_t, st.v[2 * i + 1][j]);
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const half2_t lo =
                __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(b[w], a[w], 0x05040100u));
            const half2_t hi =
                __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(b[w], a[w], 0x07060302u));
            float &o0 = o[g][j * 8 + 2 * w], &o1 = o[g][j * 8 + 2 * w + 1];
            o0 = __builtin_amdgcn_fdot2(pp, lo, o0, false);
            o1 = __builtin_amdgcn_fdot2(pp, hi, o1, false);
          }
        }
      }
    }
  };

  // A ring of R sets: set i + R - 1 is requested before set i is scored. The
  // loop body covers R sets with compile-time buffer indices, and every path
  // into its header has the same loads outstanding, which keeps the
  // compiler's wait counts partial.
  constexpr int R = ring_depth<G>();
  KvSet buf[R];
  auto ring_prologue = [&]() {
#pragma unroll
    for (int r = 0; r < R - 1; ++r)
      load_set(buf[r], begin + r * Tile);
  };
  // GATED: the workgroup whose keys include the new row P writes that row
  // (normRoped K, raw V) to the cache before it loads any key; every other
  // workgroup starts its loads first and normalises q under them.
  const bool owner = GATED && begin <= P && P < end;
  GatedStage<D, G> gst;
  if constexpr (GATED)
    gated_fetch<D, G>(ga, P, kvh, Hq, Hkv, owner, tid, gst);
  if (begin < end && !owner)
    ring_prologue();
  if constexpr (GATED) {
    gated_finish<D, G>(ga, kc, vc, P, kvh, Hkv, owner, gst, qv, tid, slice);
    if (begin < end && owner)
      ring_prologue();
  }

  if (begin < end) {
    const unsigned sets = (end - begin + Tile - 1) / Tile;
    unsigned base = begin, i = 0;
    for (; i + R <= sets; i += R) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        load_set(buf[(r + R - 1) % R], base + (r + R - 1) * Tile);
        consume_set(buf[r], base + r * Tile);
      }
      base += R * Tile;
    }
#pragma unroll
    for (int r = 0; r < R - 1; ++r)
      if (i + r < sets)
        consume_set(buf[r], base + r * Tile);
  }

  // Combine. m is wave-uniform, so the lane groups of a wave add up plainly:
  // inside each 16-lane row by DPP rotations, and for G*D > 1024 the two
  // row pairs by the gfx950 half-wave swap. The kRows row partials of every
  // wave then meet in LDS, where each thread combines one float4 column
  // across waves with the (m, l) rescale.
  constexpr int kRows = G * D <= 1024 ? 4 : 2;
  auto fold = [](float &x) {
    if constexpr (LPK <= 4)
      x += row_ror<4>(x);
    if constexpr (LPK <= 8)
      x += row_ror<8>(x);
    if constexpr (kRows == 2) {
      const LanePair p = pair32(x);
      x = p.a + p.b;
    }
  };
#pragma unroll
  for (int g = 0; g < G; ++g) {
    fold(l[g]);
#pragma unroll
    for (int x = 0; x < 16; ++x)
      fold(o[g][x]);
  }

  __shared__ float sM[W][G], sL[W][kRows][G];
  __shared__ __attribute__((aligned(16))) float sO[W][kRows][G][D];
  const unsigned rowi = lane / 16;
  if (lane == 0)
#pragma unroll
    for (int g = 0; g < G; ++g)
      sM[wave][g] = m[g];
  if (lane % 16 < (unsigned)LPK && rowi < (unsigned)kRows) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if (slice == 0)
        sL[wave][rowi][g] = l[g];
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          *reinterpret_cast<float4_t *>(&sO[wave][rowi][g][j * (D / 2) + slice * 8 + 4 * h]) =
              float4_t{o[g][j * 8 + 4 * h], o[g][j * 8 + 4 * h + 1], o[g][j * 8 + 4 * h + 2],
                       o[g][j * 8 + 4 * h + 3]};
    }
  }
  __syncthreads();

  // Column i: head g, channels [x, x + 4). Returns sum_w a_w o_w and L.
  auto combine = [&](unsigned i, float &M, float &L) {
    const unsigned g = i * 4 / D, x = i * 4 % D;
    M = sM[0][g];
#pragma unroll
    for (int w = 1; w < W; ++w)
      M = fmaxf(M, sM[w][g]);
    L = 0.0f;
    float4_t acc{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const float a = rescale(sM[w][g], M);
#pragma unroll
      for (int r = 0; r < kRows; ++r) {
        L = fmaf(sL[w][r][g], a, L);
        const float4_t v = *reinterpret_cast<const float4_t *>(&sO[w][r][g][x]);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          acc[e] = fmaf(v[e], a, acc[e]);
      }
    }
    return acc;
  };

  if (splits == 1) {
    half_t *orow = out + ((size_t)t * Hq + kvh * G) * D;
    for (unsigned i = tid; i < (unsigned)F4; i += NT) {
      float M, L;
      const float4_t acc = combine(i, M, L);
      const float inv = 1.0f / L;
      const unsigned g = i * 4 / D, x = i * 4 % D;
      half4_t y{f16_of(acc[0] * inv), f16_of(acc[1] * inv), f16_of(acc[2] * inv),
                f16_of(acc[3] * inv)};
      if constexpr (GATED) {
        const half_t *gr = ga.qproj + ((size_t)t * Hq + kvh * G + g) * 2 * D + D + x;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          y[e] = __builtin_bit_cast(half_t, gate_out((float)gr[e], (float)y[e], ga.activated));
      }
      *reinterpret_cast<half4_t *>(orow + g * D + x) = y;
    }
    return;
  }

  // Write this split's partial; the merge launch reads it.
  const size_t row = (size_t)t * Hkv + kvh;
  float *po = wo + (row * splits + split) * (size_t)(G * D);
  float *pml = wml + (row * splits + split) * (size_t)(G * 2);
  for (unsigned i = tid; i < (unsigned)F4; i += NT) {
    float M, L;
    const float4_t acc = combine(i, M, L);
    *reinterpret_cast<float4_t *>(po + i * 4) = acc;
    if (i * 4 % D == 0) {
      const unsigned g = i * 4 / D;
      pml[g * 2 + 0] = M;
      pml[g * 2 + 1] = L;
    }
  }
}

// Second-launch merge: workgroup (16-channel block, g, row) combines the
// splits of 16 output channels of query head g of one (token, kv head) row.
// Lane l serves channel l % 16 for the splits s = l / 16 + 4 u: every lane
// has at most kMaxSplits / 4 loads in flight at once, and the grid has 4x
// as many workgroups as 64-channel blocks would (each CU's share of the
// partials arrives in fewer, shorter chains). The four quarter sums meet
// through lane swaps, in a fixed order.
constexpr unsigned kMergeCols = 16;
template <int D, int G, bool GATED>
__global__ __launch_bounds__(64) void gqa_decode_merge_kernel(
    const float *__restrict__ wml, const float *__restrict__ wo,
    half_t *__restrict__ out, unsigned Hq, unsigned Hkv, unsigned splits,
    const half_t *__restrict__ qproj, unsigned activated) {
  static_assert(D % kMergeCols == 0, "whole channel blocks");
  const unsigned lane = threadIdx.x, g = blockIdx.y, row = blockIdx.z;
  const unsigned x = blockIdx.x * kMergeCols + lane % 16, quarter = lane / 16;
  const float *col = wo + (size_t)row * splits * G * D + (size_t)g * D + x;
  const float *rowMl = wml + (size_t)row * splits * G * 2;
  // Split indices past the last are clamped (valid addresses, zero
  // weight), so the loads carry no branches and all go out at once.
  constexpr int PER = kMaxSplits / 4;
  const unsigned last = splits - 1;
  float v[PER];
#pragma unroll
  for (int u = 0; u < PER; ++u)
    if (u < 16 || splits > 64)
      v[u] = col[(size_t)min(quarter + 4u * u, last) * G * D];
  float ms[2], ls[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const unsigned s = lane + 64u * h, sc = min(s, last);
    const float m = rowMl[(sc * G + g) * 2 + 0], l = rowMl[(sc * G + g) * 2 + 1];
    ms[h] = s < splits ? m : -INFINITY;
    ls[h] = s < splits ? l : 0.0f;
  }
  const float M = wave_max(fmaxf(ms[0], ms[1]));
  const float L = wave_sum(ls[0] * rescale(ms[0], M) + ls[1] * rescale(ms[1], M));
  const float invL = 1.0f / L;
  static_assert(kMaxSplits == 128, "two weights per lane");
  __shared__ float sW[kMaxSplits];
#pragma unroll
  for (int h = 0; h < 2; ++h)
    sW[lane + 64 * h] = rescale(ms[h], M) * invL; // 0 past the last split
  __syncthreads();
  float acc = 0.0f;
#pragma unroll
  for (int u = 0; u < PER; ++u)
    if (u < 16 || splits > 64)
      acc = fmaf(v[u], sW[quarter + 4u * u], acc); // weight 0 past the last split
  LanePair p = pair16(acc);
  acc = p.a + p.b;
  p = pair32(acc);
  acc = p.a + p.b;
  if (quarter != 0)
    return;
  const unsigned t = row / Hkv, kvh = row % Hkv;
  const half_t y = f16_of(acc);
  if constexpr (GATED)
    out[((size_t)t * Hq + kvh * G + g) * D + x] = __builtin_bit_cast(
        half_t, gate_out((float)qproj[((size_t)t * Hq + kvh * G + g) * 2 * D + D + x], (float)y,
                         activated));
  else
    out[((size_t)t * Hq + kvh * G + g) * D + x] = y;
}

inline unsigned activation_of(const NoRows &) { return 0; }
inline unsigned activation_of(const GatedRows &ga) { return ga.activated; }

template <int D, int G, bool GATED, typename Rows>
hipError_t launch_dgg(const GqaShape &s, const uint16_t *q, uint16_t *k,
                      uint16_t *v, const uint16_t *knew, const uint16_t *vnew,
                      uint16_t *out, void *ws, const Rows &ga, const half_t *qproj,
                      hipStream_t stream) {
  const Plan p = plan_for(s);
  const WsLayout w = layout_for(s, p);
  char *base = static_cast<char *>(ws);
  const float scale = kLog2e / sqrtf((float)D);
  hipLaunchKernelGGL((gqa_decode_kernel<D, G, GATED>), dim3(p.splits, s.Hkv, s.T),
                     dim3(64 * kWaves), 0, stream,
                     reinterpret_cast<const half_t *>(q),
                     reinterpret_cast<half_t *>(k), reinterpret_cast<half_t *>(v),
                     reinterpret_cast<const half_t *>(knew),
                     reinterpret_cast<const half_t *>(vnew),
                     reinterpret_cast<half_t *>(out),
                     reinterpret_cast<float *>(base ? base + w.ml : nullptr),
                     reinterpret_cast<float *>(base ? base + w.o : nullptr), s.Hq,
                     s.Hkv, s.P, s.T, p.keysPerSplit, p.splits, scale, ga);
  if (p.splits > 1) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
      return e;
    hipLaunchKernelGGL((gqa_decode_merge_kernel<D, G, GATED>), dim3(D / kMergeCols, G, s.T * s.Hkv),
                       dim3(64), 0, stream, reinterpret_cast<float *>(base + w.ml),
                       reinterpret_cast<float *>(base + w.o),
                       reinterpret_cast<half_t *>(out), s.Hq, s.Hkv, p.splits, qproj,
                       activation_of(ga));
  }
  return hipGetLastError();
}

template <int D, int G>
hipError_t launch_dg(const GqaShape &s, const uint16_t *q, uint16_t *k,
                     uint16_t *v, const uint16_t *knew, const uint16_t *vnew,
                     uint16_t *out, void *ws, hipStream_t stream) {
  return launch_dgg<D, G, false>(s, q, k, v, knew, vnew, out, ws, NoRows{}, nullptr, stream);
}

template <int D>
hipError_t launch_d(const GqaShape &s, const uint16_t *q, uint16_t *k,
                    uint16_t *v, const uint16_t *knew, const uint16_t *vnew,
                    uint16_t *out, void *ws, hipStream_t stream) {
  switch (s.Hq / s.Hkv) {
  case 1:
    return launch_dg<D, 1>(s, q, k, v, knew, vnew, out, ws, stream);
  case 2:
    return launch_dg<D, 2>(s, q, k, v, knew, vnew, out, ws, stream);
  case 4:
    return launch_dg<D, 4>(s, q, k, v, knew, vnew, out, ws, stream);
  case 8:
    return launch_dg<D, 8>(s, q, k, v, knew, vnew, out, ws, stream);
  }
  return hipErrorInvalidValue;
}

} // namespace

bool decode_supported(const GqaShape &s) {
  unsigned G = s.Hkv ? s.Hq / s.Hkv : 0;
  bool dOk = s.D == 64 || s.D == 128 || s.D == 256;
  bool gOk = G == 1 || G == 2 || G == 4 || G == 8;
  return dOk && gOk && s.T >= 1 && s.T <= 64;
}

size_t decode_workspace_bytes(const GqaShape &s) {
  return layout_for(s, plan_for(s)).total;
}

unsigned decode_splits(const GqaShape &s) { return plan_for(s).splits; }

unsigned decode_launches(const GqaShape &s) { return plan_for(s).splits > 1 ? 2 : 1; }

bool decode_gated_supported(const GqaShape &s, unsigned rot) {
  const unsigned G = s.Hkv ? s.Hq / s.Hkv : 0;
  return s.T == 1 && decode_supported(s) && (s.D == 128 || s.D == 256) &&
         (G == 2 || G == 4) && rot % 16 == 0 && rot <= s.D;
}

hipError_t launch_gqa_decode_gated(uint16_t *k, uint16_t *v, uint16_t *out, void *ws,
                                   const GqaShape &s, const GatedRows &ga,
                                   hipStream_t stream) {
  const half_t *qp = reinterpret_cast<const half_t *>(ga.qproj);
  if (s.D == 256 && s.Hq == 4 * s.Hkv)
    return launch_dgg<256, 4, true>(s, nullptr, k, v, nullptr, nullptr, out, ws, ga, qp,
                                    stream);
  if (s.D == 128 && s.Hq == 4 * s.Hkv)
    return launch_dgg<128, 4, true>(s, nullptr, k, v, nullptr, nullptr, out, ws, ga, qp,
                                    stream);
  if (s.D == 256 && s.Hq == 2 * s.Hkv)
    return launch_dgg<256, 2, true>(s, nullptr, k, v, nullptr, nullptr, out, ws, ga, qp,
                                    stream);
  if (s.D == 128 && s.Hq == 2 * s.Hkv)
    return launch_dgg<128, 2, true>(s, nullptr, k, v, nullptr, nullptr, out, ws, ga, qp,
                                    stream);
  return hipErrorInvalidValue;
}

hipError_t launch_gqa_decode(const uint16_t *q, uint16_t *k, uint16_t *v,
                             const uint16_t *knew, const uint16_t *vnew,
                             uint16_t *out, void *ws, const GqaShape &s,
                             hipStream_t stream) {
  switch (s.D) {
  case 64:
    return launch_d<64>(s, q, k, v, knew, vnew, out, ws, stream);
  case 128:
    return launch_d<128>(s, q, k, v, knew, vnew, out, ws, stream);
  case 256:
    return launch_d<256>(s, q, k, v, knew, vnew, out, ws, stream);
  }
  return hipErrorInvalidValue;
}

} // namespace llmi
