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
// fma chain (four interleaved chains per 16-row unit (8 at dk = 64), the 8
// unit sums added in order through LDS); the result stays within fp32
// rounding of the sequential order, and it does not depend on how the rows
// are split between lanes (the one-workgroup-per-head variant below gives
// the same bits as the default slices).
//
// With QK16 the kernel also performs the L2 normalisations of q and k that
// precede DeltaUpdate (l2NormF32, Graph.metal:96-109): q and k arrive as the
// fp16 rows the convolution produced, one lane per (token, q or k) row runs
// the reference's sequential sum of squares and forms the row factor, and
// every fp32 element is the single product x * factor -- the bits l2NormF32
// writes, so the update sees exactly the operands of the unfused pair.
#include "exact_fp.hpp"
#include "gated_norm.hpp"
#include "hip_common.hpp"
#include "kernels.hpp"

#include <stdlib.h>
#include <type_traits>

namespace llmi {
namespace {

// With NORM (and CG column groups of NW waves each, the workgroup holding
// all CG * CW columns of a value head) the kernel ends with gatedRmsNorm
// over the head's output rows (Reference.metal:228-259): the fp16 outputs
// of the T <= kRecNormMaxT tokens wait in LDS, one thread per row runs the
// row's sequential sum of squares, and every element becomes fp16(fp16(x *
// factor) * weight * silu(gate)) (gated_norm.hpp, the standalone kernel's
// arithmetic). The gate and weight values are requested at the start.
// With ACTQ the gate is the fp32 activated one (gatedRmsNorm with the
// projection's SiLU epilogue: fp16(fp16(x * factor) * weight * gate)) and
// the normalised rows are also quantized (quantizeActivation over the
// flattened [T][Hv*dv] rows: a head's row is dv / 32 whole groups), the
// bits of the standalone gated_rms_norm_tile<true, true>.
template <int DK, int CW, int NW, bool QK16, int CG = 1, bool NORM = false, bool ACTQ = false>
__global__ __launch_bounds__(64 * NW * CG) void delta_recurrent_kernel(
    const void *__restrict__ qp, const void *__restrict__ kp,
    const half_t *__restrict__ v, const float *__restrict__ beta,
    const float *__restrict__ decay, float *__restrict__ state,
    half_t *__restrict__ out, unsigned T, unsigned Hk, unsigned Hv,
    unsigned DV, float eps, float qscale, const void *__restrict__ gate,
    const float *__restrict__ nweight, float neps, int8_t *__restrict__ qout,
    float *__restrict__ scales, unsigned *invalid) {
  constexpr int RG = 64 / CW;  // row groups per wave
  constexpr int NP = NW * RG;  // lanes (row parts) per column
  constexpr int RPL = DK / NP; // rows per lane
  // The dot products are summed in NU canonical units of UR consecutive rows
  // (each four interleaved fma chains, then (c0 + c1) + (c2 + c3)), the
  // units added in row order: the same bits whatever the partition, as long
  // as NP <= 8 (a lane then holds UPL whole units).
  constexpr int NU = NP <= 8 ? 8 : NP, UR = DK / NU, UPL = RPL / UR;
  constexpr int kThreads = 64 * NW * CG;
  static_assert(RPL % 4 == 0 && RPL * NP == DK, "rows per lane must be a multiple of 4");
  static_assert(UR % 4 == 0 && UR * UPL == RPL, "a lane holds whole units");
  static_assert(!NORM || CW == 64, "the fused norm's workgroup holds 64-column groups");
  static_assert(!ACTQ || NORM, "the quantization follows the fused norm");
  const unsigned tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const unsigned cg = wave / NW, wv = wave % NW;
  const unsigned c = lane % CW, part = wv * RG + lane / CW;
  const unsigned slices = DV / (CW * CG);
  const unsigned h = blockIdx.x / slices;
  const unsigned col = (blockIdx.x % slices) * (CW * CG) + cg * CW + c;
  const unsigned kh = h / (Hv / Hk);
  const unsigned row0 = part * RPL;
  const size_t vwidth = (size_t)Hv * DV;

  __shared__ float sPred[CG][NU][CW], sY[CG][NU][CW];
  // With NORM the state is requested first: the largest read, in flight
  // while the operands below are staged (requested after them, it was
  // waited behind their staging, ~1.6 us into the kernel).
  float S[RPL];
  float *sbase = state + ((size_t)h * DK + row0) * DV + col;
  auto load_state = [&] {
#pragma unroll
    for (int m = 0; m < RPL; ++m)
      S[m] = sbase[(size_t)m * DV];
  };
  if constexpr (NORM)
    load_state();
  // NORM: the outputs x of the tokens (fp16, as the unfused kernel stores
  // them), the row factors, and the head's gate rows and the weight, staged
  // at the start (no register holds them across the token loop).
  constexpr int NX = NORM ? kRecNormMaxT : 1, NC = NORM ? CW * CG : 1;
  using GateT = typename std::conditional<ACTQ, float, half_t>::type;
  __shared__ __attribute__((aligned(16))) half_t sX[NX][NC];
  __shared__ __attribute__((aligned(16))) GateT sGate[NX][NC];
  __shared__ float sNF[NX], sW[NC];
  if constexpr (NORM) {
    for (unsigned i = tid; i < T * DV; i += kThreads)
      sGate[i / DV][i % DV] = static_cast<const GateT *>(
          gate)[(size_t)(i / DV) * vwidth + (size_t)h * DV + i % DV];
    for (unsigned j = tid; j < DV; j += kThreads)
      sW[j] = nweight[j];
  }
  // QK16: the L2 factors of kFacTok tokens' k and q rows at a time; thread
  // 2i (2i + 1) sums the k (q) row of the block's token i. The rows of the
  // first block are requested before the state, so that their sums run
  // while the state is in flight.
  // With NORM (T <= kRecNormMaxT, one block) the 2T rows are staged in LDS
  // by all threads instead, which keeps the row out of the registers.
  constexpr unsigned kFacTok = NORM ? kRecNormMaxT : 32 * NW * CG;
  __shared__ float sFac[QK16 ? 2 * kFacTok : 1];
  __shared__ uint4_t sFacRows[QK16 && NORM ? 2 * kRecNormMaxT * DK / 8 : 1];
  uint4_t facRow[QK16 && !NORM ? DK / 8 : 1];
  auto fetch_fac_row = [&](unsigned tb) {
    const unsigned tt = tb + tid / 2;
    const uint4_t *row = reinterpret_cast<const uint4_t *>(
        static_cast<const half_t *>((tid & 1u) ? qp : kp) + ((size_t)tt * Hk + kh) * DK);
#pragma unroll
    for (int c8 = 0; c8 < (QK16 && !NORM ? DK / 8 : 0); ++c8)
      facRow[c8] = row[c8];
  };
  if constexpr (QK16 && NORM) {
    // Row r = 2 t (+1 for q) of token t.
    for (unsigned i = tid; i < 2 * T * (DK / 8); i += kThreads) {
      const unsigned r = i / (DK / 8), c8 = i % (DK / 8);
      sFacRows[i] = reinterpret_cast<const uint4_t *>(
          static_cast<const half_t *>((r & 1u) ? qp : kp) + ((size_t)(r / 2) * Hk + kh) * DK)[c8];
    }
  } else if (QK16 && tid < 2 * min(kFacTok, T)) {
    fetch_fac_row(0);
  }

  if constexpr (!NORM)
    load_state();

  // A token's operands as loaded (fp16 q/k rows with QK16, else fp32). They
  // are fetched one token ahead, before the barriers of the token in hand,
  // so that no token waits for its own loads.
  using QkRaw = typename std::conditional<QK16, half4_t, float4_t>::type;
  struct Operands {
    QkRaw k[RPL / 4], q[RPL / 4];
    float a, b, vj;
  };
  auto fetch = [&](unsigned t, Operands &o) {
    const size_t qk = ((size_t)t * Hk + kh) * DK + row0;
    const QkRaw *kt = reinterpret_cast<const QkRaw *>(static_cast<const char *>(kp)) +
                      qk / 4;
    const QkRaw *qt = reinterpret_cast<const QkRaw *>(static_cast<const char *>(qp)) +
                      qk / 4;
#pragma unroll
    for (int m4 = 0; m4 < RPL / 4; ++m4) {
      o.k[m4] = kt[m4];
      o.q[m4] = qt[m4];
    }
    o.a = decay[(size_t)t * Hv + h];
    o.b = beta[(size_t)t * Hv + h];
    o.vj = (float)v[(size_t)t * vwidth + (size_t)h * DV + col];
  };
  Operands cur;
  fetch(0, cur);

  for (unsigned tb = 0; tb < T; tb += QK16 ? kFacTok : T) {
    const unsigned tn = QK16 ? min(kFacTok, T - tb) : T;
    if constexpr (QK16) {
      if (tb) {
        __syncthreads(); // the previous block's factors are no longer read
        if (tid < 2 * tn)
          fetch_fac_row(tb);
      }
      if constexpr (NORM)
        __syncthreads(); // the staged rows
      if (tid < 2 * tn) {
        float sum = 0.0f;
#pragma unroll
        for (int c8 = 0; c8 < DK / 8; ++c8)
          sum = sumsq8(NORM ? sFacRows[tid * (DK / 8) + c8] : facRow[c8], sum);
        sFac[tid] = l2_row_factor(sum, eps, (tid & 1u) ? qscale : 1.0f);
      }
      __syncthreads();
    }
    for (unsigned t = tb; t < tb + tn; ++t) {
      Operands nxt;
      if (t + 1 < T)
        fetch(t + 1, nxt);
      float kr[RPL], qr[RPL];
      const float fk = QK16 ? sFac[2 * (t - tb)] : 1.0f;
      const float fq = QK16 ? sFac[2 * (t - tb) + 1] : 1.0f;
#pragma unroll
      for (int m = 0; m < RPL; ++m) {
        if constexpr (QK16) {
          kr[m] = __fmul_rn((float)cur.k[m / 4][m % 4], fk);
          qr[m] = __fmul_rn((float)cur.q[m / 4][m % 4], fq);
        } else {
          kr[m] = cur.k[m / 4][m % 4];
          qr[m] = cur.q[m / 4][m % 4];
        }
      }
      const float a = cur.a, b = cur.b, vj = cur.vj;

      float p4[UPL][4];
#pragma unroll
      for (int u = 0; u < UPL; ++u)
        p4[u][0] = p4[u][1] = p4[u][2] = p4[u][3] = 0.0f;
#pragma unroll
      for (int m = 0; m < RPL; ++m)
        p4[m / UR][m % 4] = fmaf(S[m] * a, kr[m], p4[m / UR][m % 4]);
#pragma unroll
      for (int u = 0; u < UPL; ++u)
        sPred[cg][part * UPL + u][c] = (p4[u][0] + p4[u][1]) + (p4[u][2] + p4[u][3]);
      __syncthreads();
      float pred = 0.0f;
#pragma unroll
      for (int i = 0; i < NU; ++i)
        pred += sPred[cg][i][c];
      const float delta = (vj - pred) * b;

      float y4[UPL][4];
#pragma unroll
      for (int u = 0; u < UPL; ++u)
        y4[u][0] = y4[u][1] = y4[u][2] = y4[u][3] = 0.0f;
#pragma unroll
      for (int m = 0; m < RPL; ++m) {
        S[m] = fmaf(kr[m], delta, S[m] * a);
        y4[m / UR][m % 4] = fmaf(S[m], qr[m], y4[m / UR][m % 4]);
      }
#pragma unroll
      for (int u = 0; u < UPL; ++u)
        sY[cg][part * UPL + u][c] = (y4[u][0] + y4[u][1]) + (y4[u][2] + y4[u][3]);
      __syncthreads();
      if (part == 0) {
        float y = 0.0f;
#pragma unroll
        for (int i = 0; i < NU; ++i)
          y += sY[cg][i][c];
        if constexpr (NORM)
          sX[t][col] = (half_t)y;
        else
          out[(size_t)t * vwidth + (size_t)h * DV + col] = (half_t)y;
      }
      if (t + 1 < T)
        cur = nxt;
    }
  }

#pragma unroll
  for (int m = 0; m < RPL; ++m)
    sbase[(size_t)m * DV] = S[m];

  if constexpr (NORM) {
    __syncthreads();
    if (tid < T) {
      const uint4_t *row = reinterpret_cast<const uint4_t *>(&sX[tid][0]);
      float sum = 0.0f;
      for (unsigned k8 = 0; k8 < DV / 8; ++k8)
        sum = sumsq8(row[k8], sum);
      sNF[tid] = gated_norm_factor(sum, DV, neps);
    }
    __syncthreads();
    if constexpr (ACTQ) {
      // Chunks of eight: the four chunks of a 32-wide group are handled by
      // four consecutive lanes (dv / 8 is a multiple of 4).
      for (unsigned c8 = tid; c8 < T * (DV / 8); c8 += kThreads) {
        const unsigned t = c8 / (DV / 8), j0 = c8 % (DV / 8) * 8;
        const size_t base = (size_t)t * vwidth + (size_t)h * DV + j0;
        float y[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
          y[e] = mul32(gated_norm_scaled((float)sX[t][j0 + e], sNF[t], sW[j0 + e]),
                       sGate[t][j0 + e]);
        uint4_t o;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          o[e] = (uint32_t)f2h(y[2 * e]) | ((uint32_t)f2h(y[2 * e + 1]) << 16);
        *reinterpret_cast<uint4_t *>(out + base) = o;
        quantize_chunk8(y, qout + base, scales + base / 32, invalid, (c8 & 3u) == 0);
      }
    } else {
      for (unsigned i = tid; i < T * DV; i += kThreads) {
        const unsigned t = i / DV, j = i % DV;
        out[(size_t)t * vwidth + (size_t)h * DV + j] =
            gated_norm_out((float)sX[t][j], sNF[t], sW[j], (float)sGate[t][j]);
      }
    }
  }
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

struct RecArgs {
  const void *q, *k;
  const uint16_t *v;
  const float *beta, *decay;
  float *state;
  uint16_t *out;
  float eps, qscale;
  const void *gate = nullptr;
  const float *nweight = nullptr;
  float neps = 0.0f;
  int8_t *qout = nullptr;
  float *scales = nullptr;
  unsigned *invalid = nullptr;
};

template <int DK, int CW, int NW, bool QK16, int CG = 1, bool NORM = false, bool ACTQ = false>
hipError_t launch_rec(const RecArgs &a, const DeltaShape &s, hipStream_t stream) {
  hipLaunchKernelGGL((delta_recurrent_kernel<DK, CW, NW, QK16, CG, NORM, ACTQ>),
                     dim3(s.Hv * (s.Dv / (CW * CG))), dim3(64 * NW * CG), 0, stream, a.q, a.k,
                     reinterpret_cast<const half_t *>(a.v), a.beta, a.decay, a.state,
                     reinterpret_cast<half_t *>(a.out), s.T, s.Hk, s.Hv, s.Dv, a.eps, a.qscale,
                     a.gate, a.nweight, a.neps, a.qout, a.scales, a.invalid);
  return hipGetLastError();
}

template <int DK, int CW, bool QK16>
hipError_t launch_rec_cw(const RecArgs &a, const DeltaShape &s, hipStream_t stream) {
  // Rows per lane DK / (NW * 64 / CW) must stay a multiple of 4.
  constexpr bool ok8 = DK % (8 * (64 / CW) * 4) == 0, ok2 = DK % (2 * (64 / CW) * 4) == 0;
  const unsigned nw = waves_per_group();
  if constexpr (ok8)
    if (nw == 8)
      return launch_rec<DK, CW, 8, QK16>(a, s, stream);
  if constexpr (ok2)
    if (nw == 2)
      return launch_rec<DK, CW, 2, QK16>(a, s, stream);
  return launch_rec<DK, CW, 4, QK16>(a, s, stream);
}

template <bool QK16>
hipError_t launch_rec_any(const RecArgs &a, const DeltaShape &s, hipStream_t stream) {
  const unsigned cw = slice_cols(s.Dv);
  if (s.Dk == 64) {
    if (cw == 64)
      return launch_rec_cw<64, 64, QK16>(a, s, stream);
    if (cw == 32)
      return launch_rec_cw<64, 32, QK16>(a, s, stream);
    return launch_rec_cw<64, 16, QK16>(a, s, stream);
  }
  if (cw == 64)
    return launch_rec_cw<128, 64, QK16>(a, s, stream);
  if (cw == 32)
    return launch_rec_cw<128, 32, QK16>(a, s, stream);
  return launch_rec_cw<128, 16, QK16>(a, s, stream);
}

} // namespace

bool delta_recurrent_norm_supported(const DeltaShape &s) {
  return (s.Dk == 64 || s.Dk == 128) && (s.Dv == 64 || s.Dv == 128) && s.Hk >= 1 &&
         s.Hv % s.Hk == 0 && s.T >= 1 && s.T <= kRecNormMaxT;
}

hipError_t launch_delta_recurrent_gated_norm(const uint16_t *q, const uint16_t *k,
                                             const uint16_t *v, const float *beta,
                                             const float *decay, float *state,
                                             const uint16_t *gate, const float *nweight,
                                             uint16_t *out, float eps, float qscale,
                                             float neps, const DeltaShape &s,
                                             hipStream_t stream) {
  RecArgs a{q, k, v, beta, decay, state, out, eps, qscale, gate, nweight, neps};
  if (s.Dk == 64)
    return s.Dv == 64 ? launch_rec<64, 64, 4, true, 1, true>(a, s, stream)
                      : launch_rec<64, 64, 4, true, 2, true>(a, s, stream);
  return s.Dv == 64 ? launch_rec<128, 64, 4, true, 1, true>(a, s, stream)
                    : launch_rec<128, 64, 4, true, 2, true>(a, s, stream);
}

hipError_t launch_delta_recurrent_gated_norm_quantize(
    const uint16_t *q, const uint16_t *k, const uint16_t *v, const float *beta,
    const float *decay, float *state, const float *gate, const float *nweight, uint16_t *out,
    int8_t *qout, float *scales, unsigned *invalid, float eps, float qscale, float neps,
    const DeltaShape &s, hipStream_t stream) {
  RecArgs a{q, k, v, beta, decay, state, out, eps, qscale, gate, nweight, neps,
            qout, scales, invalid};
  if (s.Dk == 64)
    return s.Dv == 64 ? launch_rec<64, 64, 4, true, 1, true, true>(a, s, stream)
                      : launch_rec<64, 64, 4, true, 2, true, true>(a, s, stream);
  return s.Dv == 64 ? launch_rec<128, 64, 4, true, 1, true, true>(a, s, stream)
                    : launch_rec<128, 64, 4, true, 2, true, true>(a, s, stream);
}

bool delta_recurrent_supported(const DeltaShape &s) {
  return (s.Dk == 64 || s.Dk == 128) && s.Dv % 16 == 0 && s.Hk >= 1 &&
         s.Hv % s.Hk == 0 && s.T >= 1;
}

hipError_t launch_delta_recurrent(const float *q, const float *k,
                                  const uint16_t *v, const float *beta,
                                  const float *decay, float *state,
                                  uint16_t *out, const DeltaShape &s,
                                  hipStream_t stream) {
  return launch_rec_any<false>({q, k, v, beta, decay, state, out, 0.0f, 1.0f}, s, stream);
}

hipError_t launch_delta_recurrent_qk16(const uint16_t *q, const uint16_t *k,
                                       const uint16_t *v, const float *beta,
                                       const float *decay, float *state, uint16_t *out,
                                       float eps, float qscale, const DeltaShape &s,
                                       hipStream_t stream) {
  return launch_rec_any<true>({q, k, v, beta, decay, state, out, eps, qscale}, s, stream);
}

} // namespace llmi
