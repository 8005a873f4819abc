// Shared device helpers for the gfx950 kernels of the attention hot path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace llmi {

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));
typedef uint32_t uint4_t __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;

// Host-side check for the 16-byte vector paths.
inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// LDS barrier: this wave's LDS accesses complete, then the workgroup
// barrier. Unlike __syncthreads it waits for no outstanding global load or
// store, so loads issued before it stay in flight and stores keep draining
// behind the next phase. For barriers that order LDS traffic only: a wave
// reading global memory that another wave of the workgroup wrote before the
// barrier needs __syncthreads (or its own waits).
__device__ __forceinline__ void lds_sync() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// DPP lane permutations on one 16-lane row (gfx9 encodings).
enum : int {
  kDppXor1 = 0xB1,        // quad_perm [1,0,3,2]
  kDppXor2 = 0x4E,        // quad_perm [2,3,0,1]
  kDppRowHalfMirror = 0x141,
  kDppRowMirror = 0x140,
};

template <int Ctrl> __device__ __forceinline__ float dpp(float x) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(x), Ctrl, 0xF, 0xF, false));
}

// Sum over aligned groups of N lanes (N in {1,2,4,8,16}); every lane of a
// group receives the group's total. After xor1/xor2 each quad holds its sum;
// the half-row mirror pairs quad q with quad 1-q inside each 8-lane half, the
// row mirror pairs the two halves of a 16-lane row.
template <int N> __device__ __forceinline__ float group_sum(float x) {
  if constexpr (N >= 2)
    x += dpp<kDppXor1>(x);
  if constexpr (N >= 4)
    x += dpp<kDppXor2>(x);
  if constexpr (N >= 8)
    x += dpp<kDppRowHalfMirror>(x);
  if constexpr (N >= 16)
    x += dpp<kDppRowMirror>(x);
  return x;
}

// DPP rotate right by N lanes inside each 16-lane row (row_ror:N, 1..15).
template <int N> __device__ __forceinline__ float row_ror(float x) {
  static_assert(N >= 1 && N <= 15, "row_ror takes 1..15");
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x120 + N, 0xF, 0xF, false));
}

// gfx950 row-pair exchange. With both operands equal to x, the two results
// hold x of the even and of the odd 16-lane row of each row pair (stride
// 16), or of the low and the high 32 lanes (stride 32), in every lane: a
// symmetric pair, so a combine of the two is identical in both partners.
struct LanePair {
  float a, b;
};
__device__ __forceinline__ LanePair pair16(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x),
                                            false, false);
  return {__uint_as_float(r[0]), __uint_as_float(r[1])};
}
__device__ __forceinline__ LanePair pair32(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                            false, false);
  return {__uint_as_float(r[0]), __uint_as_float(r[1])};
}

__device__ __forceinline__ float fast_exp2(float x) {
  return __builtin_amdgcn_exp2f(x);
}

// fp32 dot of 8 fp16 pairs, accumulated in fp32 (v_dot2_f32_f16).
__device__ __forceinline__ float dot8(half8_t a, half8_t b, float acc) {
  acc = __builtin_amdgcn_fdot2(half2_t{a[0], a[1]}, half2_t{b[0], b[1]}, acc, false);
  acc = __builtin_amdgcn_fdot2(half2_t{a[2], a[3]}, half2_t{b[2], b[3]}, acc, false);
  acc = __builtin_amdgcn_fdot2(half2_t{a[4], a[5]}, half2_t{b[4], b[5]}, acc, false);
  acc = __builtin_amdgcn_fdot2(half2_t{a[6], a[7]}, half2_t{b[6], b[7]}, acc, false);
  return acc;
}

// v_mfma_f32_32x32x16_f16. Operand layouts (lane l, r = l % 32, h = l / 32):
//   A (32 x 16): lane holds A[r][8h .. 8h+7]
//   B (16 x 32): lane holds B[8h .. 8h+7][r]
//   C (32 x 32): lane register v holds C[8(v/4) + 4h + v%4][r]
__device__ __forceinline__ float16_t mfma32x32x16(half8_t a, half8_t b, float16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Row of the C layout that register v of lane-half h holds.
__device__ __forceinline__ int mfma_c_row(int v, int h) { return 8 * (v / 4) + 4 * h + (v % 4); }

// x = hi + lo * 2^-11 with hi = fp16(x), lo = fp16((x - hi) * 2^11): 22
// significant bits. The remainder is stored scaled by 2^11 so that it stays
// a normal fp16 for |x| >= 2^-3 (unscaled it would be subnormal there);
// fp16 subnormals that remain (|x| < 2^-14) are kept by the conversions and
// by v_mfma_f32_*_f16 on gfx950, which does not flush fp16 inputs.
constexpr float kSplitScale = 2048.0f;
constexpr float kSplitUnscale = 1.0f / 2048.0f;
// The remainder as one fused multiply-add on the scaled values, hi 2^11
// subtracted from x 2^11: both are exact and so is their difference (hi is
// x rounded to fp16), so this is (x - hi) 2^11 rounded once to fp16, the
// same bits as the subtraction followed by the scaling, in fewer
// instructions (the backend takes the fp16 hi as a mixed-precision operand).
__device__ __forceinline__ void split_f16(float x, half_t &hi, half_t &lo) {
  hi = (half_t)x;
  lo = (half_t)fmaf((float)hi, -kSplitScale, x * kSplitScale);
}

__device__ __forceinline__ half8_t load8(const half_t *p) {
  return *reinterpret_cast<const half8_t *>(p);
}

// 16-byte load marked non-temporal: for data read once (streamed K/V).
__device__ __forceinline__ half8_t load8_stream(const half_t *p) {
  return __builtin_nontemporal_load(reinterpret_cast<const half8_t *>(p));
}

} // namespace llmi
