// storeLinear (Reference.metal:14-47), shared by the W8A8 and fp16
// projections: the fp32 projection rounded to fp16, then the consumer's
// fused epilogue. Callers compile with -ffp-contract=off.
#pragma once

#include "exact_fp.hpp"
#include "rope_gate.hpp"

#include "llminfer_hip.h"

namespace llmi {

// The SwiGLU epilogue's value: SiLU of the rounded projection times the
// fp16 multiplier.
__device__ __forceinline__ uint16_t silu_mul16(float projected, uint16_t multiplier) {
  return f2h(mul32(h2f(silu16(projected)), h2f(multiplier)));
}

__device__ __forceinline__ void store_linear(void *out, const void *aux, const float *bias,
                                             size_t i, unsigned col, unsigned epilogue,
                                             unsigned block, float acc) {
  const float projected = round16(acc);
  uint16_t *o16 = static_cast<uint16_t *>(out);
  float *o32 = static_cast<float *>(out);
  switch (epilogue) {
  case LLMI_LINEAR_SILU:
    o16[i] = silu16(projected);
    return;
  case LLMI_LINEAR_SILU_MUL:
    o16[i] = silu_mul16(projected, static_cast<const uint16_t *>(aux)[i]);
    return;
  case LLMI_LINEAR_SIGMOID_COLUMNS:
    o16[i] = f2h((col / block) % 2 ? logistic16(projected) : projected);
    return;
  case LLMI_LINEAR_SILU_F32:
    o32[i] = mul32(projected, logistic_exact(projected));
    return;
  case LLMI_LINEAR_DELTA_BETA:
    o32[i] = logistic16(projected);
    return;
  case LLMI_LINEAR_DELTA_DECAY: {
    const float *a_log = static_cast<const float *>(aux);
    o32[i] = exp_cr(mul32(-exp_cr(a_log[col]), stable_softplus(__fadd_rn(projected, bias[col]))));
    return;
  }
  default:
    o16[i] = f2h(projected);
    return;
  }
}

} // namespace llmi
