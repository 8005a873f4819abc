// Gated delta rule, chunk-wise (WY) prefill. Not yet enabled: the C ABI
// routes T > 1 to the register-resident recurrent kernel until this path
// passes its parity tests.
#include "hip_common.hpp"
#include "kernels.hpp"

namespace llmi {

bool delta_chunked_supported(const DeltaShape &) { return false; }

size_t delta_chunked_workspace_bytes(const DeltaShape &) { return 0; }

hipError_t launch_delta_chunked(const float *, const float *, const uint16_t *,
                                const float *, const float *, float *,
                                uint16_t *, void *, const DeltaShape &,
                                hipStream_t) {
  return hipErrorNotSupported;
}

} // namespace llmi

#include "capi_internal.hpp"

namespace llmi {
unsigned delta_chunked_dispatches() { return 1; }
const char *delta_chunked_kernel_name(unsigned) { return "deltaChunkedWy"; }
} // namespace llmi
