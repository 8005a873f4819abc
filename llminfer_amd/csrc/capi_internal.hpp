// Internal helpers shared by the C ABI (capi.cpp) and the host-side graph /
// session code (graph.cpp, session.cpp).
#pragma once

#include "llminfer_hip.h"

#include <hip/hip_runtime.h>

namespace llmi {

// Record a formatted message for llmi_hip_last_error() and return `status`.
int fail(int status, const char *fmt, ...)
    __attribute__((format(printf, 2, 3)));
// LLMI_HIP_OK, or LLMI_HIP_LAUNCH_FAILED with the HIP error recorded.
int launched(hipError_t err, const char *what);

int check_gqa(const GqaParams &p);
int check_delta(const GraphDeltaParams &p);

enum class GqaKernel { Decode, Prefill, Generic, None };
enum class DeltaKernel { Chunked, Recurrent, Generic };
GqaKernel select_gqa(const GqaParams &p);
DeltaKernel select_delta(const GraphDeltaParams &p);

// CausalGqa with an optional fused KvAppend (k_new and v_new non-null):
// validation, workspace check and the launches (capi.cpp).
int run_gqa(const uint16_t *q, const uint16_t *k_new, const uint16_t *v_new,
            uint16_t *k_cache, uint16_t *v_cache, uint16_t *out,
            const GqaParams &p, void *workspace, size_t workspace_bytes,
            void *stream);

// Launch count and names of the chunked DeltaNet path (delta_chunked.hip).
unsigned delta_chunked_dispatches();
const char *delta_chunked_kernel_name(unsigned index);

} // namespace llmi
