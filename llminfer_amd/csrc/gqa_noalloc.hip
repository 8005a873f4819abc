// KvAppend + CausalGqa for callers that cannot allocate device memory (code
// under HIP graph capture, tight serving loops, harnesses that forbid
// hipMalloc). Same kernels and results as llmi_hip_kv_append_causal_gqa;
// the split-K decode's partials go to a fixed device array of this file
// instead of a caller workspace. Declaration: include/llminfer_hip.h.
//
// The array is resident on every device the library runs on until the
// process ends. Its address is looked up once per device, with that device
// current, on the first call there; from then on only that address is used.
// Every call on a device shares that device's array: calls that overlap on
// one device race. Nothing in it has to start at zero -- a decode writes
// every partial it reads back within the same call.
#include "llminfer_hip.h"
#include "capi_internal.hpp"
#include "kernels.hpp"

#include <hip/hip_runtime.h>
#include <mutex>

static __device__ __align__(256) unsigned char scratch[LLMI_HIP_NOALLOC_SCRATCH_BYTES];

namespace llmi {
namespace {

constexpr int kMaxDevices = 64;

struct ScratchSlot {
  std::once_flag once;
  void *ptr = nullptr;
  hipError_t err = hipSuccess;
};

ScratchSlot g_slots[kMaxDevices];

// The device address of `scratch` on the current device.
int scratch_address(void **out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(LLMI_HIP_NO_DEVICE, "noalloc decode: no usable current HIP device");
  ScratchSlot &slot = g_slots[dev];
  std::call_once(slot.once, [&slot] {
    slot.err = hipGetSymbolAddress(&slot.ptr, HIP_SYMBOL(scratch));
  });
  if (slot.err != hipSuccess || !slot.ptr)
    return fail(LLMI_HIP_NO_DEVICE, "noalloc decode: cannot find the scratch array on device %d: %s",
                dev, hipGetErrorString(slot.err));
  *out = slot.ptr;
  return LLMI_HIP_OK;
}

} // namespace
} // namespace llmi

using namespace llmi;

extern "C" int llmi_hip_kv_append_causal_gqa_noalloc(const uint16_t *q, const uint16_t *k_new,
                                                     const uint16_t *v_new, uint16_t *k_cache,
                                                     uint16_t *v_cache, uint16_t *out,
                                                     GqaParams p, void *stream) {
  if (int st = check_gqa(p))
    return st;
  if (!q || !k_new || !v_new || !k_cache || !v_cache || !out)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "KvAppend+CausalGqa: null buffer");
  size_t need = 0;
  if (select_gqa(p) == GqaKernel::Decode)
    need = decode_workspace_bytes({p.tokens, p.queryHeads, p.kvHeads, p.headDim, p.past});
  if (need > LLMI_HIP_NOALLOC_SCRATCH_BYTES)
    return fail(LLMI_HIP_WORKSPACE,
                "noalloc decode: the split partials need %zu bytes, more than the %u-byte "
                "static scratch",
                need, (unsigned)LLMI_HIP_NOALLOC_SCRATCH_BYTES);
  void *ws = nullptr;
  if (need)
    if (int st = scratch_address(&ws))
      return st;
  return run_gqa(q, k_new, v_new, k_cache, v_cache, out, p, ws, need, stream);
}
