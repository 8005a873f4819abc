// Session: device state ownership and the step contract of the reference's
// MetalSession / MetalExecutor, for one hybrid layer pair (a DeltaNet layer
// and a GQA layer). Declarations: include/llminfer_hip.h.
//
//  * open   -- MetalSession::open + MetalExecutor::initialize
//              (lib/Backend/Metal/MetalExecutor.mm:230-253, 56-94): one device
//              buffer per state slot -- K and V caches [capacity][Hkv][d]
//              fp16 and the recurrent state [Hv][dk][dv] fp32
//              (lib/Models/Qwen35/Qwen35ModelBuilder.cpp:134-139, 171-174) --
//              zeroed before first use (reset).
//  * step   -- MetalSession::step (MetalExecutor.mm:255-292): every check
//              happens before the first launch; `past` advances only when the
//              whole step succeeded; a failure after a launch leaves the
//              session invalid until reset (MetalExecutor.mm:283-290).
//  * reset  -- MetalSession::reset / MetalExecutor::reset
//              (MetalExecutor.mm:115-118, 294-298): zero every state buffer,
//              past = 0, clear the invalid flag.
#include "llminfer_hip.h"
#include "capi_internal.hpp"
#include "kernels.hpp"

#include <hip/hip_runtime.h>
#include <new>
#include <string.h>

struct llmi_hip_session {
  llmi_hip_session_config cfg;
  hipStream_t stream;
  uint16_t *kcache = nullptr, *vcache = nullptr;
  float *state = nullptr;
  void *ws = nullptr;
  size_t wsBytes = 0;
  size_t cacheBytes = 0, stateBytes = 0;
  unsigned past = 0;
  bool invalid = false;
};

namespace llmi {
namespace {

bool mul_fits(uint64_t a, uint64_t b, uint64_t limit, uint64_t *out) {
  if (a && b > limit / a)
    return false;
  *out = a * b;
  return *out <= limit;
}

int check_config(const llmi_hip_session_config &c) {
  if (!c.capacity)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "session: invalid capacity");
  GqaParams g{1, c.queryHeads, c.kvHeads, c.headDim, c.capacity - 1};
  if (int st = check_gqa(g))
    return st;
  GraphDeltaParams d{1, c.keyHeads, c.keyDim, c.valueHeads, c.valueDim};
  if (int st = check_delta(d))
    return st;
  if (select_gqa(g) == GqaKernel::None)
    return fail(LLMI_HIP_UNSUPPORTED, "session: head_dim %u is not supported",
                c.headDim);
  return LLMI_HIP_OK;
}

int check_device() {
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count == 0)
    return fail(LLMI_HIP_NO_DEVICE, "session: no HIP device");
  int dev = 0;
  hipDeviceProp_t prop;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipGetDeviceProperties(&prop, dev) != hipSuccess)
    return fail(LLMI_HIP_NO_DEVICE, "session: cannot query the HIP device");
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(LLMI_HIP_NO_DEVICE,
                "session: device %s is not gfx950 (the kernels are built for "
                "gfx950 only)",
                prop.gcnArchName);
  return LLMI_HIP_OK;
}

void release(llmi_hip_session *s) {
  if (s->kcache)
    (void)hipFree(s->kcache);
  if (s->vcache)
    (void)hipFree(s->vcache);
  if (s->state)
    (void)hipFree(s->state);
  if (s->ws)
    (void)hipFree(s->ws);
  s->kcache = s->vcache = nullptr;
  s->state = nullptr;
  s->ws = nullptr;
}

// Zero every state buffer and wait, so the host sees a clean session.
hipError_t zero_state(llmi_hip_session *s) {
  hipError_t e = hipMemsetAsync(s->kcache, 0, s->cacheBytes, s->stream);
  if (e == hipSuccess)
    e = hipMemsetAsync(s->vcache, 0, s->cacheBytes, s->stream);
  if (e == hipSuccess)
    e = hipMemsetAsync(s->state, 0, s->stateBytes, s->stream);
  if (e == hipSuccess)
    e = hipStreamSynchronize(s->stream);
  return e;
}

// Grow the workspace to `need` bytes before any launch of a step. The
// previous step ended with a stream synchronisation, so nothing in flight
// uses the old allocation.
int ensure_workspace(llmi_hip_session *s, size_t need) {
  if (need <= s->wsBytes)
    return LLMI_HIP_OK;
  void *ws = nullptr;
  if (hipMalloc(&ws, need) != hipSuccess)
    return fail(LLMI_HIP_WORKSPACE, "session: cannot allocate a %zu-byte workspace",
                need);
  if (s->ws)
    (void)hipFree(s->ws);
  s->ws = ws;
  s->wsBytes = need;
  return LLMI_HIP_OK;
}

// Plan records carry no projection epilogue on this path: epilogue "" and
// fused_op_index 0, the reference's defaults (MetalExecutionPlan.h:31-32).
void record(llmi_hip_dispatch *records, size_t cap, size_t &n, size_t op,
            const char *kernel) {
  if (records && n < cap)
    records[n] = llmi_hip_dispatch{op, kernel, "", 0};
  ++n;
}

// Everything a step checks before it allocates or launches: the config
// (every shape valid up to the full capacity), the step shape
// (Graph.cpp:382-387) and the three op contracts at this step.
int check_step(const llmi_hip_session_config &c, unsigned past, unsigned tokens) {
  if (int st = check_config(c))
    return st;
  if (!tokens || past > c.capacity || tokens > c.capacity - past)
    return fail(LLMI_HIP_INVALID_ARGUMENT,
                "token chunk is empty or exceeds session capacity");
  GraphDeltaParams dp{tokens, c.keyHeads, c.keyDim, c.valueHeads, c.valueDim};
  GqaParams gp{tokens, c.queryHeads, c.kvHeads, c.headDim, past};
  if (int st = check_delta(dp))
    return st;
  if (int st = check_gqa(gp))
    return st;
  if (select_gqa(gp) == GqaKernel::None)
    return fail(LLMI_HIP_UNSUPPORTED, "session step: no attention kernel for this shape");
  return LLMI_HIP_OK;
}

} // namespace
} // namespace llmi

using namespace llmi;

extern "C" {

int llmi_hip_session_open(const llmi_hip_session_config *config, void *stream,
                          llmi_hip_session **out) {
  if (!config || !out)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "session: null argument");
  *out = nullptr;
  if (int st = check_config(*config))
    return st;
  if (int st = check_device())
    return st;
  const llmi_hip_session_config &c = *config;
  uint64_t rows, cacheElems, headElems, stateElems;
  if (!mul_fits(c.capacity, c.kvHeads, UINT32_MAX, &rows) ||
      !mul_fits(rows, c.headDim, UINT32_MAX, &cacheElems) ||
      !mul_fits(c.keyDim, c.valueDim, UINT32_MAX, &headElems) ||
      !mul_fits(headElems, c.valueHeads, UINT32_MAX, &stateElems))
    return fail(LLMI_HIP_INVALID_ARGUMENT,
                "session: state exceeds the 32-bit index range");
  llmi_hip_session *s = new (std::nothrow) llmi_hip_session;
  if (!s)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "session: out of host memory");
  s->cfg = c;
  s->stream = static_cast<hipStream_t>(stream);
  s->cacheBytes = cacheElems * sizeof(uint16_t);
  s->stateBytes = stateElems * sizeof(float);
  if (hipMalloc(reinterpret_cast<void **>(&s->kcache), s->cacheBytes) != hipSuccess ||
      hipMalloc(reinterpret_cast<void **>(&s->vcache), s->cacheBytes) != hipSuccess ||
      hipMalloc(reinterpret_cast<void **>(&s->state), s->stateBytes) != hipSuccess) {
    release(s);
    delete s;
    return fail(LLMI_HIP_INVALID_ARGUMENT,
                "session: cannot allocate %zu bytes of device state",
                2 * (size_t)(cacheElems * 2) + (size_t)stateElems * 4);
  }
  if (hipError_t e = zero_state(s)) {
    release(s);
    delete s;
    return fail(LLMI_HIP_LAUNCH_FAILED, "session: cannot clear state: %s",
                hipGetErrorString(e));
  }
  *out = s;
  return LLMI_HIP_OK;
}

void llmi_hip_session_close(llmi_hip_session *s) {
  if (!s)
    return;
  (void)hipStreamSynchronize(s->stream);
  release(s);
  delete s;
}

void llmi_hip_session_reset(llmi_hip_session *s) {
  if (!s)
    return;
  if (zero_state(s) != hipSuccess) {
    s->invalid = true; // the state could not be cleared
    return;
  }
  s->past = 0;
  s->invalid = false;
}

unsigned llmi_hip_session_past(const llmi_hip_session *s) { return s ? s->past : 0; }

int llmi_hip_session_restore(llmi_hip_session *s, unsigned past) {
  if (!s)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "session: null session");
  if (s->invalid)
    return fail(LLMI_HIP_INVALID_ARGUMENT,
                "session is invalid after a failed GPU step; reset it first");
  if (past > s->cfg.capacity)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "session restore: past %u exceeds capacity %u",
                past, s->cfg.capacity);
  s->past = past;
  return LLMI_HIP_OK;
}

int llmi_hip_session_check(const llmi_hip_session_config *config, unsigned past,
                           unsigned tokens) {
  if (!config)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "session: null config");
  return check_step(*config, past, tokens);
}

int llmi_hip_session_invalid(const llmi_hip_session *s) { return s ? s->invalid : 1; }

uint16_t *llmi_hip_session_key_cache(llmi_hip_session *s) {
  return s ? s->kcache : nullptr;
}

uint16_t *llmi_hip_session_value_cache(llmi_hip_session *s) {
  return s ? s->vcache : nullptr;
}

float *llmi_hip_session_recurrent_state(llmi_hip_session *s) {
  return s ? s->state : nullptr;
}

int llmi_hip_session_step(llmi_hip_session *s, unsigned tokens, const float *dq,
                          const float *dk, const uint16_t *dv,
                          const float *beta, const float *decay,
                          uint16_t *delta_out, const uint16_t *q,
                          const uint16_t *k, const uint16_t *v,
                          uint16_t *gqa_out, llmi_hip_dispatch *records,
                          size_t cap, size_t *count) {
  if (!s)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "session: null session");
  if (s->invalid)
    return fail(LLMI_HIP_INVALID_ARGUMENT,
                "session is invalid after a failed GPU step");
  if (int st = check_step(s->cfg, s->past, tokens))
    return st;
  if (!dq || !dk || !dv || !beta || !decay || !delta_out || !q || !k || !v ||
      !gqa_out)
    return fail(LLMI_HIP_INVALID_ARGUMENT, "session step: null buffer");
  const llmi_hip_session_config &c = s->cfg;
  GraphDeltaParams dp{tokens, c.keyHeads, c.keyDim, c.valueHeads, c.valueDim};
  GqaParams gp{tokens, c.queryHeads, c.kvHeads, c.headDim, s->past};
  size_t need = llmi_hip_gqa_workspace_bytes(gp);
  size_t needDelta = llmi_hip_delta_workspace_bytes(dp);
  if (needDelta > need)
    need = needDelta;
  if (int st = ensure_workspace(s, need))
    return st;

  // Plan records, in graph order: DeltaUpdate (op 0), KvAppend (op 1),
  // CausalGqa (op 2). KvAppend and CausalGqa run through the fused entry
  // point: one decode launch that also appends (recorded under op 1 and
  // again under op 2), or append then prefill.
  size_t n = 0;
  for (unsigned i = 0, m = llmi_hip_dispatch_count(LLMI_HIP_OP_DELTA_UPDATE, &dp); i < m; ++i)
    record(records, cap, n, 0, llmi_hip_kernel_name(LLMI_HIP_OP_DELTA_UPDATE, &dp, i));
  const unsigned pairLaunches =
      llmi_hip_dispatch_count(LLMI_HIP_OP_KV_APPEND_CAUSAL_GQA, &gp);
  if (select_gqa(gp) == GqaKernel::Decode) {
    const char *first = llmi_hip_kernel_name(LLMI_HIP_OP_KV_APPEND_CAUSAL_GQA, &gp, 0);
    record(records, cap, n, 1, first);
    record(records, cap, n, 2, first);
    for (unsigned i = 1; i < pairLaunches; ++i)
      record(records, cap, n, 2,
             llmi_hip_kernel_name(LLMI_HIP_OP_KV_APPEND_CAUSAL_GQA, &gp, i));
  } else {
    record(records, cap, n, 1,
           llmi_hip_kernel_name(LLMI_HIP_OP_KV_APPEND_CAUSAL_GQA, &gp, 0));
    record(records, cap, n, 2,
           llmi_hip_kernel_name(LLMI_HIP_OP_KV_APPEND_CAUSAL_GQA, &gp, 1));
  }
  if (count)
    *count = n;

  // From here on a failure leaves state possibly written: invalidate.
  int st = llmi_hip_delta_update(dq, dk, dv, beta, decay, s->state, delta_out, dp,
                                 s->ws, s->wsBytes, s->stream);
  if (st == LLMI_HIP_OK)
    st = llmi_hip_kv_append_causal_gqa(q, k, v, s->kcache, s->vcache, gqa_out, gp,
                                       s->ws, s->wsBytes, s->stream);
  if (st == LLMI_HIP_OK) {
    hipError_t e = hipStreamSynchronize(s->stream);
    if (e != hipSuccess)
      st = fail(LLMI_HIP_LAUNCH_FAILED, "session step: %s", hipGetErrorString(e));
  }
  if (st != LLMI_HIP_OK) {
    s->invalid = true;
    return st == LLMI_HIP_LAUNCH_FAILED ? st : LLMI_HIP_LAUNCH_FAILED;
  }
  s->past += tokens;
  return LLMI_HIP_OK;
}

} // extern "C"
