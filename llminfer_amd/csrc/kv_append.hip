// KvAppend: copy the step's new K and V rows into the session caches.
// Same effect as the reference's cacheAppend (Reference.metal:295-301), but
// one launch moves both halves with 128-bit accesses where alignment allows.
#include "hip_common.hpp"
#include "kernels.hpp"

namespace llmi {
namespace {

// 16-byte path: count, offset and both base pointers are multiples of 8
// halves. Each thread moves 16 bytes; blockIdx.y selects K (0) or V (1).
__global__ __launch_bounds__(256) void kv_append_vec(
    const uint4_t *__restrict__ ks, const uint4_t *__restrict__ vs,
    uint4_t *__restrict__ kc, uint4_t *__restrict__ vc, unsigned vectors) {
  unsigned i = blockIdx.x * 256u + threadIdx.x;
  if (i >= vectors)
    return;
  if (blockIdx.y == 0)
    kc[i] = ks[i];
  else
    vc[i] = vs[i];
}

__global__ __launch_bounds__(256) void kv_append_scalar(
    const uint16_t *__restrict__ ks, const uint16_t *__restrict__ vs,
    uint16_t *__restrict__ kc, uint16_t *__restrict__ vc, unsigned count) {
  unsigned i = blockIdx.x * 256u + threadIdx.x;
  if (i >= count)
    return;
  if (blockIdx.y == 0)
    kc[i] = ks[i];
  else
    vc[i] = vs[i];
}

hipError_t launch(const uint16_t *ksrc, const uint16_t *vsrc, uint16_t *kcache,
                  uint16_t *vcache, unsigned count, unsigned offset,
                  unsigned halves, hipStream_t stream) {
  if (count == 0)
    return hipSuccess;
  uint16_t *kdst = kcache + offset;
  uint16_t *vdst = vcache ? vcache + offset : nullptr;
  bool vec = count % 8 == 0 && aligned16(ksrc) && aligned16(kdst) &&
             (halves == 1 || (aligned16(vsrc) && aligned16(vdst)));
  if (vec) {
    unsigned vectors = count / 8;
    dim3 grid((vectors + 255) / 256, halves);
    hipLaunchKernelGGL(kv_append_vec, grid, dim3(256), 0, stream,
                       reinterpret_cast<const uint4_t *>(ksrc),
                       reinterpret_cast<const uint4_t *>(vsrc),
                       reinterpret_cast<uint4_t *>(kdst),
                       reinterpret_cast<uint4_t *>(vdst), vectors);
  } else {
    dim3 grid((count + 255) / 256, halves);
    hipLaunchKernelGGL(kv_append_scalar, grid, dim3(256), 0, stream, ksrc,
                       vsrc, kdst, vdst, count);
  }
  return hipGetLastError();
}

} // namespace

hipError_t launch_cache_append(const uint16_t *src, uint16_t *cache,
                               unsigned count, unsigned offset,
                               hipStream_t stream) {
  return launch(src, nullptr, cache, nullptr, count, offset, 1, stream);
}

hipError_t launch_kv_append(const uint16_t *ksrc, const uint16_t *vsrc,
                            uint16_t *kcache, uint16_t *vcache, unsigned count,
                            unsigned offset, hipStream_t stream) {
  return launch(ksrc, vsrc, kcache, vcache, count, offset, 2, stream);
}

} // namespace llmi
