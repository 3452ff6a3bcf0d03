// Bandwidth probe: a streaming read of a device buffer with the loads the decode kernel uses
// (16-byte non-temporal vector loads), so that a benchmark can state the read bandwidth the box
// it runs on delivers next to the decode kernel's own. Not part of the attention path.
#include "pa_common.h"

namespace pa {

// Grid-stride read of n16 16-byte vectors, eight independent loads in flight per lane. Each lane
// folds what it read into one word and stores it only if that word equals `never`, a value the
// host picks so that the store does not happen for a buffer of zeros: the loads cannot be
// dropped, and the probe writes (practically) nothing.
__global__ __launch_bounds__(512) void hbm_read_probe_kernel(const u32x4* __restrict__ src, int64_t n16,
                                                             uint32_t never, uint32_t* __restrict__ sink) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint32_t acc = 0;
  for (; i + 7 * stride < n16; i += 8 * stride) {
    u32x4 v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = __builtin_nontemporal_load(src + i + k * stride);
#pragma unroll
    for (int k = 0; k < 8; ++k) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
  }
  for (; i < n16; i += stride) {
    const u32x4 v = __builtin_nontemporal_load(src + i);
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (acc == never) sink[blockIdx.x] = acc;
}

}  // namespace pa

extern "C" int pa_hbm_read_probe(const void* src, size_t bytes, uint32_t* sink, int32_t workgroups, void* stream) {
  pa_host::clear_error();
  PA_CHECK_ARG(src != nullptr && sink != nullptr, "null src or sink");
  PA_CHECK_ARG(bytes % 16 == 0, "bytes (%zu) must be a multiple of 16", bytes);
  PA_CHECK_ARG(workgroups > 0, "workgroups must be > 0");
  if (bytes == 0) return PA_OK;
  pa::hbm_read_probe_kernel<<<dim3((unsigned)workgroups), dim3(512), 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const pa::u32x4*>(src), (int64_t)(bytes / 16), 0xA5C3E1F7u, sink);
  PA_CHECK_LAUNCH("hbm read probe");
  return PA_OK;
}
