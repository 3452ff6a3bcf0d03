// Bandwidth probes: reads of a device buffer with the loads the decode kernel uses (16-byte
// non-temporal vector loads), so that a benchmark can state the read bandwidth the box it runs on
// delivers next to the decode kernel's own. Not part of the attention path.
//   pa_hbm_read_probe        a streaming (sequential) read, as the HBM delivers at its best;
//   pa_hbm_chunk_read_probe  4 KB chunks read in a given order, as a paged KV pool is read (one
//                            (block, head) slab of 16 tokens x 128 values x 2 bytes per chunk).
// Which grid, workgroup size and loads in flight deliver the most differs by a few percent from
// box to box, so both take them as arguments and the caller keeps the best of a sweep.
#include "pa_common.h"

namespace pa {

// Each lane folds what it read into one word and stores it only if that word equals `never`, a
// value the host picks so that the store does not happen for a buffer of zeros: the loads cannot
// be dropped, and the probes write (practically) nothing.
constexpr uint32_t kProbeNever = 0xA5C3E1F7u;

// Grid-stride read of n16 16-byte vectors, DEPTH independent loads in flight per lane.
template <int DEPTH>
__global__ __launch_bounds__(1024) void hbm_read_probe_kernel(const u32x4* __restrict__ src, int64_t n16,
                                                              uint32_t never, uint32_t* __restrict__ sink) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint32_t acc = 0;
  for (; i + (DEPTH - 1) * stride < n16; i += DEPTH * stride) {
    u32x4 v[DEPTH];
#pragma unroll
    for (int k = 0; k < DEPTH; ++k) v[k] = __builtin_nontemporal_load(src + i + k * stride);
#pragma unroll
    for (int k = 0; k < DEPTH; ++k) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
  }
  for (; i < n16; i += stride) {
    const u32x4 v = __builtin_nontemporal_load(src + i);
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (acc == never) sink[blockIdx.x] = acc;
}

// 4 KB chunks in the order `order` gives: workgroup x takes positions x, x + grid, ... of the
// order, DEPTH chunks per round, its 256 lanes reading one 16-byte vector of each chunk. Chunk ids
// outside [0, chunks) are skipped.
constexpr int kProbeChunkVecs = 256;  // 16-byte vectors per 4 KB chunk
template <int DEPTH>
__global__ __launch_bounds__(kProbeChunkVecs) void hbm_chunk_read_probe_kernel(const u32x4* __restrict__ src,
                                                                               const int32_t* __restrict__ order,
                                                                               int32_t chunks, uint32_t never,
                                                                               uint32_t* __restrict__ sink) {
  const int64_t g = gridDim.x;
  uint32_t acc = 0;
  int64_t j = blockIdx.x;
  for (; j + (DEPTH - 1) * g < chunks; j += DEPTH * g) {
    int c[DEPTH];
#pragma unroll
    for (int k = 0; k < DEPTH; ++k) c[k] = order[j + k * g];
    u32x4 v[DEPTH];
#pragma unroll
    for (int k = 0; k < DEPTH; ++k) {
      const int ck = (uint32_t)c[k] < (uint32_t)chunks ? c[k] : 0;
      v[k] = __builtin_nontemporal_load(src + (int64_t)ck * kProbeChunkVecs + threadIdx.x);
    }
#pragma unroll
    for (int k = 0; k < DEPTH; ++k)
      if ((uint32_t)c[k] < (uint32_t)chunks) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
  }
  for (; j < chunks; j += g) {
    const int c = order[j];
    if ((uint32_t)c >= (uint32_t)chunks) continue;
    const u32x4 v = __builtin_nontemporal_load(src + (int64_t)c * kProbeChunkVecs + threadIdx.x);
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (acc == never) sink[blockIdx.x] = acc;
}

}  // namespace pa

extern "C" int pa_hbm_read_probe(const void* src, size_t bytes, uint32_t* sink, int32_t workgroups,
                                 int32_t threads, int32_t depth, void* stream) {
  pa_host::clear_error();
  PA_CHECK_ARG(src != nullptr && sink != nullptr, "null src or sink");
  PA_CHECK_ARG(bytes % 16 == 0, "bytes (%zu) must be a multiple of 16", bytes);
  PA_CHECK_ARG(workgroups > 0, "workgroups must be > 0");
  PA_CHECK_ARG(threads == 256 || threads == 512 || threads == 1024, "threads must be 256, 512 or 1024, got %d",
               threads);
  PA_CHECK_ARG(depth == 1 || depth == 4 || depth == 8, "depth must be 1, 4 or 8, got %d", depth);
  if (bytes == 0) return PA_OK;
  const dim3 grid((unsigned)workgroups), block((unsigned)threads);
  const auto* s = static_cast<const pa::u32x4*>(src);
  const int64_t n16 = (int64_t)(bytes / 16);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (depth == 1) pa::hbm_read_probe_kernel<1><<<grid, block, 0, st>>>(s, n16, pa::kProbeNever, sink);
  else if (depth == 4) pa::hbm_read_probe_kernel<4><<<grid, block, 0, st>>>(s, n16, pa::kProbeNever, sink);
  else pa::hbm_read_probe_kernel<8><<<grid, block, 0, st>>>(s, n16, pa::kProbeNever, sink);
  PA_CHECK_LAUNCH("hbm read probe");
  return PA_OK;
}

extern "C" int pa_hbm_chunk_read_probe(const void* src, const int32_t* order, int32_t chunks, uint32_t* sink,
                                       int32_t workgroups, int32_t depth, void* stream) {
  pa_host::clear_error();
  PA_CHECK_ARG(src != nullptr && order != nullptr && sink != nullptr, "null src, order or sink");
  PA_CHECK_ARG(chunks >= 0, "chunks must be >= 0");
  PA_CHECK_ARG(workgroups > 0, "workgroups must be > 0");
  PA_CHECK_ARG(depth == 1 || depth == 2 || depth == 4, "depth must be 1, 2 or 4, got %d", depth);
  if (chunks == 0) return PA_OK;
  const dim3 grid((unsigned)workgroups), block(pa::kProbeChunkVecs);
  const auto* s = static_cast<const pa::u32x4*>(src);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (depth == 1) pa::hbm_chunk_read_probe_kernel<1><<<grid, block, 0, st>>>(s, order, chunks, pa::kProbeNever, sink);
  else if (depth == 2) pa::hbm_chunk_read_probe_kernel<2><<<grid, block, 0, st>>>(s, order, chunks, pa::kProbeNever, sink);
  else pa::hbm_chunk_read_probe_kernel<4><<<grid, block, 0, st>>>(s, order, chunks, pa::kProbeNever, sink);
  PA_CHECK_LAUNCH("hbm chunk read probe");
  return PA_OK;
}
