// Greedy next-token selection on the device: the argmax over the vocabulary of one logits row
// per request, written as int64 token ids.
//
// Replaces the per-request `int(torch.argmax(logits[b, row, :]).item())` of the reference's
// continuous-batching executors (src/serving/continuous_generate.py:145,238) inside the captured
// decode/prefill step, so a step hands back B token ids instead of [B, T, vocab] logits.
//
// Semantics are torch.argmax's: the first index of the maximum; NaN compares above every number
// (the first NaN wins); -0.0 and +0.0 are equal. One workgroup of 1024 threads per request (a step
// has only a few requests, so each row is spread over as many lanes as a workgroup holds and each
// lane's loads are all in flight at once): each thread scans a strided slice of the row in
// increasing index order (so a later equal value never replaces an earlier one), then the
// (value, index) pairs are reduced over the wavefront with shuffles and over the workgroup's
// wavefronts in LDS, keeping the lower index on ties.
#include "pa_common.h"

namespace pa {

constexpr int kSelectThreads = 1024;
constexpr int kSelectLoads = 8;  // loads each thread has in flight per pass (one pass up to 8192 values)

struct Best {
  float v;
  int i;
};

// True when (va, ia) should be preferred over (vb, ib) by torch.argmax's rules.
__device__ __forceinline__ bool better(float va, int ia, float vb, int ib) {
  const bool na = va != va, nb = vb != vb;
  if (na != nb) return na;
  if (!na && va != vb) return va > vb;
  return ia < ib;
}

template <typename T>
__global__ __launch_bounds__(kSelectThreads) void argmax_rows_kernel(const T* __restrict__ logits, int64_t row_stride,
                                                                     int32_t rows_per_request,
                                                                     const int32_t* __restrict__ row_index,
                                                                     int32_t vocab, int64_t* __restrict__ tokens) {
  const int b = blockIdx.x;
  int r = row_index ? row_index[b] : 0;
  if (r < 0) r += rows_per_request;  // a negative row counts from the end, as in Python indexing
  r = r < 0 ? 0 : (r >= rows_per_request ? rows_per_request - 1 : r);
  const T* row = logits + ((int64_t)b * rows_per_request + r) * row_stride;

  float bv = -INFINITY;
  int bi = 0x7fffffff;
  // All of a pass's loads are issued before any compare; a thread's indices increase within and
  // across passes, so the first of equal values is kept.
  for (int base = threadIdx.x; base < vocab; base += kSelectThreads * kSelectLoads) {
    float x[kSelectLoads];
#pragma unroll
    for (int k = 0; k < kSelectLoads; ++k) {
      const int v = base + k * kSelectThreads;
      x[k] = v < vocab ? Elem<T>::load(row + v) : -INFINITY;
    }
#pragma unroll
    for (int k = 0; k < kSelectLoads; ++k) {
      const int v = base + k * kSelectThreads;
      if (v < vocab && better(x[k], v, bv, bi)) { bv = x[k]; bi = v; }
    }
  }

#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const float ov = __shfl_xor(bv, off);
    const int oi = __shfl_xor(bi, off);
    if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
  }
  __shared__ Best part[kSelectThreads / kWave];
  const int w = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) part[w] = Best{bv, bi};
  __syncthreads();
  if (threadIdx.x == 0) {
    Best best = part[0];
#pragma unroll
    for (int k = 1; k < kSelectThreads / kWave; ++k)
      if (better(part[k].v, part[k].i, best.v, best.i)) best = part[k];
    tokens[b] = best.i < vocab ? best.i : 0;
  }
}

}  // namespace pa

using namespace pa;

extern "C" int pa_argmax_rows(const void* logits, int64_t row_stride, int32_t batch, int32_t rows_per_request,
                              const int32_t* row_index, int32_t vocab, int dtype, int64_t* tokens, void* stream_) {
  pa_host::clear_error();
  PA_CHECK_ARG(batch >= 0 && rows_per_request > 0 && vocab > 0, "bad sizes: batch=%d rows_per_request=%d vocab=%d",
               batch, rows_per_request, vocab);
  PA_CHECK_ARG(dtype == PA_DTYPE_F32 || dtype == PA_DTYPE_BF16, "bad dtype %d", dtype);
  PA_CHECK_ARG(row_stride >= vocab, "row_stride %lld < vocab %d", (long long)row_stride, vocab);
  if (batch == 0) return PA_OK;
  PA_CHECK_ARG(logits != nullptr && tokens != nullptr, "null logits/tokens");
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  const dim3 grid((unsigned)batch), block(kSelectThreads);
  if (dtype == PA_DTYPE_F32)
    argmax_rows_kernel<float><<<grid, block, 0, stream>>>(static_cast<const float*>(logits), row_stride,
                                                          rows_per_request, row_index, vocab, tokens);
  else
    argmax_rows_kernel<uint16_t><<<grid, block, 0, stream>>>(static_cast<const uint16_t*>(logits), row_stride,
                                                             rows_per_request, row_index, vocab, tokens);
  PA_CHECK_LAUNCH("argmax kernel");
  return PA_OK;
}
