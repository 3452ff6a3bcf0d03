// Argument blocks shared by the attention kernels and their host launchers.
#pragma once

#include "pa_common.h"

namespace pa {

// Everything an attention launch reads; q/out strides are in elements, head_dim stride is 1.
struct AttnArgs {
  const void* q;
  int64_t q_sb, q_sh, q_st;
  void* out;
  int64_t o_sb, o_sh, o_st;
  const void* k_pool;
  const void* v_pool;
  int64_t num_blocks;
  const int32_t* page_table;
  int64_t pt_stride;
  int32_t max_pages;
  const int32_t* seq_lens;
  const int32_t* cur_lens;
  const int32_t* order;  // decode only: request processing order, may be null
  int32_t B, H, T, head_dim, block_size;
  float scale_log2;      // softmax scale * log2(e)
  int32_t num_splits;    // workgroups per work unit along the KV axis, >= 1
  int32_t split_blocks;  // KV blocks per split when num_splits > 1
  float* ws;             // partial (m, l, acc[head_dim]) records of the splits
  int32_t* counters;     // same-launch merge: arrival counters (zero between calls); decode per
                         // (request, head), balanced wide prefill per (request, head, tile)
  int32_t die_cus;       // balanced wide prefill: compute units per die
};

// Wave-wide partner exchange on gfx950 without an LDS round trip: v_permlane16_swap /
// v_permlane32_swap with both operands equal leave, in every lane, its own value in one result
// and the value of lane ^ 16 (resp. lane ^ 32) in the other, so a symmetric op over the two
// results reduces over the lane pair.
__device__ __forceinline__ float max_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Wide-tile prefill (128 query rows per workgroup, KV staged through LDS; bf16 or fp32 KV).
// Defined in pa_prefill_wide.hip.
bool prefill_wide_supported(int kv_dtype, int head_dim, int block_size);
int64_t prefill_wide_units(int32_t batch, int32_t num_heads, int32_t query_len);
int launch_prefill_wide(const AttnArgs& a, int io_dtype, int kv_dtype, hipStream_t stream);
// Balanced launch of the wide kernels (bf16 or fp32 KV, head_dim 128 or 64): its grid (0 when the
// policy declines or it does not apply) and the bytes of its split records at that grid and
// head_dim. launch_prefill_wide takes it when a.counters is set.
int64_t prefill_balanced_grid(int32_t batch, int32_t num_heads, int32_t query_len, int32_t head_dim,
                              int32_t max_pages, int kv_dtype);
size_t prefill_balanced_record_bytes(int64_t grid, int32_t head_dim);

// Split-step prefill (32 query rows per workgroup, 8 wavefronts splitting the KV steps; bf16 KV
// at head_dim 64). Defined in pa_prefill_wide.hip.
bool prefill_split_supported(int kv_dtype, int head_dim, int block_size);
int64_t prefill_split_units(int32_t batch, int32_t num_heads, int32_t query_len);
int launch_prefill_split(const AttnArgs& a, int io_dtype, hipStream_t stream);

// Generic one-wavefront-per-(request, head, query row) kernel for shapes without a tuned kernel
// (any block_size, head_dim <= 512). Defined in pa_decode.hip.
int launch_generic_attention(const AttnArgs& a, int io_dtype, int kv_dtype, hipStream_t stream);

}  // namespace pa
