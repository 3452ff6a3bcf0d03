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
  int32_t num_splits;    // decode: workgroups per (request, head), >= 1
  int32_t split_blocks;  // decode: KV blocks per split when num_splits > 1
  float* ws;             // decode: [B*H*num_splits][head_dim + 2] partial (m, l, acc) records
};

// Generic one-wavefront-per-(request, head, query row) kernel for shapes without a tuned kernel
// (any block_size, head_dim <= 512). Defined in pa_decode.hip.
int launch_generic_attention(const AttnArgs& a, int io_dtype, int kv_dtype, hipStream_t stream);

}  // namespace pa
