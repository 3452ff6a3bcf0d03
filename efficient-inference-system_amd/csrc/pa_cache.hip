// Paged KV cache kernels for gfx950: append/scatter of new K/V rows into pool slots, ragged
// metadata packing (page table, sequence lengths, slot mapping), and batched block zeroing.
// All three are integer/byte work bound by HBM or launch latency; each is one launch.
#include <type_traits>

#include "pa_common.h"

namespace pa {

struct AppendArgs {
  const void* k_new;
  const void* v_new;
  int64_t sb, sh, st;
  void* k_pool;
  void* v_pool;
  int64_t num_blocks;
  const int32_t* slots;
  int32_t B, H, T, HD, BS;
};

// One thread per (row, head, element); rows are (request, token) pairs. Copy with conversion.
template <typename SRC, typename DST>
__global__ __launch_bounds__(256) void kv_append_kernel(const AppendArgs a) {
  const int64_t total = (int64_t)a.B * a.T * a.H * a.HD;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += stride) {
    const int d = (int)(idx % a.HD);
    const int64_t rest = idx / a.HD;
    const int h = (int)(rest % a.H);
    const int64_t row = rest / a.H;  // b * T + j
    const int32_t slot = a.slots[row];
    if (slot < 0) continue;
    const int64_t blk = slot / a.BS;
    const int off = slot - (int)blk * a.BS;
    if (blk >= a.num_blocks) continue;
    const int b = (int)(row / a.T);
    const int j = (int)(row - (int64_t)b * a.T);
    const int64_t src = (int64_t)b * a.sb + (int64_t)h * a.sh + (int64_t)j * a.st + d;
    const int64_t dst = ((blk * a.H + h) * a.BS + off) * a.HD + d;
    if constexpr (std::is_same<SRC, DST>::value) {
      static_cast<DST*>(a.k_pool)[dst] = static_cast<const SRC*>(a.k_new)[src];
      static_cast<DST*>(a.v_pool)[dst] = static_cast<const SRC*>(a.v_new)[src];
    } else {
      Elem<DST>::store(static_cast<DST*>(a.k_pool) + dst, Elem<SRC>::load(static_cast<const SRC*>(a.k_new) + src));
      Elem<DST>::store(static_cast<DST*>(a.v_pool) + dst, Elem<SRC>::load(static_cast<const SRC*>(a.v_new) + src));
    }
  }
}

struct PackArgs {
  const int32_t* ids;
  const int32_t* row_offsets;
  const int32_t* prev_lens;
  const int32_t* append_lens;
  int32_t B, T, BS, max_pages;
  int32_t* page_table;
  int64_t pt_stride;
  int32_t* seq_lens;
  int64_t* seq_lens64;
  int32_t* slots;
};

// Index space: [page table B*max_pages | seq_lens B | slot mapping B*T].
__global__ __launch_bounds__(256) void pack_metadata_kernel(const PackArgs a) {
  const int64_t n_pt = (int64_t)a.B * a.max_pages;
  const int64_t n_sl = a.B;
  const int64_t n_slot = a.slots ? (int64_t)a.B * a.T : 0;
  const int64_t total = n_pt + n_sl + n_slot;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += stride) {
    if (idx < n_pt) {
      const int b = (int)(idx / a.max_pages);
      const int p = (int)(idx - (int64_t)b * a.max_pages);
      const int beg = a.row_offsets[b];
      const int cnt = a.row_offsets[b + 1] - beg;
      a.page_table[(int64_t)b * a.pt_stride + p] = p < cnt ? a.ids[beg + p] : -1;
    } else if (idx < n_pt + n_sl) {
      const int b = (int)(idx - n_pt);
      const int32_t s = a.prev_lens[b] + a.append_lens[b];
      a.seq_lens[b] = s;
      if (a.seq_lens64) a.seq_lens64[b] = s;
    } else {
      const int64_t r = idx - n_pt - n_sl;
      const int b = (int)(r / a.T);
      const int j = (int)(r - (int64_t)b * a.T);
      int32_t slot = -1;
      if (j < a.append_lens[b]) {
        const int pos = a.prev_lens[b] + j;
        const int pi = pos / a.BS;
        const int beg = a.row_offsets[b];
        const int cnt = a.row_offsets[b + 1] - beg;
        if (pi < cnt) {
          const int32_t blk = a.ids[beg + pi];
          if (blk >= 0) slot = blk * a.BS + (pos - pi * a.BS);
        }
      }
      a.slots[r] = slot;
    }
  }
}

struct MirrorPackArgs {
  int32_t* mirror;
  int64_t mirror_stride;
  int32_t mirror_rows;
  const int32_t* mirror_row;
  const int32_t* first_page;
  const int32_t* num_pages;
  const int32_t* update_ids;
  int64_t update_stride;
  const int32_t* prev_lens;
  const int32_t* append_lens;
  int32_t B, T, BS, max_pages;
  int32_t* page_table;
  int64_t pt_stride;
  int32_t* seq_lens;
  int64_t* seq_lens64;
  int32_t* slots;
  const int32_t* stage_src;
  int32_t* stage_dst;
  int32_t stage_words;
};

constexpr int kMirrorSlice = 1024;  // update ids a workgroup stages in LDS (longer lists: read in place)

// One workgroup per request. Request b's block list is its mirror row's first first_page[b] ids
// followed by its update ids (update_ids + b * update_stride), which are also written into the row.
// The row is read only below first_page and written only from it on, so no workgroup reads what
// another writes (the host gives every request of a step its own row). The inputs may sit in host
// memory, where every dependent read costs a bus round trip: the update slice is loaded into LDS
// together with the request's header words and the staging copy, all independent of each other,
// so only the mirror row (device memory) is read after the header arrives.
__global__ __launch_bounds__(256) void pack_metadata_mirror_kernel(const MirrorPackArgs a) {
  __shared__ int32_t upd[kMirrorSlice];
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t slice = a.update_stride < kMirrorSlice ? a.update_stride : kMirrorSlice;
  const int32_t* my_upd = a.update_ids ? a.update_ids + (int64_t)b * a.update_stride : nullptr;
  if (my_upd)
    for (int k = tid; k < slice; k += 256) upd[k] = my_upd[k];
  for (int64_t i = (int64_t)b * 256 + tid; i < a.stage_words; i += (int64_t)a.B * 256) a.stage_dst[i] = a.stage_src[i];
  const int row = a.mirror_row[b];
  int first = a.first_page[b];
  int npages = a.num_pages[b];
  const int32_t prev = a.prev_lens[b];
  const int32_t app = a.append_lens[b];
  __syncthreads();

  const bool row_ok = row >= 0 && row < a.mirror_rows;
  int32_t* mrow = a.mirror + (int64_t)(row_ok ? row : 0) * a.mirror_stride;
  first = first < 0 ? 0 : (first > a.mirror_stride ? (int)a.mirror_stride : first);
  if (!row_ok) first = 0;
  int n_upd = npages - first;
  n_upd = n_upd < 0 ? 0 : (n_upd > a.update_stride ? (int)a.update_stride : n_upd);
  if (!my_upd) n_upd = 0;
  npages = first + n_upd;
  auto block_at = [&](int p) -> int32_t {
    if (p < first) return mrow[p];
    if (p < npages) return p - first < slice ? upd[p - first] : my_upd[p - first];
    return -1;
  };

  for (int p = tid; p < a.max_pages; p += 256) a.page_table[(int64_t)b * a.pt_stride + p] = block_at(p);
  if (row_ok)
    for (int k = tid; k < n_upd && first + k < a.mirror_stride; k += 256)
      mrow[first + k] = k < slice ? upd[k] : my_upd[k];
  if (tid == 0) {
    a.seq_lens[b] = prev + app;
    if (a.seq_lens64) a.seq_lens64[b] = prev + app;
  }
  if (a.slots) {
    for (int j = tid; j < a.T; j += 256) {
      int32_t slot = -1;
      if (j < app) {
        const int pos = prev + j;
        const int pi = pos / a.BS;
        if (pi < npages) {
          const int32_t blk = block_at(pi);
          if (blk >= 0) slot = blk * a.BS + (pos - pi * a.BS);
        }
      }
      a.slots[(int64_t)b * a.T + j] = slot;
    }
  }
}

// Zero K and V tiles of the listed blocks: 16-byte stores, grid-stride over (id, vector).
__global__ __launch_bounds__(256) void zero_blocks_kernel(uint4* k_pool, uint4* v_pool, int64_t num_blocks,
                                                          int64_t vecs_per_block, const int32_t* ids,
                                                          int32_t n_ids) {
  const int64_t total = (int64_t)n_ids * vecs_per_block;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const uint4 z = {0u, 0u, 0u, 0u};
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += stride) {
    const int64_t k = idx / vecs_per_block;
    const int64_t v = idx - k * vecs_per_block;
    const int32_t blk = ids[k];
    if (blk < 0 || blk >= num_blocks) continue;
    k_pool[blk * vecs_per_block + v] = z;
    v_pool[blk * vecs_per_block + v] = z;
  }
}

static unsigned grid_for(int64_t total, int cap_per_cu = 8) {
  const int64_t want = (total + 255) / 256;
  const int64_t cap = (int64_t)pa_host::device_cu_count() * cap_per_cu;
  const int64_t g = want < cap ? want : cap;
  return (unsigned)(g > 0 ? g : 1);
}

}  // namespace pa

using namespace pa;

extern "C" int pa_kv_append(const void* k_new, const void* v_new, int64_t new_stride_b, int64_t new_stride_h,
                            int64_t new_stride_t, int new_dtype,
                            void* k_pool, void* v_pool, int pool_dtype, int64_t num_blocks,
                            const int32_t* slot_mapping,
                            int32_t batch, int32_t num_heads, int32_t query_len, int32_t head_dim,
                            int32_t block_size, void* stream_) {
  pa_host::clear_error();
  PA_CHECK_ARG(batch >= 0 && num_heads > 0 && query_len >= 0 && head_dim > 0 && block_size > 0,
               "bad sizes: batch=%d heads=%d query_len=%d head_dim=%d block_size=%d", batch, num_heads,
               query_len, head_dim, block_size);
  PA_CHECK_ARG(new_dtype == PA_DTYPE_F32 || new_dtype == PA_DTYPE_BF16, "bad source dtype %d", new_dtype);
  PA_CHECK_ARG(pool_dtype == PA_DTYPE_F32 || pool_dtype == PA_DTYPE_BF16, "bad pool dtype %d", pool_dtype);
  const int64_t total = (int64_t)batch * query_len * num_heads * head_dim;
  if (total == 0) return PA_OK;
  PA_CHECK_ARG(k_new && v_new && k_pool && v_pool && slot_mapping, "null pointer argument");
  PA_CHECK_ARG(num_blocks > 0, "empty pool");
  AppendArgs a{k_new, v_new, new_stride_b, new_stride_h, new_stride_t, k_pool, v_pool, num_blocks,
               slot_mapping, batch, num_heads, query_len, head_dim, block_size};
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  const dim3 grid(grid_for(total)), block(256);
  if (new_dtype == PA_DTYPE_F32 && pool_dtype == PA_DTYPE_F32)
    kv_append_kernel<float, float><<<grid, block, 0, stream>>>(a);
  else if (new_dtype == PA_DTYPE_F32 && pool_dtype == PA_DTYPE_BF16)
    kv_append_kernel<float, uint16_t><<<grid, block, 0, stream>>>(a);
  else if (new_dtype == PA_DTYPE_BF16 && pool_dtype == PA_DTYPE_F32)
    kv_append_kernel<uint16_t, float><<<grid, block, 0, stream>>>(a);
  else
    kv_append_kernel<uint16_t, uint16_t><<<grid, block, 0, stream>>>(a);
  PA_CHECK_LAUNCH("kv append kernel");
  return PA_OK;
}

extern "C" int pa_pack_metadata(const int32_t* block_ids, const int32_t* row_offsets,
                                const int32_t* prev_lens, const int32_t* append_lens,
                                int32_t batch, int32_t query_len, int32_t block_size, int32_t max_pages,
                                int32_t* page_table, int64_t pt_stride, int32_t* seq_lens,
                                int64_t* seq_lens64, int32_t* slot_mapping, void* stream_) {
  pa_host::clear_error();
  PA_CHECK_ARG(batch >= 0 && query_len >= 0 && block_size > 0 && max_pages >= 0,
               "bad sizes: batch=%d query_len=%d block_size=%d max_pages=%d", batch, query_len, block_size,
               max_pages);
  if (batch == 0) return PA_OK;
  PA_CHECK_ARG(row_offsets && prev_lens && append_lens && seq_lens, "null metadata pointer");
  PA_CHECK_ARG(max_pages == 0 || (page_table && pt_stride >= max_pages), "page table missing or stride < max_pages");
  PackArgs a{block_ids, row_offsets, prev_lens, append_lens, batch, query_len, block_size, max_pages,
             page_table, pt_stride, seq_lens, seq_lens64, slot_mapping};
  const int64_t total = (int64_t)batch * max_pages + batch + (slot_mapping ? (int64_t)batch * query_len : 0);
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  pack_metadata_kernel<<<grid_for(total), 256, 0, stream>>>(a);
  PA_CHECK_LAUNCH("pack metadata kernel");
  return PA_OK;
}

extern "C" int pa_pack_metadata_mirror(int32_t* mirror, int64_t mirror_stride, int32_t mirror_rows,
                                       const int32_t* mirror_row, const int32_t* first_page,
                                       const int32_t* num_pages, const int32_t* update_ids, int64_t update_stride,
                                       const int32_t* prev_lens, const int32_t* append_lens,
                                       int32_t batch, int32_t query_len, int32_t block_size, int32_t max_pages,
                                       int32_t* page_table, int64_t pt_stride, int32_t* seq_lens,
                                       int64_t* seq_lens64, int32_t* slot_mapping,
                                       const int32_t* stage_src, int32_t* stage_dst, int32_t stage_words,
                                       void* stream_) {
  pa_host::clear_error();
  PA_CHECK_ARG(batch >= 0 && query_len >= 0 && block_size > 0 && max_pages >= 0 && stage_words >= 0 &&
                   update_stride >= 0,
               "bad sizes: batch=%d query_len=%d block_size=%d max_pages=%d stage_words=%d update_stride=%lld",
               batch, query_len, block_size, max_pages, stage_words, (long long)update_stride);
  PA_CHECK_ARG(mirror_rows > 0 && mirror_stride > 0, "bad mirror shape: rows=%d stride=%lld", mirror_rows,
               (long long)mirror_stride);
  if (batch == 0) {
    PA_CHECK_ARG(stage_words == 0, "stage words need at least one request");
    return PA_OK;
  }
  PA_CHECK_ARG(mirror && mirror_row && first_page && num_pages && prev_lens && append_lens && seq_lens,
               "null metadata pointer");
  PA_CHECK_ARG(update_stride == 0 || update_ids, "update_ids missing");
  PA_CHECK_ARG(max_pages == 0 || (page_table && pt_stride >= max_pages), "page table missing or stride < max_pages");
  PA_CHECK_ARG(stage_words == 0 || (stage_src && stage_dst), "null staging pointer");
  MirrorPackArgs a{mirror, mirror_stride, mirror_rows, mirror_row, first_page, num_pages, update_ids, update_stride,
                   prev_lens, append_lens, batch, query_len, block_size, max_pages, page_table, pt_stride,
                   seq_lens, seq_lens64, slot_mapping, stage_src, stage_dst, stage_words};
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  pack_metadata_mirror_kernel<<<(unsigned)batch, 256, 0, stream>>>(a);
  PA_CHECK_LAUNCH("pack metadata (mirror) kernel");
  return PA_OK;
}

extern "C" int pa_zero_blocks(void* k_pool, void* v_pool, int pool_dtype, int64_t num_blocks,
                              int32_t num_heads, int32_t block_size, int32_t head_dim,
                              const int32_t* block_ids, int32_t n_ids, void* stream_) {
  pa_host::clear_error();
  PA_CHECK_ARG(pool_dtype == PA_DTYPE_F32 || pool_dtype == PA_DTYPE_BF16, "bad pool dtype %d", pool_dtype);
  PA_CHECK_ARG(num_heads > 0 && block_size > 0 && head_dim > 0 && n_ids >= 0, "bad sizes");
  if (n_ids == 0) return PA_OK;
  PA_CHECK_ARG(k_pool && v_pool && block_ids && num_blocks > 0, "null pointer argument or empty pool");
  const int64_t bytes = (int64_t)num_heads * block_size * head_dim * (pool_dtype == PA_DTYPE_F32 ? 4 : 2);
  PA_CHECK_ARG(bytes % 16 == 0, "block tile bytes %lld not a multiple of 16", (long long)bytes);
  const int64_t vecs = bytes / 16;
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  zero_blocks_kernel<<<grid_for((int64_t)n_ids * vecs), 256, 0, stream>>>(
      static_cast<uint4*>(k_pool), static_cast<uint4*>(v_pool), num_blocks, vecs, block_ids, n_ids);
  PA_CHECK_LAUNCH("zero blocks kernel");
  return PA_OK;
}
