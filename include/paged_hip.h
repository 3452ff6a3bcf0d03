/*
 * paged_hip.h — C ABI of libpaged_hip.so, the MI355X (gfx950) paged-attention backend.
 *
 * Every entry point takes plain device pointers, element strides and sizes, plus the HIP stream
 * (as `void*`, a `hipStream_t`) to launch on. None of them allocates device memory, synchronises
 * the stream or reads device memory on the host. All return PA_OK (0) or a PA_ERR_* code;
 * pa_last_error_message() describes the most recent failure of the calling thread.
 *
 * Data layout contract (the reference's, jacobzhang22/efficient-inference-system):
 *   - KV pool K and V:  [num_blocks, num_heads, block_size, head_dim], contiguous
 *                        (src/cache/paged_kv.py:54-61 of the reference).
 *   - q / out:           [B, H, T, head_dim] with arbitrary element strides for B, H, T and unit
 *                        stride for head_dim (the reference passes a transposed view,
 *                        src/model/attention.py:25-29).
 *   - page_table:        int32 [B, max_pages] with row stride pt_stride, -1 padded
 *                        (src/cache/paged_kv.py:174-193).
 *   - seq_lens:          int32 [B], the cached length of each request AFTER the append
 *                        (src/cache/paged_kv.py:195-197).
 *   - cur_lens:          int32 [B], the request's current_lengths value
 *                        (src/kernels/paged_attention.py:27-32).
 *
 * Attention semantics (src/kernels/reference_paged_attention.py:10-59): for request b, head h and
 * query row i, with L = seq_lens[b] and C = cur_lens[b], the row attends key positions
 * t < n_i = clamp(min(L, L - C + 1 + i), 0, L) with softmax(q.k * scale) weights; a row with no
 * key (n_i == 0) is all zeros. Rows i >= C (padding) follow the same formula. Keys whose page-table
 * entry is negative or >= num_blocks are skipped, like the reference Triton kernels skip -1 pages
 * (src/kernels/triton_paged_attention.py:55).
 */
#ifndef PAGED_HIP_H_
#define PAGED_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types of q/out ("io") and of the KV pool. */
enum pa_dtype {
  PA_DTYPE_F32 = 0,
  PA_DTYPE_BF16 = 1,
};

/* Status codes. */
enum pa_status {
  PA_OK = 0,
  PA_ERR_INVALID_ARGUMENT = 1, /* a null pointer, negative size or inconsistent shape */
  PA_ERR_UNSUPPORTED = 2,      /* a dtype / head_dim / block_size combination with no kernel */
  PA_ERR_WORKSPACE = 3,        /* workspace missing or smaller than pa_decode_workspace_size() */
  PA_ERR_HIP = 4,              /* a HIP runtime call failed (launch or attribute query) */
};

/* Library version, major*10000 + minor*100 + patch. */
int pa_version(void);

/* Human-readable message for the most recent failing call on this thread ("" if none). */
const char* pa_last_error_message(void);

/*
 * Paged DECODE attention (query_len == 1).
 * Replaces the reference's paged_attention_decode_triton
 * (src/kernels/triton_paged_attention.py:179-217) behind paged_attention()
 * (src/kernels/paged_attention.py:34-42).
 *
 * One workgroup of wavefronts per (request, head, split); the wavefronts split the request's KV
 * blocks between them and merge their online-softmax states in LDS. When split_blocks > 0 and a
 * request has more than split_blocks KV blocks, its blocks are also divided among several
 * workgroups whose partial results are merged: with at most 8 splits per request (and at most
 * PA_DECODE_COUNTER_BYTES / 4 (request, head) pairs) by the split that finishes last, in the same
 * launch, otherwise by a second kernel. That path needs a workspace of pa_decode_workspace_size()
 * bytes whose first PA_DECODE_COUNTER_BYTES hold per-(request, head) arrival counters: they must
 * be zero before the workspace is first used, and every call leaves them zero, so one zeroing at
 * allocation serves all later calls of any shape; other calls (pa_prefill) must not write into
 * that region. split_blocks <= 0 means one workgroup per (request, head) and no workspace.
 *
 * order: optional int32 [B] permutation giving the processing order of requests (e.g. longest
 * first, for load balance); NULL means 0..B-1. Results do not depend on it.
 */
int pa_decode(const void* q, int64_t q_stride_b, int64_t q_stride_h,
              void* out, int64_t out_stride_b, int64_t out_stride_h, int io_dtype,
              const void* k_pool, const void* v_pool, int kv_dtype, int64_t num_blocks,
              const int32_t* page_table, int64_t pt_stride, int32_t max_pages,
              const int32_t* seq_lens, const int32_t* cur_lens, const int32_t* order,
              int32_t batch, int32_t num_heads, int32_t head_dim, int32_t block_size,
              float scale, int32_t split_blocks,
              void* workspace, size_t workspace_bytes, void* stream);

/* Bytes of workspace pa_decode needs for these sizes (0 when split_blocks <= 0 or no request can
 * need more than one split; otherwise PA_DECODE_COUNTER_BYTES + 4 * batch * num_heads * splits *
 * (head_dim + 2)). No reference counterpart: the Triton decode path has no split-K.
 * Calls that share a workspace must not run concurrently (e.g. on different streams). */
size_t pa_decode_workspace_size(int32_t batch, int32_t num_heads, int32_t head_dim,
                                int32_t max_pages, int32_t split_blocks);

/* Bytes at the start of a decode split workspace that hold the arrival counters (see pa_decode). */
#define PA_DECODE_COUNTER_BYTES ((size_t)256 << 10)

/* Size of the fixed per-device scratch array that pa_decode_noalloc keeps its arrival counters
 * and split records in (the same layout as a pa_decode workspace). */
#define PA_DECODE_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)

/*
 * pa_decode without a workspace argument and without any device allocation: the same kernels
 * and results as pa_decode with the same arguments, but the split-K records (when split_blocks
 * splits a request) go to a fixed device array of PA_DECODE_NOALLOC_SCRATCH_BYTES inside the
 * library, one per device, resolved on the first call on that device. No counterpart in the
 * reference: this is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). A call whose workspace size
 * (pa_decode_workspace_size: the counters and the records) exceeds the array fails with
 * PA_ERR_INVALID_ARGUMENT before any launch. The array starts at zero when the library is loaded
 * and every call leaves its counters zero, but every call on a device shares that device's
 * array: calls that overlap on one device (e.g. on two streams) race and must be serialised.
 */
int pa_decode_noalloc(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                      void* out, int64_t out_stride_b, int64_t out_stride_h, int io_dtype,
                      const void* k_pool, const void* v_pool, int kv_dtype, int64_t num_blocks,
                      const int32_t* page_table, int64_t pt_stride, int32_t max_pages,
                      const int32_t* seq_lens, const int32_t* cur_lens, const int32_t* order,
                      int32_t batch, int32_t num_heads, int32_t head_dim, int32_t block_size,
                      float scale, int32_t split_blocks, void* stream);

/*
 * Paged chunked-PREFILL attention (any query_len >= 1), causal over cached context plus the
 * in-chunk prefix. Replaces paged_attention_prefill_triton
 * (src/kernels/triton_paged_attention.py:220-258) behind paged_attention()
 * (src/kernels/paged_attention.py:44-51). fp32 KV uses fp32 MFMA (16x16x4); bf16 KV uses bf16
 * MFMA with fp32 accumulation (q and the softmax weights are rounded to bf16 for the products).
 * Work is one workgroup per (request, head, 16-row query tile); with split_blocks > 0 each tile's
 * KV blocks are also cut into ranges of split_blocks blocks, one workgroup each, whose partial
 * results a second kernel merges through a workspace of pa_prefill_workspace_size() bytes.
 * split_blocks == 0 means no split and no workspace. split_blocks < 0 (PA_PREFILL_BALANCED) asks
 * for the balanced launch where the library finds it faster: head_dim 128 or 64, num_heads a
 * multiple of 8, batch <= 255, at most one (request, head, 128-row tile) unit per two compute units
 * and at head_dim 128 at least 8192 unit-steps (units x ceil(max_pages / 2); fp32 KV: 4096 from one
 * unit per four compute units); at head_dim 64 at least 16384 unit-steps (steps of 64 keys for bf16
 * KV, 32 for fp32 KV) or 256 steps per unit (fp32 KV: at most one unit per 16 compute units), for
 * fp32 KV not where the 16-row kernel would run one to two workgroups per compute unit; i.e. few
 * tiles over long contexts. It runs a grid of one or two workgroups per compute unit, deals the tiles' KV steps out
 * evenly among them and merges a tile cut between workgroups in the same launch (the one that
 * finishes it last). Other calls run as with 0. The environment variable
 * PAGED_HIP_PREFILL_BALANCE=force takes it wherever it can run (as many workgroups per compute
 * unit as fit on larger grids), =off never. Every prefill workspace starts with PA_PREFILL_COUNTER_BYTES of
 * arrival counters that must be zero before its first use; every call leaves them zero. Calls that
 * share a workspace must not run concurrently (e.g. on different streams).
 */
int pa_prefill(const void* q, int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_t,
               void* out, int64_t out_stride_b, int64_t out_stride_h, int64_t out_stride_t,
               int io_dtype,
               const void* k_pool, const void* v_pool, int kv_dtype, int64_t num_blocks,
               const int32_t* page_table, int64_t pt_stride, int32_t max_pages,
               const int32_t* seq_lens, const int32_t* cur_lens,
               int32_t batch, int32_t num_heads, int32_t query_len, int32_t head_dim,
               int32_t block_size, float scale, int32_t split_blocks,
               void* workspace, size_t workspace_bytes, void* stream);

/* Bytes of workspace pa_prefill needs for these sizes (0 when neither a split nor the balanced
 * launch applies; for the balanced launch the larger of its bf16 and fp32 KV needs). No reference
 * counterpart: the Triton prefill path has no split-K. */
size_t pa_prefill_workspace_size(int32_t batch, int32_t num_heads, int32_t query_len, int32_t head_dim,
                                 int32_t max_pages, int32_t split_blocks);

#define PA_PREFILL_BALANCED (-1)
#define PA_PREFILL_COUNTER_BYTES ((size_t)64 << 10)

/*
 * KV append / scatter: writes k_new[b, :, j, :] and v_new[b, :, j, :] into pool slot
 * slot_mapping[b * query_len + j] (slot = block_id * block_size + offset; a negative slot skips
 * the row). Values are converted to the pool dtype (fp32 -> bf16 rounds to nearest even).
 * Replaces the per-request slice copies of PagedKVCacheState.append
 * (src/cache/paged_kv.py:102-120) driven by BatchedPagedKVCache.append_batch (:151-172).
 * Slots whose block is outside [0, num_blocks) are skipped.
 */
int pa_kv_append(const void* k_new, const void* v_new, int64_t new_stride_b, int64_t new_stride_h,
                 int64_t new_stride_t, int new_dtype,
                 void* k_pool, void* v_pool, int pool_dtype, int64_t num_blocks,
                 const int32_t* slot_mapping,
                 int32_t batch, int32_t num_heads, int32_t query_len, int32_t head_dim,
                 int32_t block_size, void* stream);

/*
 * Ragged metadata packing for one batched append + attention call, from a CSR list of each
 * request's block ids (block_ids[row_offsets[b] .. row_offsets[b+1]) ):
 *   page_table[b, p]  = block id p of request b, or -1 past its end (p < max_pages);
 *                       replaces BatchedPagedKVCache.page_table_tensor (src/cache/paged_kv.py:174-193)
 *   seq_lens[b]       = prev_lens[b] + append_lens[b]   (int32; seq_lens64 gets the same as int64
 *                       when non-NULL, the value append_batch returns, src/cache/paged_kv.py:172)
 *   slot_mapping[b*query_len + j] = slot of the j-th appended token of request b for
 *                       j < append_lens[b], else -1 (NULL skips it)
 * append_lens must already be clamped to [0, query_len] (src/cache/paged_kv.py:169).
 */
int pa_pack_metadata(const int32_t* block_ids, const int32_t* row_offsets,
                     const int32_t* prev_lens, const int32_t* append_lens,
                     int32_t batch, int32_t query_len, int32_t block_size, int32_t max_pages,
                     int32_t* page_table, int64_t pt_stride, int32_t* seq_lens,
                     int64_t* seq_lens64, int32_t* slot_mapping, void* stream);

/*
 * pa_pack_metadata with the block lists kept on the device between steps, so a step sends only
 * what changed: mirror is int32 [mirror_rows, mirror_stride] device memory that persists across
 * calls; request b of this step owns row mirror_row[b] (distinct rows within a call), and its
 * block list (num_pages[b] ids) is the row's first first_page[b] ids followed by the
 * num_pages[b] - first_page[b] ids at update_ids + b * update_stride, which the call also writes
 * into the row from first_page[b] on. Outputs are those of pa_pack_metadata for that list
 * (page_table, seq_lens, seq_lens64, slot_mapping; the last two may be NULL). The call also copies
 * stage_words int32 words from stage_src to stage_dst (0: none), so a step's other small inputs
 * (token ids, positions, lengths) reach device buffers in the same launch. The inputs may live in
 * pinned host memory the device can read (hipHostMalloc), which lets a captured step take new
 * inputs without a copy call; the host must then not rewrite them until the launch has run. No
 * reference counterpart as one call: together with the host's diff of each request's block list
 * against what its row holds, it replaces the per-call rebuild of page_table_tensor /
 * seq_lens_tensor (src/cache/paged_kv.py:174-197) from every request's whole block list.
 */
int pa_pack_metadata_mirror(int32_t* mirror, int64_t mirror_stride, int32_t mirror_rows,
                            const int32_t* mirror_row, const int32_t* first_page,
                            const int32_t* num_pages, const int32_t* update_ids, int64_t update_stride,
                            const int32_t* prev_lens, const int32_t* append_lens,
                            int32_t batch, int32_t query_len, int32_t block_size, int32_t max_pages,
                            int32_t* page_table, int64_t pt_stride, int32_t* seq_lens,
                            int64_t* seq_lens64, int32_t* slot_mapping,
                            const int32_t* stage_src, int32_t* stage_dst, int32_t stage_words,
                            void* stream);

/*
 * Zero the K and V tiles of n_ids pool blocks (block_ids on device), the batched form of
 * LayerBlockPool.release_block's per-block zero_() (src/cache/paged_kv.py:80-85).
 * Ids outside [0, num_blocks) are skipped.
 */
int pa_zero_blocks(void* k_pool, void* v_pool, int pool_dtype, int64_t num_blocks,
                   int32_t num_heads, int32_t block_size, int32_t head_dim,
                   const int32_t* block_ids, int32_t n_ids, void* stream);

/*
 * Step linear layers of the model around the paged attention (fp32 or bf16). No reference
 * counterpart as entry points: they replace the torch nn.Linear / nn.LayerNorm / nn.GELU calls of
 * the reference's cached forward (src/model/transformer.py:30-35, src/model/attention.py:46-48,64)
 * on one-token steps and prefill chunks, where a step is a few rows against every weight matrix.
 * Up to a few dozen rows a workgroup reads its weight tile once per 16 rows; above that a tiled
 * kernel reads it once per 32 rows. They pay off up to 48-1536 rows depending on the layer; rows is
 * at most 2048.
 *
 * pa_linear_rows: out[m, :] = act(LN(x[m, :]) W^T + bias) + residual[m, :] for m < rows.
 *   dtype (PA_DTYPE_F32 or PA_DTYPE_BF16) is the element type of x, weight, bias, LayerNorm
 *   parameters, residual and out alike; products accumulate in fp32 (bf16: LN(x) is rounded to
 *   bf16 before the product, as torch's bf16 LayerNorm output is, and out is rounded once);
 *   weight is torch's [out_features, in_features] row-major; in_features must be 128, 256, 512,
 *   1024 or 2048;
 *   ln_weight/ln_bias NULL skips the LayerNorm (biased variance, eps ln_eps, like
 *   torch.nn.LayerNorm); bias and residual may be NULL; activation 0 = none, 1 = exact (erf)
 *   GELU (torch.nn.GELU()). x, weight and LayerNorm parameters 16-byte aligned, x_stride a
 *   multiple of 16 bytes.
 *   out_copy (or NULL): the same rows are also written there (row stride out_copy_stride); it may be
 *   `residual` itself (each element is read and written by one thread). A decode step uses it to
 *   seed the buffer pa_mlp_rows accumulates into with the out_proj rows (x + attention output).
 */
int pa_linear_rows(const void* x, int64_t x_stride, int32_t rows, int32_t in_features,
                   const void* weight, const void* bias, int32_t out_features,
                   const void* ln_weight, const void* ln_bias, float ln_eps,
                   int32_t activation, const void* residual, int64_t residual_stride,
                   void* out, int64_t out_stride, void* out_copy, int64_t out_copy_stride,
                   int dtype, void* stream);

/*
 * pa_linear_select_rows: pa_linear_rows over one selected row per group of x, without a residual:
 * out[g, :] = act(LN(x[g * group_rows + r_g, :]) W^T + bias) for g < groups, where r_g =
 * row_index[g] (device int32; a negative value counts from the group's end, as Python indexing
 * does, and the result is clamped into [0, group_rows)). Same dtypes, shapes and alignment as
 * pa_linear_rows; groups is at most 2048. No reference counterpart as an entry point: it computes
 * ln_f + lm_head (src/model/transformer.py:176-177) only for the row of each request whose greedy
 * token the executors take (src/serving/continuous_generate.py:145,238), instead of every row
 * of a prefill chunk.
 * token_keys (device uint64, 8-byte aligned, or NULL; group g's key at token_keys[g *
 * token_keys_stride], token_keys_stride >= 1): when set, each group's greedy token is folded in
 * as well, the argmax the executors take (continuous_generate.py:145,238) without a separate
 * launch: group g's key is lowered (atomic minimum) to the least key over the group's
 * out_features columns, key = ((uint64)~ord(v) << 32) | column, v the column's output as stored
 * (rounded to dtype) and ord the order-preserving bits of v (NaN highest, -0.0 = +0.0). The
 * caller sets the keys to all ones before the call; afterwards the low 32 bits of group g's key
 * are torch.argmax of out[g, :] (the first index of the maximum; the first NaN if any). Every
 * workgroup of the launch sends one atomic per group, so keys 128 bytes apart (stride 16) keep
 * the groups' atomics off one cache line.
 */
int pa_linear_select_rows(const void* x, int64_t x_stride, int32_t groups, int32_t group_rows,
                          const int32_t* row_index, int32_t in_features, const void* weight,
                          const void* bias, int32_t out_features, const void* ln_weight,
                          const void* ln_bias, float ln_eps, int32_t activation, void* out,
                          int64_t out_stride, uint64_t* token_keys, int64_t token_keys_stride,
                          int dtype, void* stream);

/*
 * pa_qkv_append: the three projections of a cached attention layer in one launch, with the
 * LayerNorm before them and the KV append after them: q_out[m, :] = LN(x[m, :]) wq^T + bq, and
 * the rows LN(x[m, :]) wk^T + bk and LN(x[m, :]) wv^T + bv are written, split into num_heads
 * vectors of head_dim, into pool slot slot_mapping[m] of the K and V pools (converted to the pool
 * dtype; slot < 0 or a block outside [0, num_blocks) skips the row). dtype is the element type of
 * x, the weights, biases, LayerNorm parameters and q_out (as pa_linear_rows). Replaces
 * src/model/attention.py:46-56 (q/k/v projections, then append_batch) for rows <= 2048 and
 * d_model in {128, 256, 512, 1024, 2048}.
 */
int pa_qkv_append(const void* x, int64_t x_stride, int32_t rows, int32_t d_model,
                  const void* ln_weight, const void* ln_bias, float ln_eps,
                  const void* wq, const void* bq, const void* wk, const void* bk,
                  const void* wv, const void* bv,
                  void* q_out, int64_t q_stride,
                  void* k_pool, void* v_pool, int pool_dtype, int64_t num_blocks,
                  const int32_t* slot_mapping, int32_t num_heads, int32_t head_dim,
                  int32_t block_size, int dtype, void* stream);

/*
 * pa_embed_rows: x[b*T + t, :] = token_table[ids[b, t], :] + pos_table[min(pos_start[b] + t,
 * max_pos - 1), :] for a [batch, query_len] step (ids and pos_start int64, tables row-major
 * [vocab, d_model] / [max_pos, d_model] of element type dtype, fp32 or bf16, like out; the sum is
 * formed in fp32); an id outside [0, vocab) gives a zero token row. Replaces the position
 * arithmetic and the two nn.Embedding lookups of the reference's forward
 * (src/model/transformer.py:144-150) in one launch.
 */
int pa_embed_rows(const int64_t* ids, const int64_t* pos_start, int32_t batch, int32_t query_len,
                  const void* token_table, int64_t vocab, const void* pos_table, int32_t max_pos,
                  int32_t d_model, void* out, int64_t out_stride, int dtype, void* stream);

/*
 * pa_argmax_rows: greedy token selection for a step of `batch` requests whose logits are
 * `rows_per_request` consecutive rows each (row m at logits + m * row_stride elements, `vocab`
 * values of type dtype): tokens[b] = argmax_v logits[b * rows_per_request + r_b, v] with
 * r_b = row_index[b] (NULL: 0; a negative value counts from the end of the request's rows, as a
 * Python index does; then clamped into [0, rows_per_request)). Ties and NaN follow torch.argmax:
 * the first index of the maximum, NaN above every number. Replaces the per-request
 * `torch.argmax(logits[b, row, :]).item()` of the continuous-batching executors
 * (src/serving/continuous_generate.py:145,238) and generate_with_cache
 * (src/inference/generate_with_cache.py:151,204), so a captured step returns token ids.
 */
int pa_argmax_rows(const void* logits, int64_t row_stride, int32_t batch, int32_t rows_per_request,
                   const int32_t* row_index, int32_t vocab, int dtype, int64_t* tokens, void* stream);

/*
 * pa_mlp_rows: out[m] += fc2(act(fc1(LayerNorm(x[m])))) + residual[m] for rows m < rows (at most
 * 16), fp32 (dtype must be PA_DTYPE_F32), in one launch: one workgroup per 16 columns of fc1 adds
 * its share of fc2 to `out` with device-scope atomic adds (the sum's order, and its last bits, vary
 * from run to run), so `out` must hold its starting value when the launch runs (zeros, or the
 * residual rows themselves: pa_linear_rows' `out_copy`).
 * d_model is 128, 256 or 512, d_ff a multiple of 16; fc1_weight is [d_ff, d_model] and
 * fc2_weight [d_model, d_ff] row-major (torch Linear weights), 16-byte aligned; activation 0 =
 * none, 1 = exact GELU; biases and residual may be NULL. Replaces the MLP block and its residual
 * add of the reference's transformer block (src/model/transformer.py:32-35) on decode steps.
 */
int pa_mlp_rows(const void* x, int64_t x_stride, int32_t rows, int32_t d_model,
                const void* ln_weight, const void* ln_bias, float ln_eps,
                const void* fc1_weight, const void* fc1_bias, int32_t d_ff, int32_t activation,
                const void* fc2_weight, const void* fc2_bias,
                const void* residual, int64_t residual_stride,
                void* out, int64_t out_stride, int dtype, void* stream);

/*
 * pa_hbm_read_probe: reads `bytes` (a multiple of 16) of device memory at `src` once, in order,
 * with the 16-byte non-temporal vector loads pa_decode streams KV tiles with, over `workgroups`
 * workgroups of `threads` (256, 512 or 1024) threads, each lane keeping `depth` (1, 4 or 8) loads
 * in flight; `sink` is a device buffer of `workgroups` uint32 words, which the probe may write
 * for a non-zero buffer (a buffer of zeros leaves it untouched). No counterpart in the reference:
 * it lets a benchmark state the read bandwidth the box delivers beside the decode kernel's,
 * separating the box from the kernel (the best of a sweep over the three shape arguments).
 */
int pa_hbm_read_probe(const void* src, size_t bytes, uint32_t* sink, int32_t workgroups, int32_t threads,
                      int32_t depth, void* stream);

/*
 * pa_hbm_chunk_read_probe: reads `chunks` 4 KB chunks of device memory at `src` (which holds at
 * least chunks x 4096 bytes) once each, in the order the device array `order` gives (chunk ids in
 * [0, chunks); other ids are skipped), with the same loads, over `workgroups` workgroups of 256
 * threads that keep `depth` (1, 2 or 4) chunks in flight; `sink` as for pa_hbm_read_probe. A
 * random order reads memory as a paged KV pool is read: one (block, head) slab of 16 tokens x 128
 * values x 2 bytes is one 4 KB chunk. No counterpart in the reference.
 */
int pa_hbm_chunk_read_probe(const void* src, const int32_t* order, int32_t chunks, uint32_t* sink,
                            int32_t workgroups, int32_t depth, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PAGED_HIP_H_ */
