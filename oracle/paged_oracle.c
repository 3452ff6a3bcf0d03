/*
 * ORACLE — test infrastructure only. This file is the CPU restatement of the reference's paged
 * attention path (jacobzhang22/efficient-inference-system) that the HIP kernels are checked
 * against. Only tests, the smoke check and the benchmark's CPU-baseline leg may load it; the
 * product library never does.
 *
 * Functions and the reference code each one restates:
 *   oracle_paged_attention  src/kernels/reference_paged_attention.py:10-59
 *       for each request b, head h, query row i: past = seq_len - cur_len (:33), keys
 *       t = 0.. while t <= past + i and t < seq_len (:40-43), key/value rows read from block
 *       block_ids[t / block_size] at offset t % block_size (:44-47), scores q.k * 1/sqrt(Hd)
 *       (:30, :48), softmax over the scores and weighted sum of values (:55-57); a row with no
 *       key stays zero (:16, :51-52). Accumulation here is in double precision.
 *   oracle_append           src/cache/paged_kv.py:102-120 and :151-172
 *       request b's first n_b = clamp(current_length, 0, T) new rows go to positions
 *       prev_len .. prev_len + n_b - 1, position p landing in block block_ids[p / block_size]
 *       at offset p % block_size; a bf16 pool receives round-to-nearest-even values.
 *   oracle_page_table       src/cache/paged_kv.py:174-193
 *       int32 [B, max_pages] of each request's block ids, -1 past the end of its list.
 *
 * `mutation` plants a known mistake (for tests proving the checks would catch it):
 *   0 none, 1 causal bound t < past+i (off by one), 2 scale dropped, 3 offset within a block
 *   reversed (row bs-1-t%bs read for t), 4 the last valid key dropped from every row.
 *
 * Pinned by: tests/test_oracle.py (closed-form softmax attention on gathered K/V through
 * torch.nn.functional.scaled_dot_product_attention in fp64, invariants, planted mistakes) and
 * tests/test_paged_kv.py (the reference's own allocator/append/page-table assertions).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline double kv_at(const void* pool, int dtype, int64_t idx) {
  if (dtype == 0) return (double)((const float*)pool)[idx];
  uint32_t u = (uint32_t)((const uint16_t*)pool)[idx] << 16;
  float f;
  memcpy(&f, &u, sizeof(f));
  return (double)f;
}

static inline void key_location(int t, int bs, int mutation, int* page, int* off) {
  *page = t / bs;
  *off = mutation == 3 ? bs - 1 - t % bs : t % bs;
}

static inline uint16_t f32_to_bf16_rne(float f) {
  uint32_t u;
  memcpy(&u, &f, sizeof(u));
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)0x7fc0u;
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

/* q, out: float [B, H, T, Hd] contiguous. block_ids / row_offsets: CSR block lists.
 * Returns 0, or -1 if a key position has no block in its request's list. */
int oracle_paged_attention(const float* q, const void* k_pool, const void* v_pool, int kv_dtype,
                           int64_t num_blocks, const int32_t* block_ids, const int32_t* row_offsets,
                           const int32_t* seq_lens, const int32_t* cur_lens, int B, int H, int T,
                           int Hd, int bs, float* out, int nthreads, int mutation) {
  const double scale = mutation == 2 ? 1.0 : 1.0 / sqrt((double)Hd);
  int status = 0;
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(dynamic, 1) collapse(2)
#endif
  for (int b = 0; b < B; ++b) {
    for (int h = 0; h < H; ++h) {
      const int L = seq_lens[b];
      const int past = L - cur_lens[b];
      const int beg = row_offsets[b];
      const int nids = row_offsets[b + 1] - beg;
      double* scores = (double*)malloc(sizeof(double) * (L > 0 ? L : 1));
      double* acc = (double*)malloc(sizeof(double) * Hd);
      for (int i = 0; i < T; ++i) {
        const float* qr = q + (((int64_t)b * H + h) * T + i) * Hd;
        float* orow = out + (((int64_t)b * H + h) * T + i) * Hd;
        int n = 0;
        for (int t = 0; t < L; ++t) {
          const int limit = past + i;
          if (mutation == 1 ? t >= limit : t > limit) break;
          int page, off;
          key_location(t, bs, mutation, &page, &off);
          if (page >= nids) { status = -1; break; }
          const int64_t blk = block_ids[beg + page];
          if (blk < 0 || blk >= num_blocks) { status = -1; break; }
          const int64_t base = ((blk * H + h) * bs + off) * (int64_t)Hd;
          double dot = 0.0;
          for (int d = 0; d < Hd; ++d) dot += (double)qr[d] * kv_at(k_pool, kv_dtype, base + d);
          scores[n++] = dot * scale;
        }
        if (mutation == 4 && n > 0) n -= 1;
        if (n == 0) {
          for (int d = 0; d < Hd; ++d) orow[d] = 0.0f;
          continue;
        }
        double mx = scores[0];
        for (int t = 1; t < n; ++t) mx = scores[t] > mx ? scores[t] : mx;
        double denom = 0.0;
        for (int t = 0; t < n; ++t) { scores[t] = exp(scores[t] - mx); denom += scores[t]; }
        for (int d = 0; d < Hd; ++d) acc[d] = 0.0;
        for (int t = 0; t < n; ++t) {
          int page, off;
          key_location(t, bs, mutation, &page, &off);
          const int64_t blk = block_ids[beg + page];
          const int64_t base = ((blk * H + h) * bs + off) * (int64_t)Hd;
          const double w = scores[t] / denom;
          for (int d = 0; d < Hd; ++d) acc[d] += w * kv_at(v_pool, kv_dtype, base + d);
        }
        for (int d = 0; d < Hd; ++d) orow[d] = (float)acc[d];
      }
      free(scores);
      free(acc);
    }
  }
  return status;
}

/* k_new, v_new: float [B, H, T, Hd] contiguous; pool dtype 0 = float, 1 = bf16 (uint16).
 * current_lengths are clamped to [0, T]. Returns 0, or -1 on a missing/invalid block. */
int oracle_append(const float* k_new, const float* v_new, int B, int H, int T, int Hd,
                  void* k_pool, void* v_pool, int pool_dtype, int64_t num_blocks, int bs,
                  const int32_t* block_ids, const int32_t* row_offsets, const int32_t* prev_lens,
                  const int32_t* current_lengths) {
  for (int b = 0; b < B; ++b) {
    int n = current_lengths[b];
    n = n < 0 ? 0 : (n > T ? T : n);
    const int beg = row_offsets[b];
    const int nids = row_offsets[b + 1] - beg;
    for (int j = 0; j < n; ++j) {
      const int p = prev_lens[b] + j;
      const int page = p / bs;
      if (page >= nids) return -1;
      const int64_t blk = block_ids[beg + page];
      if (blk < 0 || blk >= num_blocks) return -1;
      for (int h = 0; h < H; ++h) {
        const int64_t src = (((int64_t)b * H + h) * T + j) * Hd;
        const int64_t dst = ((blk * H + h) * bs + (p % bs)) * (int64_t)Hd;
        for (int d = 0; d < Hd; ++d) {
          if (pool_dtype == 0) {
            ((float*)k_pool)[dst + d] = k_new[src + d];
            ((float*)v_pool)[dst + d] = v_new[src + d];
          } else {
            ((uint16_t*)k_pool)[dst + d] = f32_to_bf16_rne(k_new[src + d]);
            ((uint16_t*)v_pool)[dst + d] = f32_to_bf16_rne(v_new[src + d]);
          }
        }
      }
    }
  }
  return 0;
}

void oracle_page_table(const int32_t* block_ids, const int32_t* row_offsets, int B, int max_pages,
                       int32_t* page_table) {
  for (int b = 0; b < B; ++b) {
    const int beg = row_offsets[b];
    const int cnt = row_offsets[b + 1] - beg;
    for (int p = 0; p < max_pages; ++p) page_table[(int64_t)b * max_pages + p] = p < cnt ? block_ids[beg + p] : -1;
  }
}

/* Round-to-nearest-even fp32 -> bf16 over an array (used to build bf16 pools identically). */
void oracle_f32_to_bf16(const float* src, uint16_t* dst, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dst[i] = f32_to_bf16_rne(src[i]);
}
