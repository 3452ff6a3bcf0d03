// Paged decode attention for gfx950.
//
// Fast path (block_size 16, head_dim 64/128, fp32 or bf16 KV): one workgroup of NW wavefronts per
// (request, head, split). The wavefronts of a workgroup take the split's KV blocks round-robin.
// A (block, head) tile is block_size*head_dim contiguous elements (4 KiB for fp32/64 and
// bf16/128), so one wave-wide 16-byte load reads 1 KiB of it: lane l reads 16-byte vector
// (round*64 + l). A token row is LPR lanes wide; a lane holds EPL elements of TPL different rows
// per round. Scores are reduced over the LPR lanes of a row with DPP, and each group of LPR lanes
// keeps its own online-softmax state (max m, sum l, acc) for the rows it sees, so the inner loop
// needs no cross-row exchange. Groups merge with shuffles after the loop; wavefronts merge in LDS.
// The next block's K and V are loaded into a second register set while the current one is used.
#include <mutex>

#include "pa_attention.h"

// Tuning knobs (compile-time): wavefronts per workgroup, blocks loaded ahead of the one being
// folded, non-temporal (streaming) KV loads, and XCD-aware placement of a request's workgroups.
// Measured on MI355X on the large ragged batch (256 x 32 heads x 128, bf16, 34.9 GB per call):
// non-temporal loads raise the kernel from 76.8% to 85.6% of the 8 TB/s HBM peak; 4/8/16 waves,
// one or two tiles ahead and die-aware placement each move it by under 1% (16 waves with two
// tiles ahead spills registers and halves the rate).
#ifndef PA_DECODE_WAVES
#define PA_DECODE_WAVES 8
#endif
#ifndef PA_DECODE_DEPTH
#define PA_DECODE_DEPTH 1
#endif
#ifndef PA_DECODE_NT
#define PA_DECODE_NT 1
#endif
#ifndef PA_DECODE_XCD
#define PA_DECODE_XCD 0
#endif

namespace pa {

template <bool NT>
__device__ __forceinline__ u32x4 load16(const u32x4* p) {
  if constexpr (NT) return __builtin_nontemporal_load(p);
  return *p;
}

template <typename KV, int HD, int BS>
struct DecodeShape {
  static constexpr int EPL = Vec16<KV>::EPL;   // elements per lane per 16-byte load
  static constexpr int LPR = HD / EPL;          // lanes per token row
  static constexpr int TPL = kWave / LPR;       // token rows per wave-wide load
  static constexpr int ROUNDS = BS / TPL;       // wave-wide loads per tile
  static_assert(LPR >= 4 && LPR <= 64 && (LPR & (LPR - 1)) == 0, "row width");
  static_assert(BS % TPL == 0, "block size must be a multiple of rows per load");
};

template <bool NT, typename KV, int R>
__device__ __forceinline__ void load_tile(u32x4 (&kb)[R], u32x4 (&vb)[R], const KV* kpool,
                                          const KV* vpool, int64_t tile_off, int lane) {
  const u32x4* kt = reinterpret_cast<const u32x4*>(kpool + tile_off);
  const u32x4* vt = reinterpret_cast<const u32x4*>(vpool + tile_off);
#pragma unroll
  for (int r = 0; r < R; ++r) kb[r] = load16<NT>(kt + r * kWave + lane);
#pragma unroll
  for (int r = 0; r < R; ++r) vb[r] = load16<NT>(vt + r * kWave + lane);
}

// Fold one tile into the lane group's online-softmax state.
template <typename KV, int HD, int BS, int R, int E>
__device__ __forceinline__ void fold_tile(const u32x4 (&kb)[R], const u32x4 (&vb)[R],
                                          const float (&qv)[E], int tok0, int n, bool valid,
                                          float& m, float& l, float (&acc)[E]) {
  using S = DecodeShape<KV, HD, BS>;
  static_assert(S::ROUNDS == R && S::EPL == E, "tile shape");
  float sc[S::ROUNDS];
#pragma unroll
  for (int r = 0; r < S::ROUNDS; ++r) {
    float kf[S::EPL];
    Vec16<KV>::unpack(kb[r], kf);
    float d = 0.f;
#pragma unroll
    for (int e = 0; e < S::EPL; ++e) d = fmaf(qv[e], kf[e], d);
    d = group_sum<S::LPR>(d);
    const int t = tok0 + r * S::TPL;
    sc[r] = (valid && t < n) ? d : -INFINITY;
  }
  float mx = m;
#pragma unroll
  for (int r = 0; r < S::ROUNDS; ++r) mx = fmaxf(mx, sc[r]);
  const float alpha = fast_exp2(m - mx);
  l *= alpha;
#pragma unroll
  for (int e = 0; e < S::EPL; ++e) acc[e] *= alpha;
#pragma unroll
  for (int r = 0; r < S::ROUNDS; ++r) {
    const float p = fast_exp2(sc[r] - mx);
    l += p;
    float vf[S::EPL];
    Vec16<KV>::unpack(vb[r], vf);
#pragma unroll
    for (int e = 0; e < S::EPL; ++e) acc[e] = fmaf(p, vf[e], acc[e]);
  }
  m = mx;
}

// Stream `cnt` tiles through the online softmax with DEPTH tiles in flight ahead of the one being
// folded. Tile i of this call is page-table entry `ids` lane i. The steady-state loop issues its
// loads unconditionally (so the compiler's wait counts are exact and loads stay in flight across
// iterations); the last tiles drain in a peeled, guarded tail.
template <typename KV, int HD, int BS, int DEPTH, bool NT, int R, int E>
__device__ __forceinline__ void stream_tiles(int cnt, int ids, int tok_base, int tok_step, const KV* kpool,
                                             const KV* vpool, int64_t blk_stride, int64_t head_off,
                                             int64_t nblk, int lane, const float (&qv)[E], int n, float& m,
                                             float& l, float (&acc)[E]) {
  constexpr int S = DEPTH + 1;  // register slots
  u32x4 kb[S][R], vb[S][R];
  bool ok[S];
  auto issue = [&](int slot_unused, int i, u32x4 (&k)[R], u32x4 (&v)[R], bool& okk) {
    (void)slot_unused;
    const int blk = __builtin_amdgcn_readlane(ids, i);
    okk = blk >= 0 && blk < nblk;
    load_tile<NT, KV, R>(k, v, kpool, vpool, (okk ? blk : 0) * blk_stride + head_off, lane);
  };
  auto fold = [&](int i, const u32x4 (&k)[R], const u32x4 (&v)[R], bool okk) {
    fold_tile<KV, HD, BS>(k, v, qv, tok_base + i * tok_step, n, okk, m, l, acc);
  };
  if (cnt <= DEPTH) {
    for (int i = 0; i < cnt; ++i) {
      issue(0, i, kb[0], vb[0], ok[0]);
      fold(i, kb[0], vb[0], ok[0]);
    }
    return;
  }
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) issue(d, d, kb[d], vb[d], ok[d]);
  int i = 0;
  for (; i + DEPTH + S - 1 < cnt; i += S) {
#pragma unroll
    for (int k = 0; k < S; ++k) {
      issue((k + DEPTH) % S, i + k + DEPTH, kb[(k + DEPTH) % S], vb[(k + DEPTH) % S], ok[(k + DEPTH) % S]);
      fold(i + k, kb[k], vb[k], ok[k]);
    }
  }
  // Drain: at most S + DEPTH - 1 tiles remain; i % S == 0 here.
#pragma unroll
  for (int k = 0; k < S + DEPTH - 1; ++k) {
    if (i + k < cnt) {
      if (i + k + DEPTH < cnt)
        issue((k + DEPTH) % S, i + k + DEPTH, kb[(k + DEPTH) % S], vb[(k + DEPTH) % S], ok[(k + DEPTH) % S]);
      fold(i + k, kb[k % S], vb[k % S], ok[k % S]);
    }
  }
}

template <typename IO, bool COH>
__device__ __forceinline__ void merge_pair(const AttnArgs& a, int bh, int nact, int lane);

template <typename KV, typename IO, int HD, int NW>
__global__ __launch_bounds__(NW * kWave) void decode_fast_kernel(const AttnArgs a) {
  constexpr int BS = 16;
  using S = DecodeShape<KV, HD, BS>;
  constexpr int EPL = S::EPL, LPR = S::LPR, R = S::ROUNDS;

  __shared__ float sm_acc[NW][HD];
  __shared__ float sm_m[NW];
  __shared__ float sm_l[NW];

  const int lane = threadIdx.x & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  // The argument block spans three 64-byte lines. Left alone, the compiler loads the sizes the
  // work-unit arithmetic needs, waits, and loads the lines with the pointers afterwards: a second
  // dependent round trip before the first global load. The sizes pass through this statement
  // together with the other prologue arguments, so all argument loads go out at once.
  int nsplit = a.num_splits, nH = a.H, nB = a.B;
  asm volatile("" : "+s"(nsplit), "+s"(nH), "+s"(nB)
               : "s"(a.q), "s"(a.q_sb), "s"(a.q_sh), "s"(a.page_table), "s"(a.pt_stride), "s"(a.max_pages),
                 "s"(a.seq_lens), "s"(a.cur_lens), "s"(a.order), "s"(a.k_pool), "s"(a.v_pool), "s"(a.split_blocks));
  const int units = nH * nsplit;  // workgroups per request
  int bi, u;
#if PA_DECODE_XCD
  // Keep all workgroups of a request on one die: workgroup x runs on die x % kXcds, so request
  // slot bi takes the workgroups with x % kXcds == bi % kXcds. The grid is padded to a multiple
  // of kXcds requests.
  {
    const int x = blockIdx.x;
    const int die = x % kXcds;
    const int slot = x / kXcds;
    bi = (slot / units) * kXcds + die;
    u = slot % units;
    if (bi >= nB) return;
  }
#else
  bi = blockIdx.x / units;
  u = blockIdx.x % units;
#endif
  // Heads innermost: a request's workgroups run split by split, all heads of a split next to each
  // other, so workgroups dispatched together read the same block range of adjacent heads (a
  // block's heads are contiguous in the pool). Against splits innermost (graph replay, MI355X):
  // 8 requests x 8 heads x 64 fp32 at 128-1024 tokens 7.26-7.30 -> 6.93-6.96 us per layer; 1, 2
  // and 4 requests x 32 heads x 128 bf16 at 8k 28.1 -> 25.3, 49.8 -> 47.0 and 90.4 -> 87.0 us;
  // 1 at 32k 94.3 -> 90.5 us.
  const int split = u / nH;
  const int h = u % nH;
  const int b = a.order ? a.order[bi] : bi;

  // The first chunk of this wave's page-table entries (block jb0 + w + lane * NW) does not depend
  // on the request's length: load it now, clamped into the row, so that it travels with the
  // length loads instead of after them (one dependent memory round trip less before the first
  // KV tile). Entries past the request's blocks are discarded below.
  const int32_t* pt = a.page_table + (int64_t)b * a.pt_stride;
  const int jb0 = nsplit > 1 ? split * a.split_blocks : 0;
  int ids0 = -1;
  if (a.max_pages > 0) {
    const int idx = jb0 + w + lane * NW;
    ids0 = pt[idx < a.max_pages ? idx : a.max_pages - 1];
  }

  const int L = a.seq_lens[b];
  const int C = a.cur_lens[b];
  // q is loaded before the inactive-split return below (a branch the loads could not be moved
  // across), so it travels with the page-table and length loads.
  const int r = lane % LPR;
  const int g = lane / LPR;
  float qv[EPL];
  {
    const IO* qp = static_cast<const IO*>(a.q) + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh + r * EPL;
#pragma unroll
    for (int e = 0; e < EPL; ++e) qv[e] = Elem<IO>::load(qp + e) * a.scale_log2;
  }
  const int n = valid_keys(L, C, 0);
  int nb = (n + BS - 1) / BS;
  nb = nb < a.max_pages ? nb : a.max_pages;
  int jb = 0, je = nb, nact = 1;
  if (nsplit > 1) {
    nact = nb > 0 ? (nb + a.split_blocks - 1) / a.split_blocks : 1;
    if (split >= nact) return;  // uniform over the workgroup, before any barrier
    jb = split * a.split_blocks;
    je = jb + a.split_blocks < nb ? jb + a.split_blocks : nb;
  }


  float m = kNegBig, l = 0.f;
  float acc[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) acc[e] = 0.f;

  const KV* kpool = static_cast<const KV*>(a.k_pool);
  const KV* vpool = static_cast<const KV*>(a.v_pool);
  const int64_t tile_elems = (int64_t)BS * HD;
  const int64_t head_off = (int64_t)h * tile_elems;
  const int64_t blk_stride = (int64_t)a.H * tile_elems;

  // This wave's blocks: j = jb + w + k*NW for k < mine, in chunks of one page-table entry per lane.
  const int span = je - jb;
  const int mine = span > w ? (span - w + NW - 1) / NW : 0;
  for (int c0 = 0; c0 < mine; c0 += kWave) {
    const int cnt = (mine - c0) < kWave ? (mine - c0) : kWave;
    int ids = -1;
    if (lane < cnt) ids = c0 == 0 ? ids0 : pt[jb + w + (c0 + lane) * NW];
    stream_tiles<KV, HD, BS, PA_DECODE_DEPTH, PA_DECODE_NT != 0, R>(
        cnt, ids, (jb + w + c0 * NW) * BS + g, NW * BS, kpool, vpool, blk_stride, head_off, a.num_blocks, lane,
        qv, n, m, l, acc);
  }

  // Merge the TPL lane groups of this wave (lanes with equal r hold the same head_dim slice).
#pragma unroll
  for (int off = LPR; off < kWave; off <<= 1) {
    const float mo = __shfl_xor(m, off);
    const float lo = __shfl_xor(l, off);
    const float M = fmaxf(m, mo);
    const float sa = fast_exp2(m - M), sb = fast_exp2(mo - M);
    l = l * sa + lo * sb;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[e] = acc[e] * sa + __shfl_xor(acc[e], off) * sb;
    m = M;
  }
  if (g == 0) {
#pragma unroll
    for (int e = 0; e < EPL; ++e) sm_acc[w][r * EPL + e] = acc[e];
  }
  if (lane == 0) {
    sm_m[w] = m;
    sm_l[w] = l;
  }
  __syncthreads();

  float M = kNegBig;
#pragma unroll
  for (int ww = 0; ww < NW; ++ww) M = fmaxf(M, sm_m[ww]);
  for (int d = threadIdx.x; d < HD; d += NW * kWave) {
    float lsum = 0.f, A = 0.f;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) {
      const float f = fast_exp2(sm_m[ww] - M);
      lsum = fmaf(sm_l[ww], f, lsum);
      A = fmaf(sm_acc[ww][d], f, A);
    }
    if (nact == 1) {
      IO* op = static_cast<IO*>(a.out) + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh;
      Elem<IO>::store(op + d, lsum > 0.f ? A / lsum : 0.f);
    } else {
      float* rec = a.ws + (((int64_t)b * a.H + h) * nsplit + split) * (HD + 2);
      if (a.counters != nullptr) {  // same-launch merge: device-scope stores
        if (d == 0) {
          __hip_atomic_store(rec, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(rec + 1, lsum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __hip_atomic_store(rec + 2 + d, A, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      } else {
        if (d == 0) {
          rec[0] = M;
          rec[1] = lsum;
        }
        rec[2 + d] = A;
      }
    }
  }
  // Same-launch merge: once every wavefront's record stores have completed (at device scope),
  // one thread counts this split in; the split that arrives last resets the counter and merges
  // all records with device-scope loads.
  if (nact > 1 && a.counters != nullptr) {
    __shared__ int sm_last;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
      int32_t* cnt = a.counters + (int64_t)b * a.H + h;
      const int last = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nact - 1;
      if (last) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      sm_last = last;
    }
    __syncthreads();
    if (sm_last && threadIdx.x < kWave) merge_pair<IO, true>(a, b * a.H + h, nact, threadIdx.x);
  }
}

// Merge the partial records (m, l, acc[HD]) of each (request, head) written by its active splits
// (the number a split computes from the request's length): one wavefront per pair. The loads are
// spread over the lanes and issued together: lane s reads split s's (m, l) for the maximum and
// the denominator, and each lane's head_dim element is summed over the splits with the weights
// broadcast from the lane that computed them, eight independent loads at a time (a loop over the
// splits with one dependent load chain per split is several times slower).
// A record word: a plain load, or (COH) a device-scope load that sees the other splits' stores
// of this launch.
template <bool COH>
__device__ __forceinline__ float rec_load(const float* p) {
  if constexpr (COH) return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return *p;
}

template <typename IO, bool COH>
__device__ __forceinline__ void merge_pair(const AttnArgs& a, int bh, int nact, int lane) {
  const int b = bh / a.H, h = bh % a.H;
  const int HD = a.head_dim;
  const int64_t R = HD + 2;
  const float* base = a.ws + (int64_t)bh * a.num_splits * R;
  IO* op = static_cast<IO*>(a.out) + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh;
  if (nact <= 8 && HD <= 2 * kWave) {
    // At most 8 splits and two head_dim elements per lane: every word this lane needs (its
    // elements from every split and, on lane s < nact, split s's m and l) in one batch of loads
    // issued before any of them is used, so the merge waits for memory once. Indices past the
    // last split read its record again and get weight 0.
    const int d0 = lane < HD ? lane : HD - 1, d1 = lane + kWave < HD ? lane + kWave : HD - 1;
    const int sl = lane < nact ? lane : nact - 1;
    float x0[8], x1[8];
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) x0[jj] = rec_load<COH>(base + (jj < nact ? jj : nact - 1) * R + 2 + d0);
    if (HD > kWave) {
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) x1[jj] = rec_load<COH>(base + (jj < nact ? jj : nact - 1) * R + 2 + d1);
    }
    const float mr = rec_load<COH>(base + sl * R), lr = rec_load<COH>(base + sl * R + 1);
    const float m0 = lane < nact ? mr : kNegBig;
    const float M = wave_max(m0);
    const float f0 = lane < nact ? fast_exp2(m0 - M) : 0.f;  // weight of split `lane`
    const float lsum = wave_sum(lane < nact ? lr * f0 : 0.f);
    const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
    float A0 = 0.f, A1 = 0.f;
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      const float f = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, f0), jj));
      A0 = fmaf(x0[jj], f, A0);
      if (HD > kWave) A1 = fmaf(x1[jj], f, A1);
    }
    if (lane < HD) Elem<IO>::store(op + lane, A0 * inv);
    if (lane + kWave < HD) Elem<IO>::store(op + lane + kWave, A1 * inv);
    return;
  }
  // Lane s holds split s's (m, l) for the first 64 splits; more splits are read in further passes.
  float m0 = kNegBig, l0 = 0.f;
  if (lane < nact) {
    m0 = rec_load<COH>(base + lane * R);
    l0 = rec_load<COH>(base + lane * R + 1);
  }
  float M = m0;
  for (int s = lane + kWave; s < nact; s += kWave) M = fmaxf(M, rec_load<COH>(base + s * R));
  M = wave_max(M);
  const float f0 = lane < nact ? fast_exp2(m0 - M) : 0.f;  // weight of split `lane`, 0 past the splits
  float lsum = l0 * f0;
  for (int s = lane + kWave; s < nact; s += kWave) lsum = fmaf(rec_load<COH>(base + s * R + 1), fast_exp2(rec_load<COH>(base + s * R) - M), lsum);
  lsum = wave_sum(lsum);
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
  for (int d = lane; d - lane < HD; d += kWave) {
    const int dd = d < HD ? d : HD - 1;  // every lane takes part in the broadcasts
    float A = 0.f;
    for (int s0 = 0; s0 < nact; s0 += kWave) {
      const int n = nact - s0 < kWave ? nact - s0 : kWave;
      const float f = s0 == 0 ? f0 : (lane < n ? fast_exp2(rec_load<COH>(base + (s0 + lane) * R) - M) : 0.f);
      const float* rec = base + s0 * R + 2 + dd;
      // 8 loads in flight: indices past the last split are clamped to it (a valid record) and
      // get weight 0 (lane j0 + jj <= 63 since j0 <= n - 1 rounded down to a multiple of 8).
      for (int j0 = 0; j0 < n; j0 += 8) {
        float x[8];
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) x[jj] = rec_load<COH>(rec + (j0 + jj < n ? j0 + jj : n - 1) * R);
#pragma unroll
        for (int jj = 0; jj < 8; ++jj)
          A = fmaf(x[jj], __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, f), j0 + jj)), A);
      }
    }
    if (d < HD) Elem<IO>::store(op + d, A * inv);
  }
}

template <typename IO>
__global__ __launch_bounds__(kWave) void decode_merge_kernel(const AttnArgs a) {
  const int bh = blockIdx.x;
  const int b = bh / a.H;
  int nb = (valid_keys(a.seq_lens[b], a.cur_lens[b], 0) + 15) / 16;
  nb = nb < a.max_pages ? nb : a.max_pages;
  const int nact = nb > 0 ? (nb + a.split_blocks - 1) / a.split_blocks : 1;
  if (nact == 1) return;  // the split wrote the output itself
  merge_pair<IO, false>(a, bh, nact, threadIdx.x);
}

// ---------------------------------------------------------------------------------------------
// Generic kernel: one wavefront per (request, head, query row); lanes own head_dim elements and
// the KV positions are walked one at a time. Serves any block_size and head_dim <= 512, decode
// or prefill.
// ---------------------------------------------------------------------------------------------
constexpr int kGenericMaxHd = 512;

template <typename KV, typename IO>
__global__ __launch_bounds__(kWave) void attention_generic_kernel(const AttnArgs a) {
  constexpr int ND = kGenericMaxHd / kWave;
  const int lane = threadIdx.x;
  const int unit = blockIdx.x;
  const int i = unit % a.T;
  const int bh = unit / a.T;
  const int h = bh % a.H;
  const int b = bh / a.H;
  const int HD = a.head_dim, BS = a.block_size;

  const int L = a.seq_lens[b];
  const int C = a.cur_lens[b];
  const int n = valid_keys(L, C, i);

  const IO* qp = static_cast<const IO*>(a.q) + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh + (int64_t)i * a.q_st;
  float qv[ND], acc[ND];
#pragma unroll
  for (int k = 0; k < ND; ++k) {
    const int d = lane + k * kWave;
    qv[k] = d < HD ? Elem<IO>::load(qp + d) * a.scale_log2 : 0.f;
    acc[k] = 0.f;
  }
  float m = kNegBig, l = 0.f;
  const KV* kpool = static_cast<const KV*>(a.k_pool);
  const KV* vpool = static_cast<const KV*>(a.v_pool);
  const int32_t* pt = a.page_table + (int64_t)b * a.pt_stride;

  for (int t = 0; t < n; ++t) {
    const int p = t / BS;
    if (p >= a.max_pages) break;
    const int blk = pt[p];
    if (blk < 0 || blk >= a.num_blocks) continue;
    const int64_t row = (((int64_t)blk * a.H + h) * BS + (t % BS)) * HD;
    float dot = 0.f;
#pragma unroll
    for (int k = 0; k < ND; ++k) {
      const int d = lane + k * kWave;
      if (d < HD) dot = fmaf(qv[k], Elem<KV>::load(kpool + row + d), dot);
    }
    dot = wave_sum(dot);
    const float mx = fmaxf(m, dot);
    const float alpha = fast_exp2(m - mx);
    const float pe = fast_exp2(dot - mx);
    l = l * alpha + pe;
#pragma unroll
    for (int k = 0; k < ND; ++k) {
      const int d = lane + k * kWave;
      const float v = d < HD ? Elem<KV>::load(vpool + row + d) : 0.f;
      acc[k] = fmaf(pe, v, acc[k] * alpha);
    }
    m = mx;
  }
  IO* op = static_cast<IO*>(a.out) + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh + (int64_t)i * a.o_st;
#pragma unroll
  for (int k = 0; k < ND; ++k) {
    const int d = lane + k * kWave;
    if (d < HD) Elem<IO>::store(op + d, l > 0.f ? acc[k] / l : 0.f);
  }
}

int launch_generic_attention(const AttnArgs& a, int io_dtype, int kv_dtype, hipStream_t stream) {
  if (a.head_dim > kGenericMaxHd)
    PA_FAIL(PA_ERR_UNSUPPORTED, "head_dim %d exceeds the generic kernel limit %d", a.head_dim, kGenericMaxHd);
  const int64_t units = (int64_t)a.B * a.H * a.T;
  if (units == 0) return PA_OK;
  if (units > 0x7fffffffLL) PA_FAIL(PA_ERR_INVALID_ARGUMENT, "too many (request, head, row) units");
  const dim3 grid((unsigned)units), block(kWave);
  if (io_dtype == PA_DTYPE_F32 && kv_dtype == PA_DTYPE_F32)
    attention_generic_kernel<float, float><<<grid, block, 0, stream>>>(a);
  else if (io_dtype == PA_DTYPE_F32 && kv_dtype == PA_DTYPE_BF16)
    attention_generic_kernel<uint16_t, float><<<grid, block, 0, stream>>>(a);
  else if (io_dtype == PA_DTYPE_BF16 && kv_dtype == PA_DTYPE_F32)
    attention_generic_kernel<float, uint16_t><<<grid, block, 0, stream>>>(a);
  else
    attention_generic_kernel<uint16_t, uint16_t><<<grid, block, 0, stream>>>(a);
  PA_CHECK_LAUNCH("generic attention kernel");
  return PA_OK;
}

// ---------------------------------------------------------------------------------------------
// Fast-path dispatch
// ---------------------------------------------------------------------------------------------
constexpr int kDecodeWaves = PA_DECODE_WAVES;

template <typename KV, typename IO, int HD>
static void launch_decode_fast(const AttnArgs& a, hipStream_t stream) {
  int64_t reqs = a.B;
#if PA_DECODE_XCD
  reqs = (reqs + kXcds - 1) / kXcds * kXcds;
#endif
  const dim3 grid((unsigned)(reqs * a.H * a.num_splits)), block(kDecodeWaves * kWave);
  decode_fast_kernel<KV, IO, HD, kDecodeWaves><<<grid, block, 0, stream>>>(a);
}

template <typename IO>
static bool dispatch_decode_fast_io(const AttnArgs& a, int kv_dtype, hipStream_t stream) {
  if (kv_dtype == PA_DTYPE_F32) {
    if (a.head_dim == 64) { launch_decode_fast<float, IO, 64>(a, stream); return true; }
    if (a.head_dim == 128) { launch_decode_fast<float, IO, 128>(a, stream); return true; }
  } else {
    if (a.head_dim == 64) { launch_decode_fast<uint16_t, IO, 64>(a, stream); return true; }
    if (a.head_dim == 128) { launch_decode_fast<uint16_t, IO, 128>(a, stream); return true; }
  }
  return false;
}

static int num_splits_for(int32_t max_pages, int32_t split_blocks) {
  if (split_blocks <= 0 || max_pages <= split_blocks) return 1;
  return (int)((max_pages + split_blocks - 1) / split_blocks);
}

}  // namespace pa

using namespace pa;

// Split workspace layout: arrival counters (one int32 per (request, head), at most
// kDecodeCounterBytes / 4 pairs) at the start, zero between calls, then the split records. The
// counters region has one fixed size whatever the call's shape, so calls of any shapes can share
// a workspace and always find their counters at zero.
constexpr size_t kDecodeCounterBytes = PA_DECODE_COUNTER_BYTES;
// Splits per (request, head) up to which the last split to finish merges the records in the same
// launch; more splits are merged by a second launch (its merge reads them faster than one
// workgroup's device-scope loads).
constexpr int kSameLaunchMaxSplits = 8;

extern "C" size_t pa_decode_workspace_size(int32_t batch, int32_t num_heads, int32_t head_dim,
                                           int32_t max_pages, int32_t split_blocks) {
  const int s = num_splits_for(max_pages, split_blocks);
  if (s <= 1 || batch <= 0 || num_heads <= 0 || head_dim <= 0) return 0;
  return kDecodeCounterBytes + (size_t)batch * num_heads * s * (head_dim + 2) * sizeof(float);
}

// Shared body of pa_decode and pa_decode_noalloc. `ws_limit_is_scratch` only changes the error
// reported when the split records do not fit: the caller's workspace is too small (pa_decode) or
// the request exceeds the fixed scratch array (pa_decode_noalloc).
static int decode_entry(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                        void* out, int64_t out_stride_b, int64_t out_stride_h, int io_dtype,
                        const void* k_pool, const void* v_pool, int kv_dtype, int64_t num_blocks,
                        const int32_t* page_table, int64_t pt_stride, int32_t max_pages,
                        const int32_t* seq_lens, const int32_t* cur_lens, const int32_t* order,
                        int32_t batch, int32_t num_heads, int32_t head_dim, int32_t block_size,
                        float scale, int32_t split_blocks,
                        void* workspace, size_t workspace_bytes, bool ws_limit_is_scratch,
                        void* stream_) {
  PA_CHECK_ARG(batch >= 0 && num_heads > 0 && head_dim > 0 && block_size > 0,
               "bad sizes: batch=%d heads=%d head_dim=%d block_size=%d", batch, num_heads, head_dim,
               block_size);
  PA_CHECK_ARG(io_dtype == PA_DTYPE_F32 || io_dtype == PA_DTYPE_BF16, "bad io dtype %d", io_dtype);
  PA_CHECK_ARG(kv_dtype == PA_DTYPE_F32 || kv_dtype == PA_DTYPE_BF16, "bad kv dtype %d", kv_dtype);
  if (batch == 0) return PA_OK;
  PA_CHECK_ARG(q && out && seq_lens && cur_lens, "null q/out/seq_lens/cur_lens");
  PA_CHECK_ARG(max_pages >= 0, "max_pages must be >= 0");
  if (max_pages > 0) {
    PA_CHECK_ARG(page_table != nullptr && pt_stride >= max_pages, "page table missing or stride < max_pages");
    PA_CHECK_ARG(k_pool && v_pool && num_blocks > 0, "KV pool missing or empty");
  }
  hipStream_t stream = static_cast<hipStream_t>(stream_);

  AttnArgs a{};
  a.q = q; a.q_sb = q_stride_b; a.q_sh = q_stride_h; a.q_st = 0;
  a.out = out; a.o_sb = out_stride_b; a.o_sh = out_stride_h; a.o_st = 0;
  a.k_pool = k_pool; a.v_pool = v_pool; a.num_blocks = num_blocks;
  a.page_table = page_table; a.pt_stride = pt_stride; a.max_pages = max_pages;
  a.seq_lens = seq_lens; a.cur_lens = cur_lens; a.order = order;
  a.B = batch; a.H = num_heads; a.T = 1; a.head_dim = head_dim; a.block_size = block_size;
  a.scale_log2 = scale * kLog2e;
  a.num_splits = 1; a.split_blocks = 0; a.ws = nullptr;

  const bool fast = block_size == 16 && (head_dim == 64 || head_dim == 128);
  if (!fast) return launch_generic_attention(a, io_dtype, kv_dtype, stream);

  const int nsplit = num_splits_for(max_pages, split_blocks);
  if (nsplit > 1) {
    const size_t need = pa_decode_workspace_size(batch, num_heads, head_dim, max_pages, split_blocks);
    if (ws_limit_is_scratch && need > workspace_bytes)
      PA_FAIL(PA_ERR_INVALID_ARGUMENT,
              "pa_decode_noalloc: %d x %d heads x %d splits of head_dim %d need %zu bytes of split "
              "records, above the fixed scratch of %zu bytes (use pa_decode with a workspace, or a "
              "larger split_blocks)", batch, num_heads, nsplit, head_dim, need, workspace_bytes);
    if (workspace == nullptr || workspace_bytes < need)
      PA_FAIL(PA_ERR_WORKSPACE, "decode workspace too small: need %zu bytes, have %zu", need, workspace_bytes);
    a.num_splits = nsplit;
    a.split_blocks = split_blocks;
    a.ws = reinterpret_cast<float*>(static_cast<char*>(workspace) + kDecodeCounterBytes);
    if (nsplit <= kSameLaunchMaxSplits && (size_t)batch * num_heads * sizeof(int32_t) <= kDecodeCounterBytes)
      a.counters = static_cast<int32_t*>(workspace);
  }
  if (((int64_t)batch + kXcds) * num_heads * nsplit > 0x7fffffffLL)
    PA_FAIL(PA_ERR_INVALID_ARGUMENT, "grid too large");

  const bool ok = io_dtype == PA_DTYPE_F32 ? dispatch_decode_fast_io<float>(a, kv_dtype, stream)
                                           : dispatch_decode_fast_io<uint16_t>(a, kv_dtype, stream);
  if (!ok) PA_FAIL(PA_ERR_UNSUPPORTED, "no decode kernel for head_dim %d", head_dim);
  PA_CHECK_LAUNCH("decode kernel");
  if (nsplit > 1 && a.counters == nullptr) {
    const dim3 grid((unsigned)((int64_t)batch * num_heads)), block(kWave);
    if (io_dtype == PA_DTYPE_F32)
      decode_merge_kernel<float><<<grid, block, 0, stream>>>(a);
    else
      decode_merge_kernel<uint16_t><<<grid, block, 0, stream>>>(a);
    PA_CHECK_LAUNCH("decode merge kernel");
  }
  return PA_OK;
}

extern "C" int pa_decode(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                         void* out, int64_t out_stride_b, int64_t out_stride_h, int io_dtype,
                         const void* k_pool, const void* v_pool, int kv_dtype, int64_t num_blocks,
                         const int32_t* page_table, int64_t pt_stride, int32_t max_pages,
                         const int32_t* seq_lens, const int32_t* cur_lens, const int32_t* order,
                         int32_t batch, int32_t num_heads, int32_t head_dim, int32_t block_size,
                         float scale, int32_t split_blocks,
                         void* workspace, size_t workspace_bytes, void* stream) {
  pa_host::clear_error();
  return decode_entry(q, q_stride_b, q_stride_h, out, out_stride_b, out_stride_h, io_dtype, k_pool, v_pool,
                      kv_dtype, num_blocks, page_table, pt_stride, max_pages, seq_lens, cur_lens, order, batch,
                      num_heads, head_dim, block_size, scale, split_blocks, workspace, workspace_bytes, false,
                      stream);
}

// ---------------------------------------------------------------------------------------------
// Allocation-free decode: the split-K records live in a fixed device array instead of a caller
// workspace. Each device holds its own copy of `scratch` (in the library's code object, for the
// life of the process); host code never passes the array's name to a kernel, only the device
// address hipGetSymbolAddress returns for the current device, looked up once per device.
// ---------------------------------------------------------------------------------------------
constexpr size_t kNoAllocScratchBytes = PA_DECODE_NOALLOC_SCRATCH_BYTES;  // 16 MiB per device
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxScratchDevices] = {nullptr};

// The current device's address of `scratch`, or nullptr (error set) when it cannot be resolved.
float* scratch_for_current_device() {
  int dev = -1;
  const hipError_t ge = hipGetDevice(&dev);
  if (ge != hipSuccess || dev < 0 || dev >= kMaxScratchDevices) {
    pa_host::set_error("pa_decode_noalloc: no usable current device (%s, device %d)", hipGetErrorString(ge), dev);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      pa_host::set_error("pa_decode_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                         hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  return g_scratch_ptr[dev];
}
}  // namespace

extern "C" int pa_decode_noalloc(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                 void* out, int64_t out_stride_b, int64_t out_stride_h, int io_dtype,
                                 const void* k_pool, const void* v_pool, int kv_dtype, int64_t num_blocks,
                                 const int32_t* page_table, int64_t pt_stride, int32_t max_pages,
                                 const int32_t* seq_lens, const int32_t* cur_lens, const int32_t* order,
                                 int32_t batch, int32_t num_heads, int32_t head_dim, int32_t block_size,
                                 float scale, int32_t split_blocks, void* stream) {
  pa_host::clear_error();
  // Only a split launch touches the scratch; resolve it (first call on a device) only then.
  const bool fast = block_size == 16 && (head_dim == 64 || head_dim == 128);
  float* ws = nullptr;
  if (fast && batch > 0 && num_heads > 0 && head_dim > 0 && num_splits_for(max_pages, split_blocks) > 1) {
    ws = scratch_for_current_device();
    if (ws == nullptr) return PA_ERR_HIP;
  }
  return decode_entry(q, q_stride_b, q_stride_h, out, out_stride_b, out_stride_h, io_dtype, k_pool, v_pool,
                      kv_dtype, num_blocks, page_table, pt_stride, max_pages, seq_lens, cur_lens, order, batch,
                      num_heads, head_dim, block_size, scale, split_blocks, ws, kNoAllocScratchBytes, true,
                      stream);
}
