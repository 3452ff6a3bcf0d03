// Wide-tile chunked prefill attention for bf16 KV pools on gfx950 (long chunks over long
// contexts, where the 16-row kernel would re-read every KV block once per 16 query rows).
//
// One workgroup of 4 wavefronts per (request, head, tile of 128 query rows); wavefront w owns
// rows 32w..32w+31 of the tile. The workgroup walks the KV blocks in steps of 32 keys (head_dim
// 128) or 64 keys (head_dim 64). Each step's K and V tiles go from HBM straight into LDS with
// LDS-direct loads (global_load_lds_dwordx4, no staging registers), 2 (head_dim 128) or 1
// (head_dim 64) steps ahead of their use in a 3- or 2-stage ring; all four wavefronts read them
// there.
//
// Per step and wavefront, with v_mfma_f32_32x32x16_bf16 (fp32 accumulation):
//   S^T = K Q^T      32 keys x 32 queries; A = K rows from LDS, B = the wavefront's q (bf16,
//                    pre-scaled into the log2 domain) held in registers for the whole walk;
//   online softmax   lane (G2, c) = (lane / 32, lane % 32) holds query c's scores for keys
//                    8j + 4*G2 + r (j, r < 4), so the row max / sum are 16 registers plus one
//                    v_permlane32_swap;
//   O^T += V^T P^T   two MFMAs (mm = 0, 1) per 32-row output tile and 32 keys; the B operand is
//                    the softmax weights as held (registers 8mm..8mm+7 = keys 16mm + 8jj + 4*G2
//                    + r at k slot (G2, 4jj + r)). Output tile d row R is head_dim index 32d + R.
//                    The A operand (V^T, row = head_dim) is read from the key-major V tile with
//                    two ds_read_b64_tr_b16 (LDS transposing reads): no transposition in
//                    registers.
// LDS tiles are unpadded key rows; their 16-byte chunks are XOR-swizzled per row so that both
// operand reads use every LDS bank once per pass.
// The QK^T contraction slot (G2, e) of MFMA s is head_dim index G2*HD/2 + 8s + e. A and B of each
// product use the same slot map, so results do not depend on the hardware's k ordering.
// Rounding matches the 16-row bf16 kernel: q*scale and the softmax weights are rounded to bf16
// (nearest even) for the products, scores and accumulators stay fp32. The running max is updated
// lazily (see kRescaleSlack) and interior steps skip the causal/length mask.
//
// The file also holds the split-step kernel (prefill_split_kernel, below): the same bf16 step on
// 32-row tiles for short chunks, with a tile's steps split over 8 wavefronts instead of its rows.
#include <string.h>

#include "pa_attention.h"

namespace pa {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Lazy rescaling threshold (log2 units): the running max only moves when a step's max exceeds it
// by more than this, so softmax weights stay <= 2^8 and the accumulators are rescaled only in
// the few steps where the max jumps.
constexpr float kRescaleSlack = 8.f;

constexpr int kWideWaves = 4;
constexpr int kWideRows = kWideWaves * 32;  // query rows per workgroup

// Workgroup -> (request, head) pair and query tile. The ntiles workgroups of one pair read the
// same K/V blocks, and workgroup x runs on die x % kXcds (each die has its own L2), so they take
// indices congruent modulo kXcds: groups of kXcds pairs own kXcds * ntiles consecutive indices,
// tile-major, heaviest (last) tile first. The last group may hold fewer pairs.
__device__ __forceinline__ void wide_unit(int x, int BH, int ntiles, int& bh, int& qt) {
  const int g = x / (kXcds * ntiles);
  const int r = x - g * kXcds * ntiles;
  const int rest = BH - g * kXcds;
  const int m = rest < kXcds ? rest : kXcds;
  const int t = r / m;
  bh = g * kXcds + (r - t * m);
  qt = ntiles - 1 - t;
}

// One LDS-direct load (global_load_lds_dwordx4): lane L reads 16 bytes at base + voff and writes
// them to LDS byte address lds + 16L (lds is the wavefront-uniform M0). Issued as inline
// assembly so that the compiler does not track it: it would otherwise wait for every such load
// before any LDS read, also for loads into stages that the read does not touch. The caller
// waits for these loads itself (s_waitcnt vmcnt) before the barrier that publishes their stage.
__device__ __forceinline__ void lds_direct_load16(const void* base, uint32_t voff, const void* lds) {
  const uint32_t m0 = (uint32_t)(size_t)(const __attribute__((address_space(3))) void*)lds;
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "{m0}"(m0));
}

// A 4-byte global load that has completed on return (load and s_waitcnt vmcnt(0) in one
// assembly block, untracked by the compiler like lds_direct_load16: its own wait for a tracked
// load would be placed before every later use of the register, draining the LDS-direct loads in
// flight each time).
__device__ __forceinline__ int load_now(const int32_t* p) {
  int v;
  asm volatile("global_load_dword %0, %1, off\n\ts_waitcnt vmcnt(0)" : "=v"(v) : "v"(p) : "memory");
  return v;
}

// Longest-first order: the (request, query tile) units sorted by descending work (the valid keys
// of the tile's last row; ties by unit index), heads innermost, so the longest tiles start first
// and the short ones fill the end of the grid (contexts of different lengths otherwise leave a
// tail of long tiles running alone). Every workgroup ranks the units itself, one per thread, using
// `lds` (NTH + 1 ints) as scratch. Returns false when there are more units than threads; the
// caller then keeps wide_unit's order. ROWS = query rows per tile, NTH = threads per workgroup.
template <int ROWS, int NTH>
__device__ __forceinline__ bool tile_lpt_unit(const AttnArgs& a, int ntiles, int* lds, int& bh, int& qt) {
  const int U = a.B * ntiles;
  if (U > NTH) return false;
  const int tid = threadIdx.x;
  int key = 0;
  if (tid < U) {
    const int b = tid / ntiles;
    const int t = tid - b * ntiles;
    const int last = t * ROWS + ROWS - 1 < a.T - 1 ? t * ROWS + ROWS - 1 : a.T - 1;
    key = valid_keys(a.seq_lens[b], a.cur_lens[b], last);
    lds[tid] = key;
  }
  __syncthreads();
  const int pos = blockIdx.x / a.H;
  if (tid < U) {
    int rank = 0;
    for (int u = 0; u < U; ++u) {
      const int k2 = lds[u];
      rank += (k2 > key) || (k2 == key && u < tid);
    }
    if (rank == pos) lds[NTH] = tid;
  }
  __syncthreads();
  const int unit = __builtin_amdgcn_readfirstlane(lds[NTH]);
  __syncthreads();  // the scratch is reused by the caller
  const int b = unit / ntiles;
  qt = unit - b * ntiles;
  bh = b * a.H + (blockIdx.x - pos * a.H);
  return true;
}
constexpr int kOrderMax = kWideWaves * kWave;
__device__ __forceinline__ bool wide_lpt_unit(const AttnArgs& a, int ntiles, int* lds, int& bh, int& qt) {
  return tile_lpt_unit<kWideRows, kOrderMax>(a, ntiles, lds, bh, qt);
}

// NSUB = 32-key sub-tiles per step: the per-step costs (barrier, mask test, max/sum exchange,
// lazy-rescale test) are paid once per NSUB * 32 keys. Head_dim 64 uses NSUB 2 with 2 stages
// (a third stage's LDS costs a workgroup per CU). Head_dim 128 takes one of two shapes by grid
// size (wide128_pair below).
#ifndef WIDE_NSUB64
#define WIDE_NSUB64 2
#endif
#ifndef WIDE_NST64
#define WIDE_NST64 2
#endif
constexpr int kWideNsub64 = WIDE_NSUB64;
// LDS stages of K and V tiles (2 or 3): loads are issued NST - 1 steps ahead of their use.
constexpr int kWideStages64 = WIDE_NST64;
// Head_dim 128, bf16 KV: NSUB 2 with 2 stages (174 registers, 64 KB of LDS: 2 workgroups per CU)
// when the grid fits in one round at 2 workgroups per CU, else NSUB 1 with 2 stages (154
// registers, 32 KB: 3 per CU, registers being the limit): the wider step pays only when no second
// round of workgroups needs the CU slots it holds.
static bool wide128_pair(int64_t units) { return units <= 2 * (int64_t)pa_host::device_cu_count(); }

// Balanced launch (BAL; bf16 KV at head_dim 128 with one 32-key sub-tile per step or at head_dim
// 64 with two, fp32 KV at head_dim 128 and 64 with 32-key steps; 2 stages): the grid
// is one to three workgroups per CU (no more than the CUs hold at once), and the KV steps of all tiles are
// dealt out evenly instead of one workgroup per tile. Die k (workgroups x = k mod 8) takes the
// (request, head) pairs with head = k mod 8, listed by request, then head; a pair's work is the
// step count of its last (longest) tile, at least 1. The die's workgroups form gangs of ntiles
// members (x = 8 (g ntiles + t) + k is member t of gang g); gang g takes the share
// [lo_g, lo_g+1) of the die's list (its W steps split over the NG gangs in proportion to
// share_weight, which favours the gangs dispatched first), and member t walks tile t of each
// pair in that share over the same key steps as its mates, so a pair's tiles still read each KV
// step at about the same time (from the die's L2). A tile whose steps fall into several
// gangs' shares is cut into pieces: each leaves an (m, l, O) record (two slots per workgroup: its
// share's first and last pair; pairs inside a share are never cut), and the piece that arrives
// last (per-tile arrival counter, reset to zero by that piece) merges them in gang order.
// Workspace: a.counters holds one arrival counter per (request, head, tile), zero between calls;
// a.ws the records, slot s of workgroup x at a.ws + (2 x + s) * kWideRecFloats<HD>. A wavefront's
// part is 1 + HD / 8 groups of 16 bytes per lane (17 at head_dim 128, 9 at 64), lane-minor (group
// j of lane L at float 4 (64 j + L), so each group is one coalesced 1 KB block): group 0 holds m
// and l, group 1 + 4d + q the accumulators oacc[d][4q .. 4q + 3].
template <int HD>
constexpr int kWideRecGroups = 1 + HD / 32 * 16 / 4;
// Share weight of the gangs whose workgroups are the s-th to reach their compute units (s = 0, 1, 2
// at three workgroups per CU). Measured on MI355X with equal shares (8 x 32 heads x 128, chunk
// 512 over 1.8-3.7k contexts): the first, second and third workgroup of each CU finished at 197,
// 207 and 218 us (medians), i.e. progressed at relative rates 1.10 : 1.05 : 1.
__device__ __forceinline__ int share_weight(int s) { return s < 2 ? 22 - s : 20; }

template <int HD>
constexpr int kWideRecFloats = kWideWaves * kWideRecGroups<HD> * kWave * 4;
static_assert(kWideRecGroups<128> == 17 && kWideRecGroups<64> == 9, "record groups");

typedef float f32x4 __attribute__((ext_vector_type(4)));
// Groups 0-8 and 9-16 of a record (p: the lane's group 0; groups 1 KB apart; a head_dim 64 record
// is groups 0-8 only), read with the
// device-scope coherence bit (sc1) that relaxed agent-scope atomic loads use, nine and eight
// loads in flight, each batch waited for inside its assembly block. (As atomic loads the compiler
// issues them one at a time, waiting for each: 66 memory round trips per record.)
__device__ __forceinline__ void load_record_lo(const float* p, f32x4 (&v)[9]) {
  const float* p4 = p + 4 * 256;
  const float* p8 = p + 8 * 256;
  asm volatile(
      "global_load_dwordx4 %0, %9, off offset:-4096 sc1\n\t"
      "global_load_dwordx4 %1, %9, off offset:-3072 sc1\n\t"
      "global_load_dwordx4 %2, %9, off offset:-2048 sc1\n\t"
      "global_load_dwordx4 %3, %9, off offset:-1024 sc1\n\t"
      "global_load_dwordx4 %4, %9, off sc1\n\t"
      "global_load_dwordx4 %5, %9, off offset:1024 sc1\n\t"
      "global_load_dwordx4 %6, %9, off offset:2048 sc1\n\t"
      "global_load_dwordx4 %7, %9, off offset:3072 sc1\n\t"
      "global_load_dwordx4 %8, %10, off sc1\n\t"
      "s_waitcnt vmcnt(0)"
      : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]), "=&v"(v[6]),
        "=&v"(v[7]), "=&v"(v[8])
      : "v"(p4), "v"(p8)
      : "memory");
}
// One 16-byte record group store with the device-scope coherence bit (sc1) that relaxed
// agent-scope atomic stores use; the caller waits for its stores (s_waitcnt vmcnt(0)) before
// counting itself in.
__device__ __forceinline__ void store_record_group(float* p, f32x4 v) {
  asm volatile("global_store_dwordx4 %0, %1, off sc1" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void load_record_hi(const float* p, f32x4 (&v)[8]) {
  const float* p13 = p + 13 * 256;
  asm volatile(
      "global_load_dwordx4 %0, %8, off offset:-4096 sc1\n\t"
      "global_load_dwordx4 %1, %8, off offset:-3072 sc1\n\t"
      "global_load_dwordx4 %2, %8, off offset:-2048 sc1\n\t"
      "global_load_dwordx4 %3, %8, off offset:-1024 sc1\n\t"
      "global_load_dwordx4 %4, %8, off sc1\n\t"
      "global_load_dwordx4 %5, %8, off offset:1024 sc1\n\t"
      "global_load_dwordx4 %6, %8, off offset:2048 sc1\n\t"
      "global_load_dwordx4 %7, %8, off offset:3072 sc1\n\t"
      "s_waitcnt vmcnt(0)"
      : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]), "=&v"(v[6]),
        "=&v"(v[7])
      : "v"(p13)
      : "memory");
}

// The balanced launch (BAL) needs three workgroups per compute unit (its grid is the slots the
// CUs hold at once): at most 168 registers per lane.
template <typename IO, int HD, int NSUB, int NST, bool BAL>
__global__ __launch_bounds__(kWideWaves * kWave) __attribute__((amdgpu_waves_per_eu(BAL ? 3 : 1)))
void prefill_wide_kernel(const AttnArgs a) {
  constexpr int NW = kWideWaves;
  constexpr int KS = 32 * NSUB;          // keys per step
  constexpr int NBS = KS / 16;           // KV blocks per step
  constexpr int QH = HD / 2;             // head_dim values per lane in the QK^T operands
  constexpr int NQ = HD / 16;            // QK^T MFMAs per sub-tile (k = 16 each)
  constexpr int DU = HD / 32;            // output tiles of 32 head_dim rows
  constexpr int CPR = HD / 8;            // 16-byte chunks per key row
  constexpr int RPI = kWave / CPR;       // key rows per LDS-direct load instruction (1 KB)
  constexpr int NDMA = KS / (RPI * NW);  // such instructions per wavefront per K (or V) tile
  static_assert(NDMA >= 1 && NDMA * RPI * NW == KS && 16 % RPI == 0, "tile split");
  constexpr int RPB = 128 / HD;          // key rows per 256 bytes (one pass over the LDS banks)
  constexpr int TILE = KS * HD;          // elements per K (or V) tile

  static_assert(NST == 2 || NST == 3, "stages");
  static_assert(!BAL || (NST == 2 && NSUB == (HD == 128 ? 1 : 2)), "balanced launch shape");
  // Stage s: K tile at sbuf + 2 * s * TILE, V tile right after it (one array addressed through
  // per-stage pointers takes fewer registers than one array per tile).
  __shared__ __attribute__((aligned(16))) uint16_t sbuf[NST * 2 * TILE];

  const int lane = threadIdx.x & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int G2 = lane >> 5;
  const int c = lane & 31;
  uint16_t* const sk0 = sbuf;
  uint16_t* const sv0 = sbuf + TILE;
  uint16_t* const sk1 = sbuf + 2 * TILE;
  uint16_t* const sv1 = sbuf + 3 * TILE;
  uint16_t* const sk2 = sbuf + (NST > 2 ? 4 : 0) * TILE;
  uint16_t* const sv2 = sbuf + (NST > 2 ? 5 : 1) * TILE;

  const int ntiles = (a.T + kWideRows - 1) / kWideRows;
  // Steps of 32 * NSUB keys that tile qt of request b walks (the valid keys of its last row).
  auto tile_steps = [&](int L, int C, int rqt) {
    const int last = (rqt * kWideRows + kWideRows - 1) < (a.T - 1) ? (rqt * kWideRows + kWideRows - 1) : (a.T - 1);
    int nbb = (valid_keys(L, C, last) + 15) / 16;  // nondecreasing in the row
    nbb = nbb < a.max_pages ? nbb : a.max_pages;
    return (nbb + NBS - 1) / NBS;
  };
  int bh = 0, qt = 0;
  // BAL: this workgroup's share [lo, hi) of its die's pair list (see above), the pair it
  // has reached (request pb, head index hh: head k + 8 hh) and that pair's list position Sb and
  // work P per head.
  // The host keeps W below 2^31 / 64, so list positions fit in int.
  int k = 0, gang = 0, NG = 1, HP = 1, pb = 0, hh = 0, P = 1;
  int W = 1, lo = 0, hi = 0, Sb = 0;
  __shared__ int sm_last;                     // BAL: this piece arrived last
  __shared__ int sP[kWideWaves * kWave];      // BAL: pair work per request
  __shared__ int sS[kWideWaves * kWave];      // BAL: its prefix sums
  __shared__ int sCw[kWideWaves * kWave];     // BAL: prefix sums of the gangs' share weights
  __shared__ int sLo[kWideWaves * kWave];     // BAL: the gangs' shares: [sLo[g], sLo[g + 1])
  __shared__ int sL[kWideWaves * kWave];      // BAL: each request's seq_lens and cur_lens, read once
  __shared__ int sC[kWideWaves * kWave];
  // BAL: the gang whose share holds list position pos (the last g with sLo[g] <= pos).
  auto gang_of = [&](int pos) {
    int lg = 0, ug = NG - 1;
    while (lg < ug) {
      const int mid = (lg + ug + 1) / 2;
      if (__builtin_amdgcn_readfirstlane(sLo[mid]) <= pos) lg = mid;
      else ug = mid - 1;
    }
    return lg;
  };
  if constexpr (!BAL) {
    static_assert(sizeof(sbuf) >= (kOrderMax + 1) * sizeof(int), "order scratch");
    if (!wide_lpt_unit(a, ntiles, reinterpret_cast<int*>(sbuf), bh, qt)) wide_unit(blockIdx.x, a.B * a.H, ntiles, bh, qt);
  } else {
    k = blockIdx.x % kXcds;
    const int jx = blockIdx.x / kXcds;
    gang = jx / ntiles;
    qt = jx - gang * ntiles;
    NG = gridDim.x / (kXcds * ntiles);
    HP = a.H / kXcds;
    // S[r] = work of requests 0 .. r - 1 per head (at most 255 requests: one thread per entry).
    if (threadIdx.x < a.B) {
      const int L = a.seq_lens[threadIdx.x], C = a.cur_lens[threadIdx.x];
      sL[threadIdx.x] = L;
      sC[threadIdx.x] = C;
      const int p = tile_steps(L, C, ntiles - 1);
      sP[threadIdx.x] = p > 1 ? p : 1;
    }
    __syncthreads();
    if (threadIdx.x <= a.B) {
      int s = 0;
      for (int r = 0; r < (int)threadIdx.x; ++r) s += sP[r];
      sS[threadIdx.x] = s;
    }
    // Share weights: gang g's workgroups are the (g ntiles / die_cus)-th to reach their compute
    // units (the dispatcher deals a die's workgroups round-robin over its CUs), and the ones that
    // arrive later progress more slowly (the instruction arbiter favours older wavefronts), so
    // earlier gangs take proportionally more steps.
    if (threadIdx.x <= NG) {
      // share_weight(g ntiles / die_cus) summed over g < n: its value is share_weight(0) while
      // g ntiles < die_cus (g < n0), share_weight(1) while g ntiles < 2 die_cus (g < n1), then
      // share_weight(2). (Summed in a loop, this table took ~2.5 us of a 48 us launch at 32 gangs
      // per die; with it and the lengths kept in LDS: 4 x 32 heads x 128, 256-token chunks at two
      // workgroups per CU 50.0 -> 47.9 us, 1 x 8 heads x 64 over 32k 48.0 -> 45.4 us.)
      const int n = threadIdx.x;
      const int n0 = (a.die_cus + ntiles - 1) / ntiles, n1 = (2 * a.die_cus + ntiles - 1) / ntiles;
      const int c0 = n < n0 ? n : n0, c1 = n < n1 ? n : n1;
      sCw[threadIdx.x] = share_weight(0) * c0 + share_weight(1) * (c1 - c0) + share_weight(2) * (n - c1);
    }
    __syncthreads();
    W = HP * __builtin_amdgcn_readfirstlane(sS[a.B]);
    if (threadIdx.x <= NG) sLo[threadIdx.x] = (int)((int64_t)W * sCw[threadIdx.x] / sCw[NG]);
    __syncthreads();
    lo = __builtin_amdgcn_readfirstlane(sLo[gang]);
    hi = __builtin_amdgcn_readfirstlane(sLo[gang + 1]);
    // First pair of the share: request pb = the last with HP * S[pb] <= lo (S[0] = 0).
    int lb = 0, ub = a.B - 1;
    while (lb < ub) {
      const int mid = (lb + ub + 1) / 2;
      if (HP * __builtin_amdgcn_readfirstlane(sS[mid]) <= lo) lb = mid;
      else ub = mid - 1;
    }
    pb = lb;
    Sb = __builtin_amdgcn_readfirstlane(sS[pb]);
    P = __builtin_amdgcn_readfirstlane(sS[pb + 1]) - Sb;
    hh = (int)((lo - HP * Sb) / P);
  }
  for (bool first = true;; first = false) {
    int b, h, s_hi = 0x7fffffff;
    // BAL: the piece's step range starts at s_lo; the tile has np pieces (gangs g0 .. g0 + np - 1),
    // this one in record slot rec_slot; tile_start: the tile's list position.
    int s_lo = 0, np = 1, g0 = 0, rec_slot = 0;
    int tile_start = 0;
    if constexpr (!BAL) {
      h = bh % a.H;
      b = bh / a.H;
    } else {
      // Every member walks the share's part of every pair in it, its mates' steps included (their
      // loads and barriers, without the products past its own tile's steps), so that the gang's
      // workgroups keep reading the same KV steps at the same time.
      tile_start = HP * Sb + hh * P;
      if (lo >= hi || pb >= a.B || tile_start >= hi) break;
      s_lo = lo > tile_start ? lo - tile_start : 0;
      s_hi = hi - tile_start < P ? hi - tile_start : P;
      const int nt = tile_steps(__builtin_amdgcn_readfirstlane(sL[pb]), __builtin_amdgcn_readfirstlane(sC[pb]), qt);
      const int ntp = nt > 1 ? nt : 1;
      np = 0;  // no piece of this tile when the share starts past its steps
      if (lo < tile_start + ntp) {
        g0 = gang_of(tile_start);
        np = gang_of(tile_start + ntp - 1) - g0 + 1;
        rec_slot = lo >= tile_start ? 0 : 1;
      }
      b = pb;
      h = k + kXcds * hh;
      if (!first) __syncthreads();  // every wavefront is done with the previous piece's LDS tiles
    }
    const int i0 = qt * kWideRows;
    const int iw = i0 + 32 * w;
    const int i = iw + c;

    const int L = BAL ? __builtin_amdgcn_readfirstlane(sL[b]) : a.seq_lens[b];
    const int C = BAL ? __builtin_amdgcn_readfirstlane(sC[b]) : a.cur_lens[b];
    const int n_c = i < a.T ? valid_keys(L, C, i) : 0;
    // Blocks the walk loads: up to the last row of the tile (BAL: of the pair's last tile).
    const int last_row = BAL ? ntiles * kWideRows - 1 : i0 + kWideRows - 1;
    const int last_wg = last_row < (a.T - 1) ? last_row : (a.T - 1);
    const int n_wg = valid_keys(L, C, last_wg);  // nondecreasing in the row index
    int nb = (n_wg + 15) / 16;
    nb = nb < a.max_pages ? nb : a.max_pages;
    int nsteps = (nb + NBS - 1) / NBS;
    nsteps = nsteps < s_hi ? nsteps : s_hi;
    int wsteps = 0;  // steps this wavefront computes (its rows need no keys beyond them)
    if (iw < a.T) {
      const int last_w = (iw + 31) < (a.T - 1) ? (iw + 31) : (a.T - 1);
      wsteps = (valid_keys(L, C, last_w) + KS - 1) / KS;
      wsteps = wsteps < nsteps ? wsteps : nsteps;
    }

    // B operand of S^T = K Q^T: q[i][G2*QH + 8s + e] for MFMA s, pre-scaled, rounded to bf16.
    bf16x8 qb[NQ];
    {
      const IO* qp = static_cast<const IO*>(a.q) + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh +
                     (int64_t)(i < a.T ? i : 0) * a.q_st + G2 * QH;
      const float qs = i < a.T ? a.scale_log2 : 0.f;
#pragma unroll
      for (int s = 0; s < NQ; ++s) {
        uint32_t wd[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          wd[e] = pack_bf16x2(Elem<IO>::load(qp + 8 * s + 2 * e) * qs, Elem<IO>::load(qp + 8 * s + 2 * e + 1) * qs);
        qb[s] = __builtin_bit_cast(bf16x8, (u32x4{wd[0], wd[1], wd[2], wd[3]}));
      }
    }

    f32x16 oacc[DU];
#pragma unroll
    for (int u = 0; u < DU; ++u)
#pragma unroll
      for (int e = 0; e < 16; ++e) oacc[u][e] = 0.f;
    float m = kNegBig, l = 0.f;

    const uint16_t* kpool = static_cast<const uint16_t*>(a.k_pool);
    const uint16_t* vpool = static_cast<const uint16_t*>(a.v_pool);
    const int32_t* pt = a.page_table + (int64_t)b * a.pt_stride;
    // Page-table entries are int32: one unsigned 32-bit compare checks 0 <= e < num_blocks.
    const uint32_t nblk = a.num_blocks < 0x7fffffff ? (uint32_t)a.num_blocks : 0x7fffffffu;
    auto ok_blk = [&](int e) { return (uint32_t)e < nblk; };
    auto block_base = [&](const uint16_t* pool, int e) {
      const int blk = ok_blk(e) ? e : 0;  // masked in the softmax when invalid
      return pool + ((int64_t)blk * a.H + h) * (16 * HD);
    };

    // LDS tiles hold key rows of HD values unpadded; 16-byte chunk p of key row r holds head_dim
    // chunk p ^ kswz(r) (K) or p ^ vswz(r) (V). The swizzles make the operand reads below hit all
    // LDS banks once per pass: the 16 rows of a K read cover 16 distinct chunk positions, and the
    // 4 key rows x 4 head_dim chunks of a transposing V read cover 16 distinct chunks.
    auto kswz = [](int r) { return (r / RPB) & (CPR - 1); };
    auto vswz = [](int r) { return (4 * ((r / RPB) & 3)) & (CPR - 1); };

    // LDS-direct loads (global_load_lds_dwordx4): lane L of a wavefront's instruction writes the 16
    // bytes at LDS address dst + 16L. Instruction n of wavefront w fills key rows RPI*(w*NDMA + n)
    // ..+RPI-1 of the step tile, all in one KV block; the lane's source offset in the block is
    // fixed (kdo / vdo), only the block base changes per step.
    uint32_t kdo[NDMA], vdo[NDMA];
#pragma unroll
    for (int n = 0; n < NDMA; ++n) {
      const int r = (w * NDMA + n) * RPI + lane / CPR;
      const int p = lane % CPR;
      kdo[n] = (uint32_t)((r & 15) * HD + 8 * (p ^ kswz(r)));
      vdo[n] = (uint32_t)((r & 15) * HD + 8 * (p ^ vswz(r)));
    }
    // Page-table entries come from a per-wavefront copy of 64 consecutive entries (lane i holds
    // entry ptb + i), refreshed when a step's blocks leave it (64 is a multiple of NBS): one
    // vector load per 64 blocks instead of one scalar load and wait per step.
    int ptc = 0, ptb = -64;
    auto issue_loads = [&](int st, int (&ent)[NBS], uint16_t* skx, uint16_t* svx) {
      const int j0 = NBS * st;
      if (j0 - ptb >= 64) {
        ptb = j0;
        const int idx = j0 + lane;
        ptc = load_now(pt + (idx < nb ? idx : 0));
      }
#pragma unroll
      for (int j = 0; j < NBS; ++j) ent[j] = j0 + j < nb ? __builtin_amdgcn_readlane(ptc, j0 - ptb + j) : -1;
#pragma unroll
      for (int n = 0; n < NDMA; ++n) {
        const int r0 = (w * NDMA + n) * RPI;
        const int e = ent[r0 >> 4];
        lds_direct_load16(block_base(kpool, e), 2 * kdo[n], skx + r0 * HD);
        lds_direct_load16(block_base(vpool, e), 2 * vdo[n], svx + r0 * HD);
      }
    };

    // Per-lane LDS element offsets of the operand reads (fixed for the whole walk).
    //   K (A of S^T = K Q^T, MFMA s, sub-tile u): key row c + 32u, head_dim chunk G2*CPR/2 + s.
    //   V (A of O^T += V^T P^T, tile d): ds_read_b64_tr_b16 gives lane j of each 16-lane group
    //   element r = the value at row r' = r, column j of the 4 x 16 block its group addresses
    //   (lanes 4r' + a' supply the addresses of row r', columns 4a'..4a'+3). Lane (G2, c) reads,
    //   for 4 keys K0 + r (r = (c mod 16) / 4), head_dim 32d + 16(c / 16) + 4(c mod 4): it then
    //   holds V[K0 + r][32d + c], r = 0..3 — four k slots of row c of V^T.
    const int kx = kswz(c);
    const int vr4 = (c & 15) >> 2;
    const int vx = vswz(4 * G2 + vr4);
    auto v_off = [&](int d) {
      const int hd = 32 * d + 16 * (c >> 4) + 4 * (c & 3);
      return (4 * G2 + vr4) * HD + 8 * ((hd >> 3) ^ vx) + (hd & 4);
    };

    typedef short s16x4 __attribute__((ext_vector_type(4)));
    auto compute = [&](const uint16_t* skx, const uint16_t* svx, int st, const int (&ent)[NBS]) {
      // ---- S^T = K Q^T for each 32-key sub-tile ------------------------------------------------
      f32x16 sacc[NSUB];
#pragma unroll
      for (int u = 0; u < NSUB; ++u)
#pragma unroll
        for (int e = 0; e < 16; ++e) sacc[u][e] = 0.f;
#pragma unroll
      for (int s = 0; s < NQ; ++s)
#pragma unroll
        for (int u = 0; u < NSUB; ++u) {
          const bf16x8 kf = *reinterpret_cast<const bf16x8*>(skx + (c + 32 * u) * HD + 8 * ((G2 * (CPR / 2) + s) ^ kx));
          sacc[u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qb[s], sacc[u], 0, 0, 0);
        }
      // ---- online softmax (sub-tile u, keys 32u + 8j + 4*G2 + r of this step), in place --------
      bool all_ok = true;
#pragma unroll
      for (int j = 0; j < NBS; ++j) all_ok = all_ok && ok_blk(ent[j]);
      // Interior steps (every block valid, every key below every row's limit) need no mask.
      const bool full = all_ok && __builtin_amdgcn_ballot_w64(n_c < (st + 1) * KS) == 0;
      if (!full) {
        const int t0 = st * KS + 4 * G2;
#pragma unroll
        for (int u = 0; u < NSUB; ++u)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const bool okb = ok_blk(ent[2 * u + (j >> 1)]);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int t = t0 + 32 * u + 8 * j + r;
              sacc[u][4 * j + r] = (okb && t < n_c) ? sacc[u][4 * j + r] : -INFINITY;
            }
          }
      }
      float mloc = -INFINITY;
#pragma unroll
      for (int u = 0; u < NSUB; ++u)
#pragma unroll
        for (int e = 0; e < 16; ++e) mloc = fmaxf(mloc, sacc[u][e]);
      mloc = max_xor32(mloc);
      const bool grow = mloc > m + kRescaleSlack;
      if (__builtin_amdgcn_ballot_w64(grow) != 0) {
        const float mnew = grow ? mloc : m;
        const float alpha = fast_exp2(m - mnew);
        l *= alpha;
#pragma unroll
        for (int u = 0; u < DU; ++u) oacc[u] *= alpha;
        m = mnew;
      }
      float ps = 0.f;
#pragma unroll
      for (int u = 0; u < NSUB; ++u)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          sacc[u][e] = fast_exp2(sacc[u][e] - m);
          ps += sacc[u][e];
        }
      l += sum_xor32(ps);
      // ---- O^T += V^T P^T: MFMA (u2, mm, d) contracts keys 32u2 + 16mm + 8jj + 4*G2 + r at slot
      // (G2, 4jj + r), i.e. the lane's registers 8mm + 4jj + r ----------------------------------
      // The PV MFMAs run at raised wavefront priority, so a wavefront that reaches them issues
      // ahead of co-resident wavefronts still in their softmax and the matrix pipe stays fed (the
      // same around the QK^T MFMAs costs 20 registers and a wavefront per SIMD).
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int u2 = 0; u2 < NSUB; ++u2)
#pragma unroll
        for (int mm = 0; mm < 2; ++mm) {
          uint32_t pw[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) pw[q] = pack_bf16x2(sacc[u2][8 * mm + 2 * q], sacc[u2][8 * mm + 2 * q + 1]);
          const bf16x8 pb = __builtin_bit_cast(bf16x8, (u32x4{pw[0], pw[1], pw[2], pw[3]}));
#pragma unroll
          for (int d = 0; d < DU; ++d) {
            const uint16_t* vp = svx + v_off(d) + (32 * u2 + 16 * mm) * HD;
            const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) s16x4*)(vp));
            const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) s16x4*)(vp + 8 * HD));
            const bf16x8 vf = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
            oacc[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pb, oacc[d], 0, 0, 0);
          }
        }
      __builtin_amdgcn_s_setprio(0);
    };

    // NST-stage pipeline: the loads of step st + NST - 1 are issued once every wavefront is past
    // step st - 1 (whose stage they reuse), NST - 1 steps ahead of their use. Before computing step
    // st a wavefront waits for its own loads of step st (vmcnt: those of the later steps may still
    // be in flight) and the barrier makes every wavefront's loads of step st visible.
    if (s_lo < nsteps) {
      int e0[NBS], e1[NBS], e2[NBS];  // page-table entries of the steps in stages 0, 1, 2
      issue_loads(s_lo, e0, sk0, sv0);
      if (NST > 2 && s_lo + 1 < nsteps) issue_loads(s_lo + 1, e1, sk1, sv1);
      auto iteration = [&](int st, const int (&ec)[NBS], int (&en)[NBS], const uint16_t* skc, const uint16_t* svc,
                           uint16_t* skn, uint16_t* svn) {
        if (NST > 2 && st + 1 < nsteps) __builtin_amdgcn_s_waitcnt(0x0F70 | (2 * NDMA));  // vmcnt(2 * NDMA)
        else __builtin_amdgcn_s_waitcnt(0x0F70);                                           // vmcnt(0)
        __syncthreads();
        // The next stage's loads are issued at raised priority too, so they start right after
        // the barrier.
        __builtin_amdgcn_s_setprio(1);
        if (st + NST - 1 < nsteps) issue_loads(st + NST - 1, en, skn, svn);
        __builtin_amdgcn_s_setprio(0);
        if (st < wsteps) compute(skc, svc, st, ec);
      };
      if constexpr (NST == 3) {
        for (int st = s_lo; st < nsteps; st += 3) {
          iteration(st, e0, e2, sk0, sv0, sk2, sv2);
          if (st + 1 < nsteps) iteration(st + 1, e1, e0, sk1, sv1, sk0, sv0);
          if (st + 2 < nsteps) iteration(st + 2, e2, e1, sk2, sv2, sk1, sv1);
        }
      } else {
        for (int st = s_lo; st < nsteps; st += 2) {
          iteration(st, e0, e1, sk0, sv0, sk1, sv1);
          if (st + 1 < nsteps) iteration(st + 1, e1, e0, sk1, sv1, sk0, sv0);
        }
      }
    }

    bool store = true;
    if constexpr (BAL) {
      if (np == 0) {
        store = false;
      } else if (np > 1) {
        // Cut tile, pieces in gangs g0 .. g0 + np - 1. A piece writes its record (device-scope
        // stores), waits for them and counts itself in; the piece that arrives last resets the
        // counter and merges the pieces in gang order. Gang g0's piece ends its share, so it
        // usually arrives last: it first looks whether all the others have arrived, and then
        // writes no record. Merging starts from gang g0's state, taken from the registers when this
        // is gang g0 (the values its record would hold), so the result does not depend on which
        // piece arrives last.
        int32_t* cnt = a.counters + ((int64_t)b * a.H + h) * ntiles + qt;
        constexpr int WREC = kWideRecGroups<HD> * kWave * 4;  // a wavefront's floats in a record
        bool last = false;
        if (gang == g0) {
          if (threadIdx.x == 0) sm_last = __hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == np - 1;
          __syncthreads();
          last = __builtin_amdgcn_readfirstlane(sm_last);
        }
        if (!last) {
          float* rp = a.ws + ((int64_t)blockIdx.x * 2 + rec_slot) * kWideRecFloats<HD> + w * WREC + 4 * lane;
          store_record_group(rp, f32x4{m, l, 0.f, 0.f});
#pragma unroll
          for (int d = 0; d < DU; ++d)
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4)
              store_record_group(rp + (1 + 4 * d + q4) * 4 * kWave,
                                 f32x4{oacc[d][4 * q4], oacc[d][4 * q4 + 1], oacc[d][4 * q4 + 2], oacc[d][4 * q4 + 3]});
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
          __syncthreads();
          if (threadIdx.x == 0)
            sm_last = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == np - 1;
          __syncthreads();
          last = __builtin_amdgcn_readfirstlane(sm_last);
        }
        store = last;
        if (last) {
          if (threadIdx.x == 0) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          // Gang gg's record is in its slot 0, except gang g0's when its share starts before the
          // tile (the tile is then its share's last pair: slot 1).
          if (gang != g0) {
            m = kNegBig;
            l = 0.f;
          }
          for (int gg = gang == g0 ? g0 + 1 : g0; gg < g0 + np; ++gg) {
            const int slot = __builtin_amdgcn_readfirstlane(sLo[gg]) >= tile_start ? 0 : 1;
            const int64_t x = (int64_t)kXcds * ((int64_t)gg * ntiles + qt) + k;
            const float* rq = a.ws + (x * 2 + slot) * kWideRecFloats<HD> + w * WREC + 4 * lane;
            f32x4 lo[9];
            load_record_lo(rq, lo);
            const float mr = lo[0][0], lr = lo[0][1];
            const float mn = fmaxf(m, mr);
            const float fa = gg == g0 ? 0.f : fast_exp2(m - mn), fr = fast_exp2(mr - mn);
            l = l * fa + lr * fr;
            m = mn;
#pragma unroll
            for (int gi = 1; gi < 9; ++gi)
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const int d = (gi - 1) / 4, r = 4 * ((gi - 1) % 4) + e;
                oacc[d][r] = oacc[d][r] * fa + lo[gi][e] * fr;
              }
            if constexpr (HD == 128) {
              f32x4 hi[8];
              load_record_hi(rq, hi);
#pragma unroll
              for (int gi = 9; gi < 17; ++gi)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                  const int d = (gi - 1) / 4, r = 4 * ((gi - 1) % 4) + e;
                  oacc[d][r] = oacc[d][r] * fa + hi[gi - 9][e] * fr;
                }
            }
          }
        }
      }
    }

    // ---- write: lane holds O^T rows 8j + 4*G2 + r (head_dim 32d + row) of query column c -------
    if (store && i < a.T) {
      const float inv = l > 0.f ? 1.f / l : 0.f;
      IO* op = static_cast<IO*>(a.out) + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh + (int64_t)i * a.o_st;
#pragma unroll
      for (int d = 0; d < DU; ++d)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) Elem<IO>::store(op + 32 * d + 8 * j + 4 * G2 + r, oacc[d][4 * j + r] * inv);
    }
    if constexpr (!BAL) {
      break;
    } else {
      if (++hh == HP) {
        hh = 0;
        if (++pb < a.B) {
          Sb = __builtin_amdgcn_readfirstlane(sS[pb]);
          P = __builtin_amdgcn_readfirstlane(sS[pb + 1]) - Sb;
        }
      }
    }
  }  // pieces
}

// fp32 KV: the same workgroup layout, LDS staging and online softmax, on v_mfma_f32_32x32x2_f32
// (fp32 products, like the reference's fp32 path):
//   S^T = K Q^T      MFMA s (s < HD/2) contracts head_dim slot G2 = index G2*HD/2 + s: lane
//                    (G2, c) gives K[key c][index] (A, from LDS) and q[query c][index] (B, held
//                    in registers for the whole walk);
//   O^T += V^T P^T   MFMA (j, r) contracts key slot G2 = key 8j + 4*G2 + r, the key whose score
//                    lane (G2, c) holds in its register 4j + r: A = V[that key][c*DU + d] (output
//                    tile d, row c) and B = its softmax weight, exactly as held.
// Per 32-key step a wavefront issues HD MFMAs of 32x32x2 (HD/2 for QK^T, HD/2 for PV), so the
// per-step costs are small next to the matrix work.
template <typename IO, int HD, bool BAL>
__global__ __launch_bounds__(kWideWaves * kWave) void prefill_wide_f32_kernel(const AttnArgs a) {
  constexpr int NW = kWideWaves;
  constexpr int KS = 32;                 // keys per step (two 16-token blocks)
  constexpr int NBS = 2;
  constexpr int QH = HD / 2;             // head_dim values per lane in the QK^T operands
  constexpr int DU = HD / 32;            // output tiles of 32 head_dim rows
  constexpr int RS = HD + 4;             // LDS row stride in floats (16-byte pad)
  constexpr int RPC = HD / 4;            // 16-byte chunks per key row
  constexpr int CPT = KS * RPC / (NW * kWave);
  static_assert(CPT >= 1 && KS * RPC == CPT * NW * kWave, "tile split");
  static_assert(!BAL || HD == 128 || HD == 64, "balanced launch shape");

  __shared__ __attribute__((aligned(16))) float sk[2][KS * RS];
  __shared__ __attribute__((aligned(16))) float sv[2][KS * RS];

  const int lane = threadIdx.x & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int G2 = lane >> 5;
  const int c = lane & 31;

  const int ntiles = (a.T + kWideRows - 1) / kWideRows;
  // Steps of 32 keys that tile qt of request b walks (the valid keys of its last row).
  auto tile_steps = [&](int L, int C, int rqt) {
    const int last = (rqt * kWideRows + kWideRows - 1) < (a.T - 1) ? (rqt * kWideRows + kWideRows - 1) : (a.T - 1);
    int nbb = (valid_keys(L, C, last) + 15) / 16;  // nondecreasing in the row
    nbb = nbb < a.max_pages ? nbb : a.max_pages;
    return (nbb + NBS - 1) / NBS;
  };
  int bh = 0, qt = 0;
  // BAL (as in prefill_wide_kernel): this workgroup's share [lo, hi) of its die's pair list, the
  // pair it has reached (request pb, head k + 8 hh), that pair's list position Sb and work P.
  int k = 0, gang = 0, NG = 1, HP = 1, pb = 0, hh = 0, P = 1;
  int W = 1, lo = 0, hi = 0, Sb = 0;
  __shared__ int sm_last;                     // BAL: this piece arrived last
  __shared__ int sP[kWideWaves * kWave];      // BAL: pair work per request
  __shared__ int sS[kWideWaves * kWave];      // BAL: its prefix sums
  __shared__ int sCw[kWideWaves * kWave];     // BAL: prefix sums of the gangs' share weights
  __shared__ int sLo[kWideWaves * kWave];     // BAL: the gangs' shares: [sLo[g], sLo[g + 1])
  __shared__ int sL[kWideWaves * kWave];      // BAL: each request's seq_lens and cur_lens, read once
  __shared__ int sC[kWideWaves * kWave];
  auto gang_of = [&](int pos) {
    int lg = 0, ug = NG - 1;
    while (lg < ug) {
      const int mid = (lg + ug + 1) / 2;
      if (__builtin_amdgcn_readfirstlane(sLo[mid]) <= pos) lg = mid;
      else ug = mid - 1;
    }
    return lg;
  };
  if constexpr (!BAL) {
    static_assert(sizeof(sk) >= (kOrderMax + 1) * sizeof(int), "order scratch");
    if (!wide_lpt_unit(a, ntiles, reinterpret_cast<int*>(&sk[0][0]), bh, qt)) wide_unit(blockIdx.x, a.B * a.H, ntiles, bh, qt);
  } else {
    k = blockIdx.x % kXcds;
    const int jx = blockIdx.x / kXcds;
    gang = jx / ntiles;
    qt = jx - gang * ntiles;
    NG = gridDim.x / (kXcds * ntiles);
    HP = a.H / kXcds;
    if (threadIdx.x < a.B) {
      const int L = a.seq_lens[threadIdx.x], C = a.cur_lens[threadIdx.x];
      sL[threadIdx.x] = L;
      sC[threadIdx.x] = C;
      const int p = tile_steps(L, C, ntiles - 1);
      sP[threadIdx.x] = p > 1 ? p : 1;
    }
    __syncthreads();
    if (threadIdx.x <= a.B) {
      int s = 0;
      for (int r = 0; r < (int)threadIdx.x; ++r) s += sP[r];
      sS[threadIdx.x] = s;
    }
    if (threadIdx.x <= NG) {
      // share_weight(g ntiles / die_cus) summed over g < n: its value is share_weight(0) while
      // g ntiles < die_cus (g < n0), share_weight(1) while g ntiles < 2 die_cus (g < n1), then
      // share_weight(2).
      const int n = threadIdx.x;
      const int n0 = (a.die_cus + ntiles - 1) / ntiles, n1 = (2 * a.die_cus + ntiles - 1) / ntiles;
      const int c0 = n < n0 ? n : n0, c1 = n < n1 ? n : n1;
      sCw[threadIdx.x] = share_weight(0) * c0 + share_weight(1) * (c1 - c0) + share_weight(2) * (n - c1);
    }
    __syncthreads();
    W = HP * __builtin_amdgcn_readfirstlane(sS[a.B]);
    if (threadIdx.x <= NG) sLo[threadIdx.x] = (int)((int64_t)W * sCw[threadIdx.x] / sCw[NG]);
    __syncthreads();
    lo = __builtin_amdgcn_readfirstlane(sLo[gang]);
    hi = __builtin_amdgcn_readfirstlane(sLo[gang + 1]);
    int lb = 0, ub = a.B - 1;
    while (lb < ub) {
      const int mid = (lb + ub + 1) / 2;
      if (HP * __builtin_amdgcn_readfirstlane(sS[mid]) <= lo) lb = mid;
      else ub = mid - 1;
    }
    pb = lb;
    Sb = __builtin_amdgcn_readfirstlane(sS[pb]);
    P = __builtin_amdgcn_readfirstlane(sS[pb + 1]) - Sb;
    hh = (int)((lo - HP * Sb) / P);
  }
  for (bool first = true;; first = false) {
  int b, h, s_hi = 0x7fffffff;
  int s_lo = 0, np = 1, g0 = 0, rec_slot = 0;
  int tile_start = 0;
  if constexpr (!BAL) {
    h = bh % a.H;
    b = bh / a.H;
  } else {
    tile_start = HP * Sb + hh * P;
    if (lo >= hi || pb >= a.B || tile_start >= hi) break;
    s_lo = lo > tile_start ? lo - tile_start : 0;
    s_hi = hi - tile_start < P ? hi - tile_start : P;
    const int nt = tile_steps(__builtin_amdgcn_readfirstlane(sL[pb]), __builtin_amdgcn_readfirstlane(sC[pb]), qt);
    const int ntp = nt > 1 ? nt : 1;
    np = 0;  // no piece of this tile when the share starts past its steps
    if (lo < tile_start + ntp) {
      g0 = gang_of(tile_start);
      np = gang_of(tile_start + ntp - 1) - g0 + 1;
      rec_slot = lo >= tile_start ? 0 : 1;
    }
    b = pb;
    h = k + kXcds * hh;
    if (!first) __syncthreads();  // every wavefront is done with the previous piece's LDS tiles
  }
  const int i0 = qt * kWideRows;
  const int iw = i0 + 32 * w;
  const int i = iw + c;

  const int L = BAL ? __builtin_amdgcn_readfirstlane(sL[b]) : a.seq_lens[b];
  const int C = BAL ? __builtin_amdgcn_readfirstlane(sC[b]) : a.cur_lens[b];
  const int n_c = i < a.T ? valid_keys(L, C, i) : 0;
  // Blocks the walk loads: up to the last row of the tile (BAL: of the pair's last tile, so that
  // a gang's workgroups walk the same steps).
  const int last_row = BAL ? ntiles * kWideRows - 1 : i0 + kWideRows - 1;
  const int last_wg = last_row < (a.T - 1) ? last_row : (a.T - 1);
  const int n_wg = valid_keys(L, C, last_wg);
  int nb = (n_wg + 15) / 16;
  nb = nb < a.max_pages ? nb : a.max_pages;
  int nsteps = (nb + NBS - 1) / NBS;
  nsteps = nsteps < s_hi ? nsteps : s_hi;
  int wsteps = 0;
  if (iw < a.T) {
    const int last_w = (iw + 31) < (a.T - 1) ? (iw + 31) : (a.T - 1);
    wsteps = (valid_keys(L, C, last_w) + KS - 1) / KS;
    wsteps = wsteps < nsteps ? wsteps : nsteps;
  }

  // B operand of S^T = K Q^T: q[i][G2*QH + s], pre-scaled into the log2 domain.
  float qf[QH];
  {
    const IO* qp = static_cast<const IO*>(a.q) + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh +
                   (int64_t)(i < a.T ? i : 0) * a.q_st + G2 * QH;
    const float qs = i < a.T ? a.scale_log2 : 0.f;
#pragma unroll
    for (int s = 0; s < QH; ++s) qf[s] = Elem<IO>::load(qp + s) * qs;
  }

  f32x16 oacc[DU];
#pragma unroll
  for (int d = 0; d < DU; ++d)
#pragma unroll
    for (int e = 0; e < 16; ++e) oacc[d][e] = 0.f;
  float m = kNegBig, l = 0.f;

  const float* kpool = static_cast<const float*>(a.k_pool);
  const float* vpool = static_cast<const float*>(a.v_pool);
  const int32_t* pt = a.page_table + (int64_t)b * a.pt_stride;
  // Page-table entries are int32: one unsigned 32-bit compare checks 0 <= e < num_blocks.
  const uint32_t nblk = a.num_blocks < 0x7fffffff ? (uint32_t)a.num_blocks : 0x7fffffffu;
  auto ok_blk = [&](int e) { return (uint32_t)e < nblk; };

  u32x4 kr[CPT], vr[CPT];
  auto gload = [&](int st, int (&ent)[NBS]) {
#pragma unroll
    for (int j = 0; j < NBS; ++j) ent[j] = NBS * st + j < nb ? pt[NBS * st + j] : -1;
#pragma unroll
    for (int n = 0; n < CPT; ++n) {
      const int q = threadIdx.x + n * NW * kWave;
      const int kk = q / RPC;
      const int col = (q - kk * RPC) * 4;
      const int e = ent[kk >> 4];
      const int blk = ok_blk(e) ? e : 0;  // masked in the softmax when invalid
      const int64_t off = (((int64_t)blk * a.H + h) * 16 + (kk & 15)) * HD + col;
      kr[n] = *reinterpret_cast<const u32x4*>(kpool + off);
      vr[n] = *reinterpret_cast<const u32x4*>(vpool + off);
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int n = 0; n < CPT; ++n) {
      const int q = threadIdx.x + n * NW * kWave;
      const int kk = q / RPC;
      const int col = (q - kk * RPC) * 4;
      *reinterpret_cast<u32x4*>(&sk[buf][kk * RS + col]) = kr[n];
      *reinterpret_cast<u32x4*>(&sv[buf][kk * RS + col]) = vr[n];
    }
  };

  auto compute = [&](int buf, int st, const int (&ent)[NBS]) {
    // ---- S^T = K Q^T ------------------------------------------------------------------------
    f32x16 sacc;
#pragma unroll
    for (int e = 0; e < 16; ++e) sacc[e] = 0.f;
    const float* krow = &sk[buf][c * RS + G2 * QH];
#pragma unroll
    for (int s = 0; s < QH; s += 4) {
      const f32x4 kv = *reinterpret_cast<const f32x4*>(krow + s);
#pragma unroll
      for (int e = 0; e < 4; ++e) sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[e], qf[s + e], sacc, 0, 0, 0);
    }
    // ---- online softmax (keys 8j + 4*G2 + r of this step) --------------------------------------
    const bool ok0 = ok_blk(ent[0]), ok1 = ok_blk(ent[1]);
    const bool full = ok0 && ok1 && __builtin_amdgcn_ballot_w64(n_c < (st + 1) * KS) == 0;
    float p[16];
    float mloc = -INFINITY;
    if (full) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        p[e] = sacc[e];
        mloc = fmaxf(mloc, p[e]);
      }
    } else {
      const int t0 = st * KS + 4 * G2;
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = t0 + 8 * j + r;
          p[4 * j + r] = ((j < 2 ? ok0 : ok1) && t < n_c) ? sacc[4 * j + r] : -INFINITY;
          mloc = fmaxf(mloc, p[4 * j + r]);
        }
    }
    mloc = max_xor32(mloc);
    const bool grow = mloc > m + kRescaleSlack;
    if (__builtin_amdgcn_ballot_w64(grow) != 0) {
      const float mnew = grow ? mloc : m;
      const float alpha = fast_exp2(m - mnew);
      l *= alpha;
#pragma unroll
      for (int d = 0; d < DU; ++d) oacc[d] *= alpha;
      m = mnew;
    }
    float ps = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      p[e] = fast_exp2(p[e] - m);
      ps += p[e];
    }
    l += sum_xor32(ps);
    // ---- O^T += V^T P^T: four keys (one row group j) at a time ----------------------------------
    // At raised wavefront priority, as in the bf16 kernel.
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float vv[4][DU];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float* vp = &sv[buf][(8 * j + 4 * G2 + r) * RS + c * DU];
        if constexpr (DU == 4) {
          const f32x4 x = *reinterpret_cast<const f32x4*>(vp);
          vv[r][0] = x[0]; vv[r][1] = x[1]; vv[r][2] = x[2]; vv[r][3] = x[3];
        } else {
          const u32x2 x = *reinterpret_cast<const u32x2*>(vp);
          vv[r][0] = __uint_as_float(x[0]); vv[r][1] = __uint_as_float(x[1]);
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int d = 0; d < DU; ++d)
          oacc[d] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv[r][d], p[4 * j + r], oacc[d], 0, 0, 0);
    }
    __builtin_amdgcn_s_setprio(0);
  };

  if (s_lo < nsteps) {
    int cur[NBS], nxt[NBS];
    gload(s_lo, cur);
    lstore(0);
    __syncthreads();
    for (int st = s_lo; st < nsteps; ++st) {
      const bool more = st + 1 < nsteps;
      if (more) gload(st + 1, nxt);
      if (st < wsteps) compute((st - s_lo) & 1, st, cur);
      if (more) lstore((st + 1 - s_lo) & 1);
      __syncthreads();
#pragma unroll
      for (int j = 0; j < NBS; ++j) cur[j] = nxt[j];
    }
  }

  bool store = true;
  if constexpr (BAL) {
    if (np == 0) {
      store = false;
    } else if (np > 1) {
      // Cut tile: the record and merge protocol of prefill_wide_kernel (same accumulator layout).
      int32_t* cnt = a.counters + ((int64_t)b * a.H + h) * ntiles + qt;
      constexpr int WREC = kWideRecGroups<HD> * kWave * 4;  // a wavefront's floats in a record
      bool last = false;
      if (gang == g0) {
        if (threadIdx.x == 0) sm_last = __hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == np - 1;
        __syncthreads();
        last = __builtin_amdgcn_readfirstlane(sm_last);
      }
      if (!last) {
        float* rp = a.ws + ((int64_t)blockIdx.x * 2 + rec_slot) * kWideRecFloats<HD> + w * WREC + 4 * lane;
        store_record_group(rp, f32x4{m, l, 0.f, 0.f});
#pragma unroll
        for (int d = 0; d < DU; ++d)
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4)
            store_record_group(rp + (1 + 4 * d + q4) * 4 * kWave,
                               f32x4{oacc[d][4 * q4], oacc[d][4 * q4 + 1], oacc[d][4 * q4 + 2], oacc[d][4 * q4 + 3]});
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (threadIdx.x == 0)
          sm_last = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == np - 1;
        __syncthreads();
        last = __builtin_amdgcn_readfirstlane(sm_last);
      }
      store = last;
      if (last) {
        if (threadIdx.x == 0) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (gang != g0) {
          m = kNegBig;
          l = 0.f;
        }
        for (int gg = gang == g0 ? g0 + 1 : g0; gg < g0 + np; ++gg) {
          const int slot = __builtin_amdgcn_readfirstlane(sLo[gg]) >= tile_start ? 0 : 1;
          const int64_t x = (int64_t)kXcds * ((int64_t)gg * ntiles + qt) + k;
          const float* rq = a.ws + (x * 2 + slot) * kWideRecFloats<HD> + w * WREC + 4 * lane;
          f32x4 lo4[9];
          load_record_lo(rq, lo4);
          const float mr = lo4[0][0], lr = lo4[0][1];
          const float mn = fmaxf(m, mr);
          const float fa = gg == g0 ? 0.f : fast_exp2(m - mn), fr = fast_exp2(mr - mn);
          l = l * fa + lr * fr;
          m = mn;
#pragma unroll
          for (int gi = 1; gi < 9; ++gi)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int d = (gi - 1) / 4, r = 4 * ((gi - 1) % 4) + e;
              oacc[d][r] = oacc[d][r] * fa + lo4[gi][e] * fr;
            }
          if constexpr (HD == 128) {
            f32x4 hi4[8];
            load_record_hi(rq, hi4);
#pragma unroll
            for (int gi = 9; gi < 17; ++gi)
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const int d = (gi - 1) / 4, r = 4 * ((gi - 1) % 4) + e;
                oacc[d][r] = oacc[d][r] * fa + hi4[gi - 9][e] * fr;
              }
          }
        }
      }
    }
  }

  if (store && i < a.T) {
  const float inv = l > 0.f ? 1.f / l : 0.f;
  IO* op = static_cast<IO*>(a.out) + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh + (int64_t)i * a.o_st;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int R = 8 * j + 4 * G2 + r;
#pragma unroll
      for (int d = 0; d < DU; ++d) Elem<IO>::store(op + R * DU + d, oacc[d][4 * j + r] * inv);
    }
  }
  if constexpr (!BAL) {
    break;
  } else {
    if (++hh == HP) {
      hh = 0;
      if (++pb < a.B) {
        Sb = __builtin_amdgcn_readfirstlane(sS[pb]);
        P = __builtin_amdgcn_readfirstlane(sS[pb + 1]) - Sb;
      }
    }
  }
  }  // pieces
}

// ---------------------------------------------------------------------------------------------
// Split-step kernel for short chunks with bf16 KV: one workgroup of 8 wavefronts per (request,
// head, tile of 32 query rows). Every wavefront holds the tile's 32 rows and takes every 8th
// 32-key step of the tile's keys (steps w, w + 8, ...), streaming its steps' K and V tiles into its
// own two-stage LDS ring with LDS-direct loads; the wavefronts' online-softmax states are merged
// in LDS at the end. A step is the wide kernel's step on v_mfma_f32_32x32x16_bf16 (same operand
// layouts, swizzles, masking and lazy rescale): 32 x 32 scores per MFMA chain and 16 scores per
// lane per exchange, where the 16-row kernel's 16 x 16 blocks give 4. At chunk sizes where the
// wide kernel's 128-row tiles leave most compute units idle (4 x 8 heads x 256 rows: 64 tiles),
// this grid has one workgroup per compute unit.
constexpr int kSplitWaves = 8;
constexpr int kSplitRows = 32;

template <typename IO, int HD>
__global__ __launch_bounds__(kSplitWaves * kWave) void prefill_split_kernel(const AttnArgs a) {
  constexpr int NW = kSplitWaves;
  constexpr int KS = 32;                 // keys per step: two KV blocks
  constexpr int QH = HD / 2;             // head_dim values per lane in the QK^T operands
  constexpr int NQ = HD / 16;            // QK^T MFMAs per step (k = 16 each)
  constexpr int DU = HD / 32;            // output tiles of 32 head_dim rows
  constexpr int CPR = HD / 8;            // 16-byte chunks per key row
  constexpr int RPI = kWave / CPR;       // key rows per LDS-direct load instruction (1 KB)
  constexpr int NDMA = KS / RPI;         // such instructions per K (or V) tile
  constexpr int RPB = 128 / HD;          // key rows per 256 bytes (one pass over the LDS banks)
  constexpr int TILE = KS * HD;          // elements per K (or V) tile
  constexpr int kRing = 2 * 2 * TILE * 2;          // bytes: two stages of (K, V)
  constexpr int kOS = HD + 4;                       // floats per merge row
  constexpr int kOB = kSplitRows * kOS * 4;         // bytes of a wavefront's merge rows
  constexpr int kWaveB = kRing > kOB ? kRing : kOB;
  static_assert(NDMA >= 1 && NDMA * RPI == KS && 16 % RPI == 0 && kWaveB % 16 == 0, "tile split");
  constexpr int TPR = NW * kWave / kSplitRows;      // merge: threads per row
  constexpr int VPT = HD / TPR;                     // merge: head_dim values per thread
  static_assert(VPT % 4 == 0, "merge: 16-byte pieces");
  __shared__ __attribute__((aligned(16))) unsigned char smem[NW * kWaveB];
  __shared__ float sm_m[NW][kSplitRows];
  __shared__ float sm_l[NW][kSplitRows];
  constexpr int kQRB = HD * (int)sizeof(IO);  // bytes of a q row
  constexpr int kQS = kQRB + 16;               // LDS stride of the staged q rows
  __shared__ __attribute__((aligned(16))) unsigned char sm_q[kSplitRows * kQS];

  const int lane = threadIdx.x & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int G2 = lane >> 5;
  const int c = lane & 31;

  // Unit: (request, head) pair and 32-row tile; when the pairs divide over the dies, all tiles of
  // a pair run on one die (workgroup x on die x % kXcds), so its KV is fetched into one L2.
  const int ntiles = (a.T + kSplitRows - 1) / kSplitRows;
  const int pairs = a.B * a.H;
  int bh, qt;
  {
    const int x = blockIdx.x;
    if (pairs % kXcds == 0) {
      const int y = x / kXcds;
      bh = (y / ntiles) * kXcds + x % kXcds;
      qt = ntiles - 1 - y % ntiles;
    } else {
      bh = x / ntiles;
      qt = ntiles - 1 - x % ntiles;
    }
  }
  const int h = bh % a.H;
  const int b = bh / a.H;
  const int i0 = qt * kSplitRows;
  const int i = i0 + c;

  const int L = a.seq_lens[b];
  const int C = a.cur_lens[b];
  // The first page-table chunk (see the walk below) is read together with the lengths, for every
  // block of the table's row, and cut to the request's blocks once the lengths are known: one
  // dependent round trip less before the first KV load.
  const int32_t* pt = a.page_table + (int64_t)b * a.pt_stride;
  int ent0 = -1;
  {
    const int blk = 2 * (w + NW * (lane / 2)) + (lane & 1);
    if (blk < a.max_pages) ent0 = pt[blk];
  }
  const int n_c = i < a.T ? valid_keys(L, C, i) : 0;
  const int last = (i0 + kSplitRows - 1) < (a.T - 1) ? (i0 + kSplitRows - 1) : (a.T - 1);
  int nb = (valid_keys(L, C, last) + 15) / 16;
  nb = nb < a.max_pages ? nb : a.max_pages;
  const int nsteps = (nb + 1) / 2;
  const int mine = nsteps > w ? (nsteps - w + NW - 1) / NW : 0;  // this wavefront's steps

  // B operand of S^T = K Q^T: q[i][G2*QH + 8s + e] for MFMA s, pre-scaled, rounded to bf16. Every
  // wavefront needs the same 32 rows: they are read once per workgroup, 16 bytes per thread with
  // consecutive threads along a row, into LDS rows padded by 16 bytes (the 8 rows of a 16-byte read
  // pass then fall in distinct banks), and each lane reads its half row from there, instead of 8
  // copies of the tile loaded by every wavefront with each load instruction touching 64 rows.
  // Rows that are not 16-byte aligned take element loads instead.
  bf16x8 qb[NQ];
  const float qsc = i < a.T ? a.scale_log2 : 0.f;
  constexpr int64_t kIOB = sizeof(IO);
  if ((((uint64_t)(size_t)a.q | (uint64_t)(a.q_sb * kIOB) | (uint64_t)(a.q_sh * kIOB) | (uint64_t)(a.q_st * kIOB)) &
       15) == 0) {
    constexpr int CH = kQRB / 16;  // 16-byte chunks per row
    const unsigned char* qrow0 =
        static_cast<const unsigned char*>(a.q) + ((int64_t)b * a.q_sb + (int64_t)h * a.q_sh) * kIOB;
    for (int idx = threadIdx.x; idx < kSplitRows * CH; idx += NW * kWave) {
      const int r = idx / CH, ch = idx - r * CH;
      const int row = i0 + r < a.T ? i0 + r : 0;
      *reinterpret_cast<u32x4*>(sm_q + r * kQS + 16 * ch) =
          *reinterpret_cast<const u32x4*>(qrow0 + (int64_t)row * a.q_st * kIOB + 16 * ch);
    }
    __syncthreads();
    constexpr int EPC = 16 / (int)sizeof(IO);  // elements per 16-byte chunk
#pragma unroll
    for (int s2 = 0; s2 < NQ; ++s2) {
      float f[8];
#pragma unroll
      for (int k = 0; k < 8 / EPC; ++k) {
        const u32x4 x = *reinterpret_cast<const u32x4*>(sm_q + c * kQS + (G2 * QH + 8 * s2 + EPC * k) * (int)kIOB);
        if constexpr (sizeof(IO) == 4) {
#pragma unroll
          for (int e = 0; e < 4; ++e) f[4 * k + e] = __uint_as_float(x[e]);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            f[2 * e] = bf16_lo(x[e]);
            f[2 * e + 1] = bf16_hi(x[e]);
          }
        }
      }
      uint32_t wd[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) wd[e] = pack_bf16x2(f[2 * e] * qsc, f[2 * e + 1] * qsc);
      qb[s2] = __builtin_bit_cast(bf16x8, (u32x4{wd[0], wd[1], wd[2], wd[3]}));
    }
  } else {
    const IO* qp = static_cast<const IO*>(a.q) + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh +
                   (int64_t)(i < a.T ? i : 0) * a.q_st + G2 * QH;
#pragma unroll
    for (int s2 = 0; s2 < NQ; ++s2) {
      uint32_t wd[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        wd[e] = pack_bf16x2(Elem<IO>::load(qp + 8 * s2 + 2 * e) * qsc, Elem<IO>::load(qp + 8 * s2 + 2 * e + 1) * qsc);
      qb[s2] = __builtin_bit_cast(bf16x8, (u32x4{wd[0], wd[1], wd[2], wd[3]}));
    }
  }

  f32x16 oacc[DU];
#pragma unroll
  for (int u = 0; u < DU; ++u)
#pragma unroll
    for (int e = 0; e < 16; ++e) oacc[u][e] = 0.f;
  float m = kNegBig, l = 0.f;

  const uint16_t* kpool = static_cast<const uint16_t*>(a.k_pool);
  const uint16_t* vpool = static_cast<const uint16_t*>(a.v_pool);
  const uint32_t nblk = a.num_blocks < 0x7fffffff ? (uint32_t)a.num_blocks : 0x7fffffffu;
  auto ok_blk = [&](int e) { return (uint32_t)e < nblk; };

  auto kswz = [](int r) { return (r / RPB) & (CPR - 1); };
  auto vswz = [](int r) { return (4 * ((r / RPB) & 3)) & (CPR - 1); };
  uint32_t kdo[NDMA], vdo[NDMA];  // byte offsets of this lane's source chunk in its block
#pragma unroll
  for (int n = 0; n < NDMA; ++n) {
    const int r = n * RPI + lane / CPR;
    const int p = lane % CPR;
    kdo[n] = (uint32_t)(2 * ((r & 15) * HD + 8 * (p ^ kswz(r))));
    vdo[n] = (uint32_t)(2 * ((r & 15) * HD + 8 * (p ^ vswz(r))));
  }
  const int kx = kswz(c);
  const int vr4 = (c & 15) >> 2;
  const int vx = vswz(4 * G2 + vr4);
  auto v_off = [&](int d) {
    const int hd = 32 * d + 16 * (c >> 4) + 4 * (c & 3);
    return (4 * G2 + vr4) * HD + 8 * ((hd >> 3) ^ vx) + (hd & 4);
  };
  unsigned char* ring = smem + w * kWaveB;
  typedef short s16x4 __attribute__((ext_vector_type(4)));

  // This wavefront's steps st = w + NW * k, in chunks of 32 steps: lane 2k + j holds the page-table
  // entry of block j of the chunk's step k (-1 past the request's blocks).
  for (int k0 = 0; k0 < mine; k0 += kWave / 2) {
    const int cnt = (mine - k0) < kWave / 2 ? (mine - k0) : kWave / 2;
    int ent = -1;
    {
      const int blk = 2 * (w + NW * (k0 + lane / 2)) + (lane & 1);
      if (lane < 2 * cnt && blk < nb) ent = k0 == 0 ? ent0 : pt[blk];
    }
    // A walk of one chunk starts at the tile's index modulo its step count, so the tiles of a
    // (request, head) pair (on one die) ask for different steps first and meet the rest in L2.
    const int rot = (mine <= kWave / 2 && cnt > 1) ? qt % cnt : 0;
    auto rk = [&](int k) { const int r = k + rot; return r < cnt ? r : r - cnt; };
    auto issue = [&](int stg, int k) {
      const int kr = rk(k);
      const int e0 = __builtin_amdgcn_readlane(ent, 2 * kr), e1 = __builtin_amdgcn_readlane(ent, 2 * kr + 1);
      const uint16_t* kb0 = kpool + ((int64_t)(ok_blk(e0) ? e0 : 0) * a.H + h) * (16 * HD);
      const uint16_t* kb1 = kpool + ((int64_t)(ok_blk(e1) ? e1 : 0) * a.H + h) * (16 * HD);
      const uint16_t* vb0 = vpool + ((int64_t)(ok_blk(e0) ? e0 : 0) * a.H + h) * (16 * HD);
      const uint16_t* vb1 = vpool + ((int64_t)(ok_blk(e1) ? e1 : 0) * a.H + h) * (16 * HD);
      unsigned char* dk = ring + stg * 4 * TILE;
      unsigned char* dv = dk + 2 * TILE;
#pragma unroll
      for (int n = 0; n < NDMA; ++n) {
        const bool second = n * RPI >= 16;
        lds_direct_load16(second ? kb1 : kb0, kdo[n], dk + n * 1024);
        lds_direct_load16(second ? vb1 : vb0, vdo[n], dv + n * 1024);
      }
    };
    issue(0, 0);
    for (int k = 0; k < cnt; ++k) {
      if (k + 1 < cnt) {
        lds_read_wait();  // the stage refilled now was read in step k - 1
        issue((k + 1) & 1, k + 1);
        vm_wait<2 * NDMA>();
      } else {
        vm_wait<0>();
      }
      const uint16_t* skx = reinterpret_cast<const uint16_t*>(ring + (k & 1) * 4 * TILE);
      const uint16_t* svx = skx + TILE;
      const int kr = rk(k);
      const int st = w + NW * (k0 + kr);
      const int e0 = __builtin_amdgcn_readlane(ent, 2 * kr), e1 = __builtin_amdgcn_readlane(ent, 2 * kr + 1);
      // ---- S^T = K Q^T ---------------------------------------------------------------------------
      f32x16 sacc;
#pragma unroll
      for (int e = 0; e < 16; ++e) sacc[e] = 0.f;
#pragma unroll
      for (int s2 = 0; s2 < NQ; ++s2) {
        const bf16x8 kf = *reinterpret_cast<const bf16x8*>(skx + c * HD + 8 * ((G2 * (CPR / 2) + s2) ^ kx));
        sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qb[s2], sacc, 0, 0, 0);
      }
      // ---- online softmax (keys st*32 + 8j + 4*G2 + r of this step), in place ---------------------
      const bool ok0 = ok_blk(e0), ok1 = ok_blk(e1);
      const bool full = ok0 && ok1 && __builtin_amdgcn_ballot_w64(n_c < (st + 1) * KS) == 0;
      if (!full) {
        const int t0 = st * KS + 4 * G2;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const bool okb = j < 2 ? ok0 : ok1;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int t = t0 + 8 * j + r;
            sacc[4 * j + r] = (okb && t < n_c) ? sacc[4 * j + r] : -INFINITY;
          }
        }
      }
      float mloc = -INFINITY;
#pragma unroll
      for (int e = 0; e < 16; ++e) mloc = fmaxf(mloc, sacc[e]);
      mloc = max_xor32(mloc);
      const bool grow = mloc > m + kRescaleSlack;
      if (__builtin_amdgcn_ballot_w64(grow) != 0) {
        const float mnew = grow ? mloc : m;
        const float alpha = fast_exp2(m - mnew);
        l *= alpha;
#pragma unroll
        for (int u = 0; u < DU; ++u) oacc[u] *= alpha;
        m = mnew;
      }
      float ps = 0.f;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        sacc[e] = fast_exp2(sacc[e] - m);
        ps += sacc[e];
      }
      l += sum_xor32(ps);
      // ---- O^T += V^T P^T ------------------------------------------------------------------------
#pragma unroll
      for (int mm = 0; mm < 2; ++mm) {
        uint32_t pw[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) pw[q] = pack_bf16x2(sacc[8 * mm + 2 * q], sacc[8 * mm + 2 * q + 1]);
        const bf16x8 pb = __builtin_bit_cast(bf16x8, (u32x4{pw[0], pw[1], pw[2], pw[3]}));
#pragma unroll
        for (int d = 0; d < DU; ++d) {
          const uint16_t* vp = svx + v_off(d) + 16 * mm * HD;
          const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(vp));
          const s16x4 hi =
              __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(vp + 8 * HD));
          const bf16x8 vf = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
          oacc[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pb, oacc[d], 0, 0, 0);
        }
      }
    }
  }

  // ---- merge: lane (G2, c) holds O[query c][32d + 8j + 4*G2 + r] in oacc[d][4j + r] --------------
  float* mrow = reinterpret_cast<float*>(ring) + c * kOS;
#pragma unroll
  for (int d = 0; d < DU; ++d)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      *reinterpret_cast<f32x4*>(mrow + 32 * d + 8 * j + 4 * G2) =
          f32x4{oacc[d][4 * j], oacc[d][4 * j + 1], oacc[d][4 * j + 2], oacc[d][4 * j + 3]};
  if (G2 == 0) {
    sm_m[w][c] = m;
    sm_l[w][c] = l;
  }
  __syncthreads();
  const int row = threadIdx.x / TPR;
  const int d0 = (threadIdx.x % TPR) * VPT;
  if (i0 + row < a.T) {
    float M = kNegBig;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) M = fmaxf(M, sm_m[ww][row]);
    float lsum = 0.f, A[VPT];
#pragma unroll
    for (int e = 0; e < VPT; ++e) A[e] = 0.f;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) {
      const float f = fast_exp2(sm_m[ww][row] - M);
      lsum = fmaf(sm_l[ww][row], f, lsum);
      const float* src = reinterpret_cast<const float*>(smem + ww * kWaveB) + row * kOS + d0;
#pragma unroll
      for (int t4 = 0; t4 < VPT / 4; ++t4) {
        const f32x4 o = *reinterpret_cast<const f32x4*>(src + 4 * t4);
#pragma unroll
        for (int e = 0; e < 4; ++e) A[4 * t4 + e] = fmaf(o[e], f, A[4 * t4 + e]);
      }
    }
    IO* op = static_cast<IO*>(a.out) + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh + (int64_t)(i0 + row) * a.o_st + d0;
    const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
#pragma unroll
    for (int e = 0; e < VPT; ++e) Elem<IO>::store(op + e, lsum > 0.f ? A[e] * inv : 0.f);
  }
}

bool prefill_split_supported(int kv_dtype, int head_dim, int block_size) {
  return kv_dtype == PA_DTYPE_BF16 && block_size == 16 && head_dim == 64;
}

int64_t prefill_split_units(int32_t batch, int32_t num_heads, int32_t query_len) {
  return (int64_t)batch * num_heads * ((query_len + kSplitRows - 1) / kSplitRows);
}

int launch_prefill_split(const AttnArgs& a, int io_dtype, hipStream_t stream) {
  const int64_t units = prefill_split_units(a.B, a.H, a.T);
  if (units > 0x7fffffffLL) PA_FAIL(PA_ERR_INVALID_ARGUMENT, "grid too large");
  const dim3 grid((unsigned)units), block(kSplitWaves * kWave);
  if (io_dtype == PA_DTYPE_F32) prefill_split_kernel<float, 64><<<grid, block, 0, stream>>>(a);
  else prefill_split_kernel<uint16_t, 64><<<grid, block, 0, stream>>>(a);
  PA_CHECK_LAUNCH("split prefill kernel");
  return PA_OK;
}

bool prefill_wide_supported(int kv_dtype, int head_dim, int block_size) {
  return (kv_dtype == PA_DTYPE_BF16 || kv_dtype == PA_DTYPE_F32) && block_size == 16 &&
         (head_dim == 64 || head_dim == 128);
}

int64_t prefill_wide_units(int32_t batch, int32_t num_heads, int32_t query_len) {
  return (int64_t)batch * num_heads * ((query_len + kWideRows - 1) / kWideRows);
}

// Workgroups of the balanced kernel for `kv_dtype` and `head_dim` one compute unit holds at once
// (the smaller of its two output types), per device.
static int balanced_slots_per_cu(int kv_dtype, int head_dim) {
  constexpr int kMaxDevices = 64;
  static int cached[4][kMaxDevices] = {};
  const int kind = (kv_dtype == PA_DTYPE_F32 ? 1 : 0) + (head_dim == 64 ? 2 : 0);
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
  if (cached[kind][dev] == 0) {
    int nf = 0, nb = 0;
    hipError_t e1, e2;
    if (kind == 1) {
      e1 = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nf, prefill_wide_f32_kernel<float, 128, true>,
                                                        kWideWaves * kWave, 0);
      e2 = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, prefill_wide_f32_kernel<uint16_t, 128, true>,
                                                        kWideWaves * kWave, 0);
    } else if (kind == 3) {
      e1 = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nf, prefill_wide_f32_kernel<float, 64, true>,
                                                        kWideWaves * kWave, 0);
      e2 = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, prefill_wide_f32_kernel<uint16_t, 64, true>,
                                                        kWideWaves * kWave, 0);
    } else if (kind == 2) {
      e1 = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nf, prefill_wide_kernel<float, 64, kWideNsub64, 2, true>,
                                                        kWideWaves * kWave, 0);
      e2 = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, prefill_wide_kernel<uint16_t, 64, kWideNsub64, 2, true>,
                                                        kWideWaves * kWave, 0);
    } else {
      e1 = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nf, prefill_wide_kernel<float, 128, 1, 2, true>,
                                                        kWideWaves * kWave, 0);
      e2 = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, prefill_wide_kernel<uint16_t, 128, 1, 2, true>,
                                                        kWideWaves * kWave, 0);
    }
    if (e1 != hipSuccess || e2 != hipSuccess) nf = nb = 0;
    cached[kind][dev] = (nf < nb ? nf : nb) > 0 ? (nf < nb ? nf : nb) : -1;
  }
  return cached[kind][dev] > 0 ? cached[kind][dev] : 0;
}

int64_t prefill_balanced_grid(int32_t batch, int32_t num_heads, int32_t query_len, int32_t head_dim,
                              int32_t max_pages, int kv_dtype) {
  if ((head_dim != 128 && head_dim != 64) || batch < 1 || batch > 255 || num_heads < kXcds ||
      num_heads % kXcds != 0 || query_len < 1 || max_pages < 0)
    return 0;
  const int64_t ntiles = (query_len + kWideRows - 1) / kWideRows;
  const int64_t units = (int64_t)batch * num_heads * ntiles;
  if (units * (int64_t)sizeof(int32_t) > (int64_t)PA_PREFILL_COUNTER_BYTES) return 0;
  const int slots = balanced_slots_per_cu(kv_dtype, head_dim);
  // KV blocks per step: 32-key steps, except 64-key steps for bf16 KV at head_dim 64 (the same
  // products per query row as a 32-key step at 128).
  const int nbs = head_dim == 64 && kv_dtype == PA_DTYPE_BF16 ? 2 * kWideNsub64 : 2;
  const int64_t cus = pa_host::device_cu_count();
  // Where it pays (MI355X, head_dim 128, graph-free eager timings; default launch -> balanced):
  // few tiles over long contexts, where the default launch leaves CUs idle or each tile walks
  // hundreds of steps alone. bf16 KV: 1 x 32 heads, 512-token chunk over 8k 159 -> 96 us, over 3k
  // 81 -> 59 us; 2 x 32, 256-token chunks over 8k 208 -> 103 us; 1 x 32, 128-token chunk over 16k
  // 130 -> 86 us; it loses on short contexts (1 x 32, 128-token chunk over 4k 31 -> 38 us; 256
  // over 2k 28 -> 34 us) and on grids of two or more tiles per CU (8 x 32 heads, 512-token chunks:
  // 237 -> 250 us), and ties in between (256 tiles: 0 to -5%). fp32 KV (a step costs more, so
  // cutting pays sooner): 1 x 32, 512-token chunk over 8k 807 -> 574 us, over 1k 144 -> 126 us;
  // 256-token chunk over 2k 109 -> 105 us; 128-token chunk over 16k 356 -> 321 us, over 4k 92 ->
  // 108 us (loses). So: at most half a tile per CU and at least 8192 tile-steps (tiles x the
  // longest tile's 32-key steps, from the page table's width), 4096 for fp32 KV from a quarter
  // tile per CU; two workgroups per CU unless that cuts a tile more than 8 ways (then one).
  const int64_t steps = ((int64_t)max_pages + nbs - 1) / nbs;
  const int64_t min_steps = kv_dtype == PA_DTYPE_F32 && 4 * units >= cus ? 4096 : 8192;
  bool pays = 2 * units <= cus && units * steps >= min_steps;
  // Head_dim 64 (bf16 KV, 64-key steps: twice the softmax work per matrix product of a head_dim 128
  // step, and the split-step kernel as the alternative): 1 x 32 heads, 512-token chunk over 8k
  // 64.6 -> 56.9 us, 2 x 32, 256 over 8k 63.8 -> 57.3 us, 1 x 32, 128 over 16k 52.8 -> 46.8 us;
  // ties at 1 x 32, 512 over 4k (38.8 / 38.1) and 1 x 8, 512 over 8k (32.2 / 31.4); loses at
  // 1 x 16, 512 over 8k (33.1 -> 38.1), 4 x 8, 256 over 4k (19.3 -> 28.5) and 1 x 32, 512 over 2k
  // (25.1 -> 28.8). So at least 16384 tile-steps, or 256 steps (16k keys) per tile.
  if (head_dim == 64 && kv_dtype == PA_DTYPE_BF16) pays = 2 * units <= cus && (units * steps >= 16384 || steps >= 256);
  int per_cu = 4 * units >= cus ? 2 : 1;  // two per CU cut each tile into 2 cus / units pieces
  // Head_dim 64, fp32 KV (32-key steps; the alternative is the 16-row kernel, whose B * H *
  // ceil(T / 16) workgroups leave CUs idle when tiles are few): 1 x 8 heads, 128-token chunk over
  // 32k 369.6 -> 126.2 us, over 8k 94.5 -> 54.7 us (one workgroup per CU); 512 over 16k 209.2 ->
  // 173.3 us, 1 x 32, 128 over 16k 190.8 -> 169.8 us, 1 x 32, 512 over 8k 351.7 -> 307.1 us,
  // 2 x 32, 256 over 8k 354.1 -> 306.6 us (two per CU); ties at 1 x 16, 256 over 8k (98.0 / 98.2)
  // and 1 x 8, 512 over 8k (113.0 / 104.9); loses at 4 x 8, 256 over 4k (79.9 -> 97.1), 2 x 8,
  // 512 over 4k (83.7 -> 96.6), 1 x 32, 512 over 2k (99.6 -> 102.6) and 4 x 8, 256 over 768
  // (23.4 -> 33.9). Checked on further shapes: 1 x 8, 256 over 16k 187.6 -> 107.9 us, 2 x 8, 128
  // over 16k 186.2 -> 109.6 us, 1 x 8, 512 over 32k 371.0 -> 302.5 us, 2 x 16, 512 over 8k 340.0 ->
  // 307.5 us, 1 x 32, 512 over 4k 180.4 -> 171.6 us; but 1 x 32, 256 over 8k 151.1 -> 165.9 us and
  // 1 x 64, 128 over 8k 153.2 -> 176.7 us lose: there the 16-row kernel has two workgroups per
  // CU, its LDS-staged build at its best. So at least 16384 tile-steps unless the 16-row grid
  // holds one to two workgroups per CU, or 256 steps per tile at most one tile per 16 CUs; two
  // workgroups per CU from one tile per 8 CUs.
  if (head_dim == 64 && kv_dtype == PA_DTYPE_F32) {
    const int64_t rows16 = (int64_t)batch * num_heads * ((query_len + 15) / 16);
    const bool rows16_at_best = rows16 > cus && rows16 <= 2 * cus;
    pays = 2 * units <= cus &&
           ((units * steps >= 16384 && !rows16_at_best) || (steps >= 256 && 16 * units <= cus));
    per_cu = 8 * units >= cus ? 2 : 1;
  }
  if (!pays && units > 2 * cus) per_cu = slots;
  if (const char* env = getenv("PAGED_HIP_PREFILL_BALANCE")) {
    if (strcmp(env, "force") == 0) pays = true;
    if (strcmp(env, "off") == 0) pays = false;
  }
  if (!pays) return 0;
  if (const char* env = getenv("PAGED_HIP_BALANCED_PER_CU")) {
    const int v = atoi(env);
    if (v >= 1) per_cu = v;
  }
  per_cu = per_cu < slots ? per_cu : slots;
  const int64_t gangs = (int64_t)per_cu * cus / (kXcds * ntiles);
  if (gangs < 1) return 0;
  // The kernel's list positions are int: a die's work W (steps of at most max_pages / nbs + 1 per
  // pair, at least 1) stays below 2^31 / 64; its share table holds gangs + 1 entries.
  const int64_t w = (int64_t)(num_heads / kXcds) * batch * ((int64_t)max_pages / nbs + 1);
  if (w >= (0x7fffffffLL >> 6) || gangs + 1 > kWideWaves * kWave) return 0;
  return gangs * kXcds * ntiles;
}

size_t prefill_balanced_record_bytes(int64_t grid, int32_t head_dim) {
  return (size_t)grid * 2 * (head_dim == 64 ? kWideRecFloats<64> : kWideRecFloats<128>) * sizeof(float);
}

int launch_prefill_wide(const AttnArgs& a, int io_dtype, int kv_dtype, hipStream_t stream) {
  const int64_t units = prefill_wide_units(a.B, a.H, a.T);
  if (units > 0x7fffffffLL) PA_FAIL(PA_ERR_INVALID_ARGUMENT, "grid too large");
  const dim3 block(kWideWaves * kWave);
  if (a.counters != nullptr) {
    // Balanced launch: the caller checked prefill_balanced_grid > 0 and sized the workspace.
    const int64_t g = prefill_balanced_grid(a.B, a.H, a.T, a.head_dim, a.max_pages, kv_dtype);
    if (g <= 0) PA_FAIL(PA_ERR_INVALID_ARGUMENT, "balanced prefill does not apply");
    const dim3 grid((unsigned)g);
    AttnArgs ab = a;
    ab.die_cus = pa_host::device_cu_count() / kXcds > 0 ? pa_host::device_cu_count() / kXcds : 1;
    if (kv_dtype == PA_DTYPE_F32 && a.head_dim == 64) {
      if (io_dtype == PA_DTYPE_F32) prefill_wide_f32_kernel<float, 64, true><<<grid, block, 0, stream>>>(ab);
      else prefill_wide_f32_kernel<uint16_t, 64, true><<<grid, block, 0, stream>>>(ab);
    } else if (kv_dtype == PA_DTYPE_F32) {
      if (io_dtype == PA_DTYPE_F32) prefill_wide_f32_kernel<float, 128, true><<<grid, block, 0, stream>>>(ab);
      else prefill_wide_f32_kernel<uint16_t, 128, true><<<grid, block, 0, stream>>>(ab);
    } else if (a.head_dim == 64) {
      if (io_dtype == PA_DTYPE_F32) prefill_wide_kernel<float, 64, kWideNsub64, 2, true><<<grid, block, 0, stream>>>(ab);
      else prefill_wide_kernel<uint16_t, 64, kWideNsub64, 2, true><<<grid, block, 0, stream>>>(ab);
    } else if (io_dtype == PA_DTYPE_F32) {
      prefill_wide_kernel<float, 128, 1, 2, true><<<grid, block, 0, stream>>>(ab);
    } else {
      prefill_wide_kernel<uint16_t, 128, 1, 2, true><<<grid, block, 0, stream>>>(ab);
    }
    PA_CHECK_LAUNCH("balanced wide prefill kernel");
    return PA_OK;
  }
  const dim3 grid((unsigned)units);
  if (kv_dtype == PA_DTYPE_F32) {
    if (io_dtype == PA_DTYPE_F32) {
      if (a.head_dim == 64) prefill_wide_f32_kernel<float, 64, false><<<grid, block, 0, stream>>>(a);
      else prefill_wide_f32_kernel<float, 128, false><<<grid, block, 0, stream>>>(a);
    } else {
      if (a.head_dim == 64) prefill_wide_f32_kernel<uint16_t, 64, false><<<grid, block, 0, stream>>>(a);
      else prefill_wide_f32_kernel<uint16_t, 128, false><<<grid, block, 0, stream>>>(a);
    }
  } else if (io_dtype == PA_DTYPE_F32) {
    if (a.head_dim == 64) prefill_wide_kernel<float, 64, kWideNsub64, kWideStages64, false><<<grid, block, 0, stream>>>(a);
    else if (wide128_pair(units)) prefill_wide_kernel<float, 128, 2, 2, false><<<grid, block, 0, stream>>>(a);
    else prefill_wide_kernel<float, 128, 1, 2, false><<<grid, block, 0, stream>>>(a);
  } else {
    if (a.head_dim == 64) prefill_wide_kernel<uint16_t, 64, kWideNsub64, kWideStages64, false><<<grid, block, 0, stream>>>(a);
    else if (wide128_pair(units)) prefill_wide_kernel<uint16_t, 128, 2, 2, false><<<grid, block, 0, stream>>>(a);
    else prefill_wide_kernel<uint16_t, 128, 1, 2, false><<<grid, block, 0, stream>>>(a);
  }
  PA_CHECK_LAUNCH("wide prefill kernel");
  return PA_OK;
}

}  // namespace pa
