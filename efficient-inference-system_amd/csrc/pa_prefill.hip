// Chunked causal prefill attention over paged KV for gfx950, on matrix cores.
//
// Work unit = (request, head, tile of 16 query rows). One workgroup of 4 wavefronts per unit and
// KV split; the wavefronts take the split's KV blocks round-robin and
// merge their online-softmax states in LDS at the end. For each 16-token KV block a wavefront
// computes the transposed score tile S^T = K Q^T (16 keys x 16 queries) and accumulates the
// transposed output O^T += V^T P^T.
// With the 16x16 MFMA output layout (lane = 16*G + c holds rows 4G..4G+3 of column c), lane
// (G, c) then owns query c's scores for keys 4G..4G+3, its output column, and its softmax state:
//   - the row max / row sum over keys is a few registers plus two cross-group permlane swaps;
//   - the score registers ARE the B operand (P^T) of the next product, with no data movement;
//   - rescaling the output by the new running max is a per-lane scalar.
// The contraction index of each product is permuted so that every lane reads contiguous 16-byte
// vectors: the QK^T contraction slot (G, s) is head_dim index G*HD/4 + s, the PV slot (G, i) is
// key 4G + i, and output tile t, row r holds head_dim index r*HD/16 + t. A and B use the same
// slot->index map, so the products are exact regardless of the hardware's k ordering.
// fp32 KV uses v_mfma_f32_16x16x4_f32 (fp32 products, like the reference). bf16 KV uses
// v_mfma_f32_16x16x32_bf16 for QK^T (q rounded to bf16) and v_mfma_f32_16x16x16_bf16 for PV
// (softmax weights rounded to bf16), accumulating in fp32.
//
// KV staging. The K operand puts key row c on lane c, so a load straight into the operand
// registers has every 4-lane group of an instruction touching 4 cache lines; the compute unit's L1
// serves one line per lane group per access, which made the walk L1-bound with bf16 KV. At
// head_dim 64 (and 128 with bf16 KV) each wavefront instead copies its blocks' K and V slabs into
// its own two-stage LDS ring with LDS-direct loads, which read the contiguous slab 16 bytes per
// lane (one line per lane group), and reads the operands from LDS (prefill_stage_in_lds picks the
// staging per launch).
//
// Split-K: when num_splits > 1 each unit's KV blocks are cut into ranges of split_blocks blocks,
// one workgroup per range. Work items are ordered split-major, so the grid holds many
// equal-sized items instead of a few long ones. A unit with one active split writes its output
// directly; otherwise each split writes its (m, l, acc) rows to the workspace and
// prefill_merge_kernel combines them. (A same-launch merge by the last split to finish needs
// agent-scope fences, which write back the die-local L2 in every workgroup: slower on MI355X than
// the second launch.)
#include <stdlib.h>
#include <string.h>

#include <type_traits>

#include "pa_attention.h"

namespace pa {

// Work unit -> ((request, head) pair, 16-row query tile). The tiles of one pair read the same KV
// blocks, and workgroup x runs on die x % kXcds, each die with its own L2. When the pairs divide
// evenly over the dies, pair p's tiles all go to die p % kXcds, so each die's L2 holds only its
// pairs' KV. Within a die, its i-th workgroup and the one half a die's worth later share a compute
// unit under round-robin dispatch: the first half of the die's pairs walks its tiles from the last
// (heaviest) one, the second half from the first, so a heavy tile pairs with a light one.
// Otherwise units stay pair-major with the same descending / ascending halves over all pairs.
__device__ __forceinline__ void prefill_unit(int unit, int ntiles, int pairs, int& bh, int& qt) {
  int y = unit, lanes = 1, lane = 0;
  if (pairs % kXcds == 0) {
    lanes = kXcds;
    lane = unit % kXcds;
    y = unit / kXcds;
  }
  const int npl = pairs / lanes;  // pairs per die (or all pairs)
  const int lp = y / ntiles;
  const int slot = y - lp * ntiles;
  bh = lp * lanes + lane;
  qt = lp >= npl / 2 ? slot : ntiles - 1 - slot;
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

// Load NW 32-bit words (NW in {2, 4, 8, ...}) from a 8- or 16-byte aligned address.
template <int NWORDS>
__device__ __forceinline__ void load_words(const void* p, uint32_t (&w)[NWORDS]) {
  if constexpr (NWORDS % 4 == 0) {
    const u32x4* v = static_cast<const u32x4*>(p);
#pragma unroll
    for (int k = 0; k < NWORDS / 4; ++k) {
      const u32x4 x = v[k];
      w[4 * k + 0] = x[0]; w[4 * k + 1] = x[1]; w[4 * k + 2] = x[2]; w[4 * k + 3] = x[3];
    }
  } else {
    static_assert(NWORDS == 2, "word count");
    const u32x2 x = *static_cast<const u32x2*>(p);
    w[0] = x[0]; w[1] = x[1];
  }
}

template <typename KV, int HD>
struct PrefillShape {
  static constexpr bool kBf16 = std::is_same<KV, uint16_t>::value;
  static constexpr int QD = HD / 4;              // head_dim values per lane in the QK^T operands
  static constexpr int DT = HD / 16;             // output tiles of 16 head_dim columns
  static constexpr int KW = kBf16 ? QD / 2 : QD;  // 32-bit words of K per lane per block
  static constexpr int VW = kBf16 ? DT / 2 : DT;  // 32-bit words per V row per lane per block
};

// Wavefronts per workgroup of the 16-row kernel (they split each tile's KV blocks): four, two per
// SIMD at the kernel's register use. More wavefronts per tile lengthen the merge and leave fewer
// workgroups per CU, which measured slower for both KV types.
#ifndef PA_PREFILL_WAVES_F32
#define PA_PREFILL_WAVES_F32 4
#endif
#ifndef PA_PREFILL_WAVES_BF16
#define PA_PREFILL_WAVES_BF16 4
#endif
template <typename KV>
constexpr int prefill_waves() { return std::is_same<KV, float>::value ? PA_PREFILL_WAVES_F32 : PA_PREFILL_WAVES_BF16; }

// KV tiles each wavefront keeps in flight ahead of the one it folds: one, except two for bf16 KV
// at head_dim 128. More costs registers (a wavefront per SIMD) without hiding more latency.
#ifndef PA_PREFILL_DEPTH_F32_64
#define PA_PREFILL_DEPTH_F32_64 1
#endif
#ifndef PA_PREFILL_DEPTH_F32_128
#define PA_PREFILL_DEPTH_F32_128 1
#endif
#ifndef PA_PREFILL_DEPTH_BF16_64
#define PA_PREFILL_DEPTH_BF16_64 1
#endif
#ifndef PA_PREFILL_DEPTH_BF16_128
#define PA_PREFILL_DEPTH_BF16_128 2
#endif
// KV blocks folded per softmax round: one. Two per round (interleaved QK^T chains, one max / sum
// exchange and rescale test per 32 keys) costs more registers than it saves and does not fit two
// wavefronts per SIMD at head_dim 128. The walk is bound neither by the matrix cores (bf16 KV has
// 1/16 of fp32's MFMA time and is not 16x faster) nor by its instruction count; with K loaded
// straight into the operand registers (key row per lane, four cache lines per 4-lane group) it
// is bound by the compute unit's L1, which the LDS staging of prefill_stage_in_lds removes.
template <typename KV, int HD, bool OCC4>
constexpr int prefill_round() { return 1; }

// Lazy rescaling threshold (log2 units) of the 16-row kernel's running max.
constexpr float kPrefillRescaleSlack = 8.f;

template <typename KV, int HD>
constexpr int prefill_depth() {
  return std::is_same<KV, float>::value ? (HD == 64 ? PA_PREFILL_DEPTH_F32_64 : PA_PREFILL_DEPTH_F32_128)
                                        : (HD == 64 ? PA_PREFILL_DEPTH_BF16_64 : PA_PREFILL_DEPTH_BF16_128);
}

// OCC4: registers capped at 128 so that 4 wavefronts share a SIMD (4 workgroups per CU instead of
// 3). Only fp32 KV at head_dim 64 is near the cap; the launch takes the capped build when the grid
// would not fit on the GPU at 3 workgroups per CU, and the unconstrained one otherwise.
template <typename KV, typename IO, int HD, bool OCC4 = false, bool LDSK = false>
__global__ __launch_bounds__(prefill_waves<KV>() * kWave) __attribute__((amdgpu_waves_per_eu(OCC4 ? 4 : 1)))
void prefill_mfma_kernel(const AttnArgs a) {
  constexpr int BS = 16;
  constexpr int NW = prefill_waves<KV>();
  using Sh = PrefillShape<KV, HD>;
  constexpr int QD = Sh::QD, DT = Sh::DT, KW = Sh::KW, VW = Sh::VW;
  constexpr bool kBf16 = Sh::kBf16;

  // Per wavefront: its merge rows (16 x (HD + 4) floats: 16-byte aligned rows whose stride is one
  // 16-byte bank group past a multiple of 128 bytes, so 8 consecutive rows of a 16-byte access
  // hit distinct banks) and, with LDSK, a two-stage ring of (K slab, V slab) the merge rows reuse
  // after the walk.
  constexpr int kRowB = HD * (int)sizeof(KV);  // bytes of one key row
  constexpr int kSlab = BS * kRowB;            // bytes of one (block, head) K or V slab
  constexpr int kOS = HD + 4;                  // floats per merge row
  constexpr int kOB = 16 * kOS * 4;
  constexpr int kWaveB = LDSK ? (4 * kSlab > kOB ? 4 * kSlab : kOB) : kOB;
  constexpr int TPC = NW * kWave / 16;  // merge: threads per query column
  constexpr int VPT = HD / TPC;         // merge: consecutive head_dim values per thread
  static_assert(HD % TPC == 0 && (VPT == 2 || VPT % 4 == 0), "merge: whole 8- or 16-byte pieces per thread");
  __shared__ __attribute__((aligned(16))) unsigned char smem[NW * kWaveB];
  __shared__ float sm_m[NW][16];
  __shared__ float sm_l[NW][16];
  auto sm_o = [&](int ww, int cc) -> float* { return reinterpret_cast<float*>(smem + ww * kWaveB) + cc * kOS; };

  const int lane = threadIdx.x & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int G = lane >> 4;
  const int c = lane & 15;

  // Work item: split-major, then (request, head), then query tiles from the last (heaviest) one.
  const int ntiles = (a.T + 15) / 16;
  const int units = a.B * a.H * ntiles;
  const int split = blockIdx.x / units;
  const int unit = blockIdx.x - split * units;
  int bh, qt;
  prefill_unit(unit, ntiles, a.B * a.H, bh, qt);
  const int h = bh % a.H;
  const int b = bh / a.H;
  const int i0 = qt * 16;
  const int i = i0 + c;

  // The first chunk of this wave's page-table entries (blocks jb0 + w + lane * NW) does not depend
  // on the request's lengths: load it now, clamped into the row, so it travels with the length
  // loads instead of after them (one dependent memory round trip less before the first KV tile).
  // Entries past the tile's blocks are never used.
  const int32_t* pt = a.page_table + (int64_t)b * a.pt_stride;
  const int jb0 = a.num_splits > 1 ? split * a.split_blocks : 0;
  int ids0 = -1;
  if (a.max_pages > 0) {
    const int idx = jb0 + w + lane * NW;
    ids0 = pt[idx < a.max_pages ? idx : a.max_pages - 1];
  }
  const int L = a.seq_lens[b];
  const int C = a.cur_lens[b];
  const int n_c = i < a.T ? valid_keys(L, C, i) : 0;
  const int i_last = (i0 + 15) < (a.T - 1) ? (i0 + 15) : (a.T - 1);
  const int n_max = valid_keys(L, C, i_last);  // nondecreasing in the row index
  int nb = (n_max + BS - 1) / BS;
  nb = nb < a.max_pages ? nb : a.max_pages;
  int jb = 0, je = nb, nact = 1;
  if (a.num_splits > 1) {
    nact = nb > 0 ? (nb + a.split_blocks - 1) / a.split_blocks : 1;
    if (split >= nact) return;  // uniform over the workgroup, before any barrier
    jb = split * a.split_blocks;
    je = jb + a.split_blocks < nb ? jb + a.split_blocks : nb;
  }

  // Q operand: row i, head_dim [G*QD, G*QD + QD), pre-scaled into the log2 domain.
  float qv[QD];
  {
    const IO* qp = static_cast<const IO*>(a.q) + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh +
                   (int64_t)(i < a.T ? i : 0) * a.q_st + G * QD;
    // The row index is clamped in bounds, so load unconditionally and zero rows past T after.
    const float qscale = i < a.T ? a.scale_log2 : 0.f;
#pragma unroll
    for (int s = 0; s < QD; ++s) qv[s] = Elem<IO>::load(qp + s) * qscale;
  }
  bf16x8 qb[kBf16 ? QD / 8 : 1];
  if constexpr (kBf16) {
#pragma unroll
    for (int s = 0; s < QD / 8; ++s) {
      uint32_t wd[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        wd[e] = (uint32_t)f32_to_bf16(qv[8 * s + 2 * e]) | ((uint32_t)f32_to_bf16(qv[8 * s + 2 * e + 1]) << 16);
      const u32x4 x = {wd[0], wd[1], wd[2], wd[3]};
      qb[s] = __builtin_bit_cast(bf16x8, x);
    }
  }

  f32x4 oacc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) oacc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = kNegBig, l = 0.f;

  const KV* kpool = static_cast<const KV*>(a.k_pool);
  const KV* vpool = static_cast<const KV*>(a.v_pool);

  // Registers of one KV tile as this lane needs them: K row c, head_dim [G*QD, G*QD + QD), and
  // V rows 4G..4G+3, head_dim [c*DT, c*DT + DT).
  struct Tile {
    uint32_t k[KW];
    uint32_t v[4][VW];
    bool ok;
  };
  auto issue = [&](Tile& t, int64_t base, bool ok) {
    t.ok = ok;
    load_words<KW>(kpool + base + c * HD + G * QD, t.k);
#pragma unroll
    for (int r = 0; r < 4; ++r) load_words<VW>(vpool + base + (4 * G + r) * HD + c * DT, t.v[r]);
  };

  // Fold NV tiles (this wave's blocks k0 .. k0 + NV - 1 of the current chunk) into the running
  // state with one softmax round: the QK^T chains of the tiles interleave (independent
  // accumulators), and the row max / sum exchanges and the rescale test are paid once per round.
  // The running max moves lazily (only when a round's max exceeds it by more than
  // kPrefillRescaleSlack in log2 units, tested for the whole wavefront), so the output
  // accumulators are rescaled only in the rounds where it jumps; weights stay <= 2^slack.
  auto fold_round = [&](const Tile* tr, auto nv_tag, int j0, int jstep) {
    constexpr int NV = decltype(nv_tag)::value;
    // ---- S^T = K Q^T ------------------------------------------------------------------------
    f32x4 sacc[NV];
#pragma unroll
    for (int q = 0; q < NV; ++q) sacc[q] = f32x4{0.f, 0.f, 0.f, 0.f};
    if constexpr (!kBf16) {
#pragma unroll
      for (int s2 = 0; s2 < QD; ++s2)
#pragma unroll
        for (int q = 0; q < NV; ++q)
          sacc[q] = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(tr[q].k[s2]), qv[s2], sacc[q], 0, 0, 0);
    } else {
#pragma unroll
      for (int s2 = 0; s2 < QD / 8; ++s2)
#pragma unroll
        for (int q = 0; q < NV; ++q) {
          const u32x4 x = {tr[q].k[4 * s2], tr[q].k[4 * s2 + 1], tr[q].k[4 * s2 + 2], tr[q].k[4 * s2 + 3]};
          sacc[q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, x), qb[s2], sacc[q], 0, 0, 0);
        }
    }
    // ---- online softmax over the round's keys, per query column c ---------------------------
    // Interior rounds (every block valid, every key below every column's limit) need no mask.
    bool all_ok = true;
#pragma unroll
    for (int q = 0; q < NV; ++q) all_ok = all_ok && tr[q].ok;
    const int j_last = j0 + (NV - 1) * jstep;
    const bool full = all_ok && __builtin_amdgcn_ballot_w64(n_c < (j_last + 1) * BS) == 0;
    if (!full) {
#pragma unroll
      for (int q = 0; q < NV; ++q)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = (j0 + q * jstep) * BS + 4 * G + r;
          sacc[q][r] = (tr[q].ok && t < n_c) ? sacc[q][r] : -INFINITY;
        }
    }
    // A column's max over the round can pass m + slack only where one of its four lanes' partial
    // maxima does, so the cross-lane reduction and the rescale run only in the rounds where some
    // lane's partial max passes (same results as reducing every round).
    float mloc = -INFINITY;
#pragma unroll
    for (int q = 0; q < NV; ++q)
#pragma unroll
      for (int r = 0; r < 4; ++r) mloc = fmaxf(mloc, sacc[q][r]);
    if (__builtin_amdgcn_ballot_w64(mloc > m + kPrefillRescaleSlack) != 0) {
      const float mcol = max_xor32(max_xor16(mloc));
      const float mnew = mcol > m + kPrefillRescaleSlack ? mcol : m;
      const float alpha = fast_exp2(m - mnew);
      l *= alpha;
#pragma unroll
      for (int t = 0; t < DT; ++t) oacc[t] *= alpha;
      m = mnew;
    }
    // l is this lane's part of the row sum (its four keys of every round); the four lanes of a
    // column are summed once, after the walk.
#pragma unroll
    for (int q = 0; q < NV; ++q)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sacc[q][r] = fast_exp2(sacc[q][r] - m);
        l += sacc[q][r];
      }
    // ---- O^T += V^T P^T -----------------------------------------------------------------------
    // fp32 KV at head_dim 128: the PV MFMAs run at raised wavefront priority, so a wavefront that
    // reaches them issues ahead of co-resident ones still in their softmax (faster there; no
    // change at head_dim 64 or for bf16 KV, where it stays off).
    constexpr bool kPrio = !kBf16 && HD == 128;
    if constexpr (kPrio) __builtin_amdgcn_s_setprio(1);
    if constexpr (!kBf16) {
#pragma unroll
      for (int q = 0; q < NV; ++q)
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int t = 0; t < DT; ++t)
            oacc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(tr[q].v[r][t]), sacc[q][r], oacc[t], 0, 0,
                                                           0);
    } else {
#pragma unroll
      for (int q = 0; q < NV; ++q) {
        const uint32_t p01 = pack_bf16x2(sacc[q][0], sacc[q][1]);
        const uint32_t p23 = pack_bf16x2(sacc[q][2], sacc[q][3]);
        const s16x4 pb = {(short)(p01 & 0xffff), (short)(p01 >> 16), (short)(p23 & 0xffff), (short)(p23 >> 16)};
#pragma unroll
        for (int t = 0; t < DT; ++t) {
          const int sh = (t & 1) * 16;
          const s16x4 av = {(short)(tr[q].v[0][t >> 1] >> sh), (short)(tr[q].v[1][t >> 1] >> sh),
                            (short)(tr[q].v[2][t >> 1] >> sh), (short)(tr[q].v[3][t >> 1] >> sh)};
          oacc[t] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(av, pb, oacc[t], 0, 0, 0);
        }
      }
    }
    if constexpr (kPrio) __builtin_amdgcn_s_setprio(0);
  };

  // This wave's blocks j = jb + w + k*NW, k < mine, in chunks of one page-table entry per lane,
  // folded R blocks per round (the last round of the walk may hold fewer). D rounds load into a
  // ring of D + 1 register sets while the oldest one is folded; the steady-state loop issues its
  // loads unconditionally so the compiler's wait counts stay exact, and the tail is peeled.
  const int span = je - jb;
  const int mine = span > w ? (span - w + NW - 1) / NW : 0;
  constexpr int R = prefill_round<KV, HD, OCC4>();  // KV blocks per softmax round
  constexpr int D = prefill_depth<KV, HD>();  // rounds in flight ahead of the one being folded
  constexpr int S = D + 1;                    // register sets of R tiles
  static_assert(kWave % R == 0, "a page-table chunk holds whole rounds");
  using Full = std::integral_constant<int, R>;
  using One = std::integral_constant<int, 1>;
  if constexpr (LDSK) {
    // KV through LDS: each block's K and V slabs are copied into the wavefront's ring with
    // LDS-direct loads (each instruction copies 1 KB of the contiguous slab, so every 4 lanes read
    // one cache line), then read in the operand layouts. K rows are stored with their 16-byte
    // chunks XOR-swizzled by row so that the 16 rows of an operand read hit every bank once; bf16
    // V rows r and r ^ 1 trade places in every other group of four, so that the two lane groups of
    // a 64-bit read pass land in different bank halves. The loads are untracked by the compiler:
    // the walk waits for them itself (vmcnt), one block ahead.
    static_assert(R == 1 && kRowB <= 256, "LDS staging: one block per round, key rows of at most 256 bytes");
    constexpr int CPR = kRowB / 16;        // 16-byte chunks per row
    constexpr int RPB = 256 / kRowB;       // rows per 256 bytes (one pass over the banks)
    constexpr int NI = kSlab / (16 * kWave);  // LDS-direct instructions per slab
    auto ksw = [](int r) { return (r / RPB) & (CPR - 1); };
    auto vpos = [](int r) { return kRowB == 128 ? (r ^ ((r >> 2) & 1)) : r; };  // an involution
    uint32_t kso[NI], vso[NI];
#pragma unroll
    for (int n = 0; n < NI; ++n) {
      const int sl = n * kWave + lane;  // the LDS chunk this lane fills
      const int r = sl / CPR, p = sl % CPR;
      kso[n] = (uint32_t)(r * kRowB + 16 * (p ^ ksw(r)));
      vso[n] = (uint32_t)(vpos(r) * kRowB + 16 * p);
    }
    unsigned char* ring = smem + w * kWaveB;
    for (int c0 = 0; c0 < mine; c0 += kWave) {
      const int cnt = (mine - c0) < kWave ? (mine - c0) : kWave;
      int ids = -1;
      if (lane < cnt) ids = c0 == 0 ? ids0 : pt[jb + w + (c0 + lane) * NW];
      const bool okl = ids >= 0 && ids < a.num_blocks;
      const uint64_t okmask = __builtin_amdgcn_ballot_w64(okl);
      const int64_t offl = ((int64_t)(okl ? ids : 0) * a.H + h) * (BS * HD);
      auto stage_issue = [&](int st, int k) {
        const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)offl, k);
        const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)((uint64_t)offl >> 32), k);
        const int64_t off = (int64_t)(((uint64_t)hi << 32) | lo);
        unsigned char* dst = ring + st * 2 * kSlab;
#pragma unroll
        for (int n = 0; n < NI; ++n) stage_load16(kpool + off, kso[n], dst + n * 16 * kWave);
#pragma unroll
        for (int n = 0; n < NI; ++n) stage_load16(vpool + off, vso[n], dst + kSlab + n * 16 * kWave);
      };
      stage_issue(0, 0);
      for (int k = 0; k < cnt; ++k) {
        const int st = k & 1;
        if (k + 1 < cnt) {
          lds_read_wait();  // the stage refilled now was read in step k - 1
          stage_issue(st ^ 1, k + 1);
          vm_wait<2 * NI>();
        } else {
          vm_wait<0>();
        }
        const unsigned char* sb = ring + st * 2 * kSlab;
        Tile tt;
        tt.ok = ((okmask >> k) & 1) != 0;
#pragma unroll
        for (int s2 = 0; s2 < KW / 4; ++s2) {  // K row c, head_dim chunks G * KW / 4 + s2
          const int q = G * (KW / 4) + s2;
          const u32x4 x = *reinterpret_cast<const u32x4*>(sb + c * kRowB + 16 * (q ^ ksw(c)));
#pragma unroll
          for (int e = 0; e < 4; ++e) tt.k[4 * s2 + e] = x[e];
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {  // V row 4G + r, head_dim [c * DT, c * DT + DT)
          const unsigned char* vp = sb + kSlab + vpos(4 * G + r) * kRowB + 4 * VW * c;
          if constexpr (VW == 2) {
            const u32x2 x = *reinterpret_cast<const u32x2*>(vp);
            tt.v[r][0] = x[0];
            tt.v[r][1] = x[1];
          } else {
            static_assert(VW == 4, "V words per lane");
            const u32x4 x = *reinterpret_cast<const u32x4*>(vp);
#pragma unroll
            for (int e = 0; e < 4; ++e) tt.v[r][e] = x[e];
          }
        }
        fold_round(&tt, One{}, jb + w + (c0 + k) * NW, NW);
      }
    }
  } else
  for (int c0 = 0; c0 < mine; c0 += kWave) {
    const int cnt = (mine - c0) < kWave ? (mine - c0) : kWave;
    const int nr = (cnt + R - 1) / R;
    int ids = -1;
    if (lane < cnt) ids = c0 == 0 ? ids0 : pt[jb + w + (c0 + lane) * NW];
    // Each lane turns its entry into the element offset of its (block, head) slab and a validity
    // bit once per chunk; a block then costs two lane reads. Entries outside the pool (and lanes
    // past the chunk) read slab (0, h) and are masked.
    const bool okl = ids >= 0 && ids < a.num_blocks;
    const uint64_t okmask = __builtin_amdgcn_ballot_w64(okl);
    const int64_t offl = ((int64_t)(okl ? ids : 0) * a.H + h) * (BS * HD);
    auto put = [&](Tile* tr, int rr) {
#pragma unroll
      for (int q = 0; q < R; ++q) {
        const int k = rr * R + q;  // < nr * R <= kWave; lanes past cnt hold -1
        const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)offl, k);
        const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)((uint64_t)offl >> 32), k);
        issue(tr[q], (int64_t)(((uint64_t)hi << 32) | lo), ((okmask >> k) & 1) != 0);
      }
    };
    auto fold = [&](const Tile* tr, int rr) {
      const int j0 = jb + w + (c0 + rr * R) * NW;
      if (R == 1 || rr * R + R <= cnt) fold_round(tr, Full{}, j0, NW);
      else fold_round(tr, One{}, j0, NW);  // the walk's last round holds a single block
    };
    Tile t[S][R];
#pragma unroll
    for (int d = 0; d < D; ++d)
      if (d < nr) put(t[d], d);
    int rr = 0;
    for (; rr + D + S - 1 < nr; rr += S) {
#pragma unroll
      for (int u = 0; u < S; ++u) {
        put(t[(u + D) % S], rr + u + D);
        fold(t[u], rr + u);
      }
    }
    // Drain: at most S + D - 1 rounds remain; rr % S == 0 here, so round rr + u sits in slot u % S.
#pragma unroll
    for (int u = 0; u < S + D - 1; ++u) {
      if (rr + u < nr) {
        if (rr + u + D < nr) put(t[(u + D) % S], rr + u + D);
        fold(t[u % S], rr + u);
      }
    }
  }

  // ---- merge the wavefronts' states ---------------------------------------------------------
  // Lane (G, c) holds head_dim d = (4G + r) * DT + t of query column c in oacc[t][r]: for each r
  // the DT values over t are consecutive, so they go to LDS as DT / 4 16-byte vectors. Then 16
  // threads per column combine the wavefronts' states, each over DT consecutive head_dim values,
  // in one pass, with vector LDS reads instead of a scalar read and max / exp chain per output.
  l = sum_xor32(sum_xor16(l));
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int t4 = 0; t4 < DT / 4; ++t4)
      *reinterpret_cast<f32x4*>(sm_o(w, c) + (4 * G + r) * DT + 4 * t4) =
          f32x4{oacc[4 * t4][r], oacc[4 * t4 + 1][r], oacc[4 * t4 + 2][r], oacc[4 * t4 + 3][r]};
  if (G == 0) {
    sm_m[w][c] = m;
    sm_l[w][c] = l;
  }
  __syncthreads();

  const int rows = a.T - i0 < 16 ? a.T - i0 : 16;
  const int cc = threadIdx.x / TPC;
  const int d0 = (threadIdx.x % TPC) * VPT;
  if (cc < rows) {
    float M = kNegBig;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) M = fmaxf(M, sm_m[ww][cc]);
    float lsum = 0.f;
    float A[VPT];
#pragma unroll
    for (int e = 0; e < VPT; ++e) A[e] = 0.f;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) {
      const float f = fast_exp2(sm_m[ww][cc] - M);
      lsum = fmaf(sm_l[ww][cc], f, lsum);
      if constexpr (VPT == 2) {
        const f32x2 o = *reinterpret_cast<const f32x2*>(sm_o(ww, cc) + d0);
        A[0] = fmaf(o[0], f, A[0]);
        A[1] = fmaf(o[1], f, A[1]);
      } else {
#pragma unroll
        for (int t4 = 0; t4 < VPT / 4; ++t4) {
          const f32x4 o = *reinterpret_cast<const f32x4*>(sm_o(ww, cc) + d0 + 4 * t4);
#pragma unroll
          for (int e = 0; e < 4; ++e) A[4 * t4 + e] = fmaf(o[e], f, A[4 * t4 + e]);
        }
      }
    }
    if (nact == 1) {
      IO* op = static_cast<IO*>(a.out) + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh + (int64_t)(i0 + cc) * a.o_st + d0;
      const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
#pragma unroll
      for (int e = 0; e < VPT; ++e) Elem<IO>::store(op + e, lsum > 0.f ? A[e] * inv : 0.f);
    } else {
      float* rec = a.ws + (((int64_t)unit * a.num_splits + split) * 16 + cc) * (HD + 2);
      if (d0 == 0) {
        rec[0] = M;
        rec[1] = lsum;
      }
#pragma unroll
      for (int e = 0; e < VPT; ++e) rec[2 + d0 + e] = A[e];
    }
  }
}

// Merge the partial rows of each unit's active splits (the number a split computes from the
// request's lengths): one workgroup per (request, head, 16-row tile).
template <typename IO, int HD>
__global__ __launch_bounds__(256) void prefill_merge_kernel(const AttnArgs a) {
  const int ntiles = (a.T + 15) / 16;
  const int unit = blockIdx.x;
  int bh, qt;
  prefill_unit(unit, ntiles, a.B * a.H, bh, qt);
  const int h = bh % a.H;
  const int b = bh / a.H;
  const int i0 = qt * 16;
  const int i_last = (i0 + 15) < (a.T - 1) ? (i0 + 15) : (a.T - 1);
  int nb = (valid_keys(a.seq_lens[b], a.cur_lens[b], i_last) + 15) / 16;
  nb = nb < a.max_pages ? nb : a.max_pages;
  const int nact = nb > 0 ? (nb + a.split_blocks - 1) / a.split_blocks : 1;
  if (nact == 1) return;  // the split wrote the output itself
  const int rows = a.T - i0 < 16 ? a.T - i0 : 16;
  const float* rec0 = a.ws + ((int64_t)unit * a.num_splits) * 16 * (HD + 2);
  for (int idx = threadIdx.x; idx < rows * HD; idx += 256) {
    const int cc = idx / HD;
    const int d = idx - cc * HD;
    float M = kNegBig;
    for (int s = 0; s < nact; ++s) M = fmaxf(M, rec0[((int64_t)s * 16 + cc) * (HD + 2)]);
    float lsum = 0.f, A = 0.f;
    for (int s = 0; s < nact; ++s) {
      const float* rec = rec0 + ((int64_t)s * 16 + cc) * (HD + 2);
      const float f = fast_exp2(rec[0] - M);
      lsum = fmaf(rec[1], f, lsum);
      A = fmaf(rec[2 + d], f, A);
    }
    IO* op = static_cast<IO*>(a.out) + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh + (int64_t)(i0 + cc) * a.o_st;
    Elem<IO>::store(op + d, lsum > 0.f ? A / lsum : 0.f);
  }
}

// KV staging of the 16-row kernel: through LDS for bf16 KV always (both head_dims), and for fp32
// KV at head_dim 64 only while the grid fits 2 workgroups per CU: its 64 KB of LDS per workgroup
// halves the workgroups a CU holds against the register-staged build, which wins on larger grids
// (fp32 KV at head_dim 128 would need 128 KB per workgroup: registers only). The ring has two
// stages (one block ahead); deeper rings cost workgroups per CU without hiding more.
// PAGED_HIP_PREFILL_STAGING=lds / regs forces one of them (tests cover both).
static bool prefill_stage_in_lds(bool fp32_kv, unsigned grid) {
  const char* env = getenv("PAGED_HIP_PREFILL_STAGING");
  if (env != nullptr && strcmp(env, "lds") == 0) return true;
  if (env != nullptr && strcmp(env, "regs") == 0) return false;
  return !fp32_kv || (int64_t)grid <= 2 * (int64_t)pa_host::device_cu_count();
}

template <typename KV, typename IO>
static bool dispatch_prefill_io(const AttnArgs& a, dim3 grid, hipStream_t stream) {
  constexpr int threads = prefill_waves<KV>() * kWave;
  if (a.head_dim == 64) {
    if (prefill_stage_in_lds(std::is_same<KV, float>::value, grid.x)) {
      prefill_mfma_kernel<KV, IO, 64, false, true><<<grid, threads, 0, stream>>>(a);
      return true;
    }
    if constexpr (std::is_same<KV, float>::value) {
      if ((int64_t)grid.x > 3 * (int64_t)pa_host::device_cu_count()) {
        prefill_mfma_kernel<KV, IO, 64, true><<<grid, threads, 0, stream>>>(a);
        return true;
      }
    }
    prefill_mfma_kernel<KV, IO, 64><<<grid, threads, 0, stream>>>(a);
    return true;
  }
  if (a.head_dim == 128) {
    if constexpr (!std::is_same<KV, float>::value) {
      if (prefill_stage_in_lds(false, grid.x)) {
        prefill_mfma_kernel<KV, IO, 128, false, true><<<grid, threads, 0, stream>>>(a);
        return true;
      }
    }
    prefill_mfma_kernel<KV, IO, 128><<<grid, threads, 0, stream>>>(a);
    return true;
  }
  return false;
}

template <typename IO>
static void launch_prefill_merge(const AttnArgs& a, dim3 grid, hipStream_t stream) {
  if (a.head_dim == 64) prefill_merge_kernel<IO, 64><<<grid, 256, 0, stream>>>(a);
  else prefill_merge_kernel<IO, 128><<<grid, 256, 0, stream>>>(a);
}

static bool prefill_fast_shape(int32_t head_dim, int32_t block_size) {
  return block_size == 16 && (head_dim == 64 || head_dim == 128);
}

// Kernel choice between the wide-tile kernel (128 query rows per workgroup) and the 16-row one, by
// the wide kernel's unit count U = B * H * ceil(T / 128) against the CU count. The wide kernel
// shares each staged KV step among 128 rows but needs enough units to fill the GPU: it is taken
// from U >= 2 CUs always, for bf16 KV from U >= 3/4 of the CUs, and for fp32 KV at head_dim 128
// from U >= CUs (the crossovers measured on MI355X). PAGED_HIP_PREFILL_KERNEL=wide / tile forces
// one of them (tests use it to cover both at small sizes).
static bool use_wide_prefill(int kv_dtype, int32_t head_dim, int32_t batch, int32_t num_heads, int32_t query_len) {
  const char* env = getenv("PAGED_HIP_PREFILL_KERNEL");
  if (env != nullptr && strcmp(env, "wide") == 0) return true;
  if (env != nullptr && strcmp(env, "tile") == 0) return false;
  const int64_t units = prefill_wide_units(batch, num_heads, query_len);
  const int64_t cus = pa_host::device_cu_count();
  if (units >= 2 * cus) return true;
  if (kv_dtype == PA_DTYPE_BF16) return 4 * units >= 3 * cus;
  return head_dim == 128 && units >= cus;
}

// Split-step kernel (32-row tiles, 8 wavefronts splitting the KV steps; bf16 KV at head_dim 64)
// instead of the 16-row kernel, by its unit count U = B * H * ceil(T / 32) (one workgroup per CU
// at most) and the page-table width: it is taken for chunks longer than 64 rows from half the CUs
// to the CU count, and up to twice the CU count (two rounds) once the widest request spans 96
// pages, where it measured faster on MI355X (its 32-row tiles read each KV step half as often as
// the 16-row kernel's, which pays once the context outweighs the second round's tail: at 512
// units 0.96-1.02x of the 16-row time at 48-64 pages, 0.74-0.87x from 96 pages; at 384 units a
// tie at 88-96 pages, 0.92-0.97x from 120); below half the CUs or for short chunks the 16-row
// kernel's extra workgroups win. PAGED_HIP_PREFILL_KERNEL=split forces it where it applies (tile
// forces the 16-row kernel).
static bool use_split_prefill(int32_t batch, int32_t num_heads, int32_t query_len, int32_t max_pages) {
  const char* env = getenv("PAGED_HIP_PREFILL_KERNEL");
  if (env != nullptr && strcmp(env, "split") == 0) return true;
  if (env != nullptr && strcmp(env, "tile") == 0) return false;
  const int64_t units = prefill_split_units(batch, num_heads, query_len);
  const int64_t cus = pa_host::device_cu_count();
  if (query_len <= 64 || 2 * units < cus) return false;
  return units <= cus || (units <= 2 * cus && max_pages >= 96);
}

static int prefill_num_splits(int32_t max_pages, int32_t split_blocks) {
  if (split_blocks <= 0 || max_pages <= split_blocks) return 1;
  return (int)((max_pages + split_blocks - 1) / split_blocks);
}

}  // namespace pa

using namespace pa;

extern "C" size_t pa_prefill_workspace_size(int32_t batch, int32_t num_heads, int32_t query_len, int32_t head_dim,
                                            int32_t max_pages, int32_t split_blocks) {
  if (batch <= 0 || num_heads <= 0 || query_len <= 0 || !prefill_fast_shape(head_dim, 16)) return 0;
  if (split_blocks < 0) {  // the larger of the bf16 and fp32 KV launches' needs
    const int64_t gb = prefill_balanced_grid(batch, num_heads, query_len, head_dim, max_pages, PA_DTYPE_BF16);
    const int64_t gf = prefill_balanced_grid(batch, num_heads, query_len, head_dim, max_pages, PA_DTYPE_F32);
    const int64_t grid = gb > gf ? gb : gf;
    return grid > 0 ? PA_PREFILL_COUNTER_BYTES + prefill_balanced_record_bytes(grid, head_dim) : 0;
  }
  const int s = prefill_num_splits(max_pages, split_blocks);
  if (s <= 1) return 0;
  const int64_t units = (int64_t)batch * num_heads * ((query_len + 15) / 16);
  return PA_PREFILL_COUNTER_BYTES + (size_t)units * s * 16 * (head_dim + 2) * sizeof(float);
}

extern "C" int pa_prefill(const void* q, int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_t,
                          void* out, int64_t out_stride_b, int64_t out_stride_h, int64_t out_stride_t,
                          int io_dtype,
                          const void* k_pool, const void* v_pool, int kv_dtype, int64_t num_blocks,
                          const int32_t* page_table, int64_t pt_stride, int32_t max_pages,
                          const int32_t* seq_lens, const int32_t* cur_lens,
                          int32_t batch, int32_t num_heads, int32_t query_len, int32_t head_dim,
                          int32_t block_size, float scale, int32_t split_blocks,
                          void* workspace, size_t workspace_bytes, void* stream_) {
  pa_host::clear_error();
  PA_CHECK_ARG(batch >= 0 && num_heads > 0 && query_len >= 0 && head_dim > 0 && block_size > 0,
               "bad sizes: batch=%d heads=%d query_len=%d head_dim=%d block_size=%d", batch, num_heads,
               query_len, head_dim, block_size);
  PA_CHECK_ARG(io_dtype == PA_DTYPE_F32 || io_dtype == PA_DTYPE_BF16, "bad io dtype %d", io_dtype);
  PA_CHECK_ARG(kv_dtype == PA_DTYPE_F32 || kv_dtype == PA_DTYPE_BF16, "bad kv dtype %d", kv_dtype);
  if (batch == 0 || query_len == 0) return PA_OK;
  PA_CHECK_ARG(q && out && seq_lens && cur_lens, "null q/out/seq_lens/cur_lens");
  PA_CHECK_ARG(max_pages >= 0, "max_pages must be >= 0");
  if (max_pages > 0) {
    PA_CHECK_ARG(page_table != nullptr && pt_stride >= max_pages, "page table missing or stride < max_pages");
    PA_CHECK_ARG(k_pool && v_pool && num_blocks > 0, "KV pool missing or empty");
  }
  hipStream_t stream = static_cast<hipStream_t>(stream_);

  AttnArgs a{};
  a.q = q; a.q_sb = q_stride_b; a.q_sh = q_stride_h; a.q_st = q_stride_t;
  a.out = out; a.o_sb = out_stride_b; a.o_sh = out_stride_h; a.o_st = out_stride_t;
  a.k_pool = k_pool; a.v_pool = v_pool; a.num_blocks = num_blocks;
  a.page_table = page_table; a.pt_stride = pt_stride; a.max_pages = max_pages;
  a.seq_lens = seq_lens; a.cur_lens = cur_lens; a.order = nullptr;
  a.B = batch; a.H = num_heads; a.T = query_len; a.head_dim = head_dim; a.block_size = block_size;
  a.scale_log2 = scale * kLog2e;
  a.num_splits = 1; a.split_blocks = 0; a.ws = nullptr;

  if (!prefill_fast_shape(head_dim, block_size)) return launch_generic_attention(a, io_dtype, kv_dtype, stream);
  if (split_blocks < 0 && prefill_wide_supported(kv_dtype, head_dim, block_size)) {
    const int64_t grid = prefill_balanced_grid(batch, num_heads, query_len, head_dim, max_pages, kv_dtype);
    if (grid > 0) {
      const size_t need = PA_PREFILL_COUNTER_BYTES + prefill_balanced_record_bytes(grid, head_dim);
      if (workspace == nullptr || workspace_bytes < need)
        PA_FAIL(PA_ERR_WORKSPACE, "prefill workspace too small: need %zu bytes, have %zu", need, workspace_bytes);
      a.counters = static_cast<int32_t*>(workspace);
      a.ws = reinterpret_cast<float*>(static_cast<char*>(workspace) + PA_PREFILL_COUNTER_BYTES);
      return launch_prefill_wide(a, io_dtype, kv_dtype, stream);
    }
  }
  if (split_blocks <= 0 && prefill_wide_supported(kv_dtype, head_dim, block_size) &&
      use_wide_prefill(kv_dtype, head_dim, batch, num_heads, query_len))
    return launch_prefill_wide(a, io_dtype, kv_dtype, stream);
  if (split_blocks <= 0 && prefill_split_supported(kv_dtype, head_dim, block_size) &&
      use_split_prefill(batch, num_heads, query_len, max_pages))
    return launch_prefill_split(a, io_dtype, stream);

  const int64_t units = (int64_t)batch * num_heads * ((query_len + 15) / 16);
  const int nsplit = prefill_num_splits(max_pages, split_blocks);
  if (nsplit > 1) {
    const size_t need = pa_prefill_workspace_size(batch, num_heads, query_len, head_dim, max_pages, split_blocks);
    if (workspace == nullptr || workspace_bytes < need)
      PA_FAIL(PA_ERR_WORKSPACE, "prefill workspace too small: need %zu bytes, have %zu", need, workspace_bytes);
    a.num_splits = nsplit;
    a.split_blocks = split_blocks;
    a.ws = reinterpret_cast<float*>(static_cast<char*>(workspace) + PA_PREFILL_COUNTER_BYTES);
  }
  if (units * nsplit > 0x7fffffffLL) PA_FAIL(PA_ERR_INVALID_ARGUMENT, "grid too large");
  const dim3 grid((unsigned)(units * nsplit));
  bool ok;
  if (kv_dtype == PA_DTYPE_F32)
    ok = io_dtype == PA_DTYPE_F32 ? dispatch_prefill_io<float, float>(a, grid, stream)
                                  : dispatch_prefill_io<float, uint16_t>(a, grid, stream);
  else
    ok = io_dtype == PA_DTYPE_F32 ? dispatch_prefill_io<uint16_t, float>(a, grid, stream)
                                  : dispatch_prefill_io<uint16_t, uint16_t>(a, grid, stream);
  if (!ok) PA_FAIL(PA_ERR_UNSUPPORTED, "no prefill kernel for head_dim %d", head_dim);
  PA_CHECK_LAUNCH("prefill kernel");
  if (nsplit > 1) {
    if (io_dtype == PA_DTYPE_F32) launch_prefill_merge<float>(a, dim3((unsigned)units), stream);
    else launch_prefill_merge<uint16_t>(a, dim3((unsigned)units), stream);
    PA_CHECK_LAUNCH("prefill merge kernel");
  }
  return PA_OK;
}
