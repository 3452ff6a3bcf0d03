// Small-M linear layers for the decode step of the paged-attention model (gfx950), with fp32 or
// bf16 weights and activations (fp32 accumulation either way).
//
// A decode step (or a short prefill chunk) multiplies at most 64 token rows by each weight matrix,
// so the work is a stream of the weights (N x K) against a few rows of activations. Library GEMMs
// tile such shapes into a few tens of workgroups; here one workgroup of 8 (16 at K = 2048)
// wavefronts owns a 16-row x 16-column tile of the output (grid x: column tiles, y: row tiles),
// its wavefronts split K, and each wavefront accumulates the 16 (rows) x 16 (columns) tile over
// its K range, with v_mfma_f32_16x16x4_f32 (fp32 products, like torch's fp32 GEMM) or
// v_mfma_f32_16x16x16_bf16 (bf16 products); the partial tiles are summed in LDS and the epilogue
// is applied once. Every global load of a workgroup (weights, activations, LayerNorm parameters,
// bias, residual) is issued at its start, so a launch costs one memory round trip.
//   A: lane (G, c) holds x[row r0 + c][k(G, s, e)]  (rows >= M are zero)
//   B: lane (G, c) holds W[col n0 + c][k(G, s, e)] (torch Linear weight, row-major [N, K])
// with the contraction slot (G, e) of MFMA s mapped to k = k_wave + G*KL + E*s + e (E = 1 for
// fp32, 4 for bf16), so every lane reads KL contiguous values of one activation row and of one
// weight row (8- or 16-byte loads), and A and B use the same slot map.
// Fusions:
//   prologue  LayerNorm of the activation rows (biased variance, like torch.nn.LayerNorm; fp32
//             statistics, bf16 rows rounded to bf16 after normalisation as torch's bf16 LayerNorm
//             output is), computed from the slices the lanes already hold;
//   epilogue  bias, exact (erf) GELU, residual add, one rounding to the output type; or, for the
//             K/V projections, a scatter of each row's head_dim vectors into its KV-pool slot (the
//             append of the decode step).
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <type_traits>

#include "pa_attention.h"

namespace pa {

constexpr int kLinRows = 16;     // activation rows per workgroup (MFMA tile height)
// Rows per call, in 16-row tiles along grid y. A workgroup reads its weight tile once per 16-row
// tile, so these kernels are for small row counts; against torch's LayerNorm / GEMM / epilogue
// sequence they win up to 32-512 rows depending on the layer (the graph runner picks per layer).
constexpr int kLinMaxRows = 2048;

struct LinArgs {
  const void* x;      // [M, K] rows of type T
  int64_t x_stride;
  int32_t M, K;
  const void* ln_w;   // null: no LayerNorm
  const void* ln_b;
  float ln_eps;
  const void* w[3];   // segment weights, each [seg_n, K]
  const void* b[3];   // segment biases (null: none)
  int32_t seg_n, nseg;
  int32_t act;        // 0 none, 1 GELU (erf)
  const void* res;    // residual rows (null: none), same columns as out
  int64_t res_stride;
  void* out;          // segment 0's rows (and all segments' when there is no pool)
  int64_t out_stride;
  void* out_copy;     // when set: the same rows written a second time (row stride out_copy_stride)
  int64_t out_copy_stride;
  void* k_pool;       // when set: segments 1 and 2 are scattered into the K / V pools
  void* v_pool;
  int32_t pool_bf16;
  int64_t num_blocks;
  const int32_t* slots;  // per row: block * block_size + offset, < 0 = skip
  int32_t H, Hd, bs;
  int32_t bf16;       // T = bf16 (else fp32)
  int32_t cw_log2;    // output columns per workgroup: 1 << cw_log2 (4, 8 or 16)
  const int32_t* row_sel;  // when set: row m of the product is x row m * sel_group + row_sel[m]
  int32_t sel_group;       // (a negative entry counts from the group's end; clamped into the group)
  unsigned long long* token_keys;  // when set: per row, the running minimum of token_key over the
                                   // row's outputs (the row's greedy token in the low 32 bits)
  int64_t keys_stride;             // elements between rows' keys
  // Second layer folded into the first (small_linear_kernel with F2; fp32, one 16-row tile, 16
  // columns per workgroup): with h = this workgroup's 16 output columns n0.. of the first layer
  // (after bias and activation), out2[m][j] += sum_c h[m][c] * w2[j][n0 + c] for j < n2, by
  // device-scope atomic adds; workgroup 0 also adds res2[m][j] + b2[j]. out2 must hold zeros
  // before the launch.
  const void* w2;     // [n2, seg_n] row-major (torch Linear weight of the second layer)
  const void* b2;     // [n2] or null
  const void* res2;   // [M, res2_stride] or null
  int64_t res2_stride;
  void* out2;         // [M, out2_stride]
  int64_t out2_stride;
  int32_t n2;         // second layer's output features, <= threads per workgroup
};

// Greedy selection folded into a layer's epilogue: a key whose minimum over a row's columns picks
// what torch.argmax picks on the row as stored (value rounded to the output type): the largest
// value, NaN above every number, -0.0 equal to +0.0, and the lowest column among equals. High
// word: the bitwise complement of the value's order-preserving bits; low word: the column.
__device__ __forceinline__ unsigned long long token_key(float v, int n) {
  uint32_t b = __float_as_uint(v);
  uint32_t ord;
  if (v != v) {
    ord = 0xffffffffu;
  } else {
    if (v == 0.f) b = 0u;
    ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  }
  return ((unsigned long long)(~ord) << 32) | (uint32_t)n;
}

// The x row that product row m reads.
__device__ __forceinline__ int64_t lin_x_row(const LinArgs& a, int m) {
  if (a.row_sel == nullptr) return m;
  int r = a.row_sel[m];
  if (r < 0) r += a.sel_group;
  r = r < 0 ? 0 : (r >= a.sel_group ? a.sel_group - 1 : r);
  return (int64_t)m * a.sel_group + r;
}

// Wavefronts per workgroup (they split K): 16 at K = 2048 keeps more of the 128 KB weight tile in
// flight per compute unit.
template <int K>
constexpr int lin_waves() { return K >= 2048 ? 16 : 8; }

// Element access of a lane's slice held as 32-bit words (1 fp32 or 2 bf16 per word).
template <typename T> struct LinT;
template <> struct LinT<float> {
  static constexpr int EPW = 1;
  __device__ static __forceinline__ float get(const uint32_t* w, int e) { return __uint_as_float(w[e]); }
};
template <> struct LinT<uint16_t> {
  static constexpr int EPW = 2;
  __device__ static __forceinline__ float get(const uint32_t* w, int e) {
    return __uint_as_float((e & 1) ? (w[e >> 1] & 0xffff0000u) : (w[e >> 1] << 16));
  }
};

// NWD consecutive 32-bit words from p (16-byte loads, or one 8-byte load when NWD == 2); zeros
// when !ok.
template <int NWD>
__device__ __forceinline__ void load_words(uint32_t (&dst)[NWD], const void* p, bool ok) {
  const uint32_t* q = static_cast<const uint32_t*>(p);
  if constexpr (NWD % 4 == 0) {
#pragma unroll
    for (int i = 0; i < NWD; i += 4) {
      const u32x4 t = ok ? *reinterpret_cast<const u32x4*>(q + i) : u32x4{0u, 0u, 0u, 0u};
      dst[i] = t[0]; dst[i + 1] = t[1]; dst[i + 2] = t[2]; dst[i + 3] = t[3];
    }
  } else {
    static_assert(NWD == 2, "8- or 16-byte slices");
    const u32x2 t = ok ? *reinterpret_cast<const u32x2*>(q) : u32x2{0u, 0u};
    dst[0] = t[0]; dst[1] = t[1];
  }
}

typedef short s16x4 __attribute__((ext_vector_type(4)));

// Output element (m, n) of segment seg, bias and activation applied: the K/V segments of a
// q/k/v launch go to the row's pool slot (skipped for slot < 0 or outside the pool); otherwise
// v + residual is stored (and, with out_copy, stored a second time).
template <typename T>
__device__ __forceinline__ void lin_store(const LinArgs& a, int seg, int m, int n, float v, float res_v) {
  if (a.k_pool != nullptr && seg > 0) {
    const int slot = a.slots[m];
    const int64_t blk = slot >= 0 ? slot / a.bs : -1;
    if (blk < 0 || blk >= a.num_blocks) return;
    const int h = n / a.Hd, dd = n - h * a.Hd;
    const int64_t off = ((blk * a.H + h) * a.bs + (slot - blk * a.bs)) * a.Hd + dd;
    void* pool = seg == 1 ? a.k_pool : a.v_pool;
    if (a.pool_bf16)
      static_cast<uint16_t*>(pool)[off] = f32_to_bf16(v);
    else
      static_cast<float*>(pool)[off] = v;
    return;
  }
  Elem<T>::store(static_cast<T*>(a.out) + (int64_t)m * a.out_stride + seg * a.seg_n + n, v + res_v);
  if (a.out_copy != nullptr)
    Elem<T>::store(static_cast<T*>(a.out_copy) + (int64_t)m * a.out_copy_stride + seg * a.seg_n + n, v + res_v);
}

// STG: the weight rows of the tile and, where LDS allows (at most 128 KB for both), the
// activation rows go through LDS. Loaded straight into the operand registers, lane (G, c) reads
// row c, so every 4-lane group of a load touches 4 rows (4 cache lines), and the compute unit's
// L1 serves one line per 4-lane group per access; LDS-direct copies of each wavefront's slice
// read every row contiguously (one line per 4-lane group) and the operands are then read from LDS,
// with each row's 16-byte chunks XOR-swizzled by row so that the 16 rows of a read hit every bank
// once.
template <int K, bool LN, typename T, bool STG = false, bool F2 = false>
__global__ __launch_bounds__(lin_waves<K>() * kWave) void small_linear_kernel(const LinArgs a) {
  constexpr bool BF = sizeof(T) == 2;
  constexpr int kLinWaves = lin_waves<K>();
  constexpr int KW = K / kLinWaves;  // K range of one wavefront
  constexpr int KL = KW / 4;         // contiguous k values per lane
  constexpr int NWD = KL / LinT<T>::EPW;  // 32-bit words per lane per row slice
  static_assert(KL % 4 == 0 && (NWD % 4 == 0 || NWD == 2), "whole 8- or 16-byte slices");
  constexpr int RB = KW * (int)sizeof(T);         // bytes of one row's slice
  constexpr int CPR = RB / 16;                    // its 16-byte chunks
  constexpr int RPB = RB >= 256 ? 1 : 256 / RB;   // rows per 256 bytes (one pass over the banks)
  constexpr bool STG_W = STG && NWD % 4 == 0;
  constexpr bool STG_X = STG_W && 2 * 16 * RB * kLinWaves <= 128 * 1024;
  constexpr int kStageB = STG_W ? (STG_X ? 32 : 16) * RB : 16;  // LDS bytes per wavefront

  static_assert(!F2 || (!BF && kLinWaves * kWave >= 256), "the folded second layer is fp32");
  __shared__ float sm_part[kLinWaves][16][17];
  __shared__ float sm_h[F2 ? kLinRows : 1][F2 ? 17 : 1];
  __shared__ float sm_red[2][kLinWaves][kLinRows];
  __shared__ __attribute__((aligned(16))) unsigned char sm_stage[kLinWaves * kStageB];

  const int lane = threadIdx.x & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int G = lane >> 4;
  const int c = lane & 15;

  // The argument block spans four 64-byte lines. Left alone, the compiler loads the sizes the
  // tile arithmetic needs, waits, then loads the segment's weight pointer (an indexed load, a
  // second round trip) and the activation pointer (a third) before the first global load. The
  // sizes and the three weight pointers pass through this statement together with the other
  // arguments the loads below need, so all argument loads go out at once.
  int cwl = a.cw_log2, segn = a.seg_n;
  const void *w0 = a.w[0], *w1 = a.w[1], *w2 = a.w[2];
  asm volatile("" : "+s"(cwl), "+s"(segn), "+s"(w0), "+s"(w1), "+s"(w2)
               : "s"(a.x), "s"(a.x_stride), "s"(a.M), "s"(a.K), "s"(a.row_sel), "s"(a.sel_group), "s"(a.ln_w),
                 "s"(a.ln_b), "s"(a.res), "s"(a.res_stride), "s"(a.b[0]), "s"(a.b[1]), "s"(a.b[2]));

  // CW = 1 << cw_log2 output columns per workgroup (16, or 8 / 4 to spread a narrow layer over more
  // compute units: a launch is limited by how fast each workgroup can pull its weight tile); the
  // MFMA tile is always 16 wide, lanes c >= CW carry zero weights and load nothing.
  const int cw = 1 << cwl;
  const int tiles_per_seg = (segn + cw - 1) >> cwl;
  const int seg = blockIdx.x / tiles_per_seg;
  const int n0 = (blockIdx.x - seg * tiles_per_seg) << cwl;
  const T* W = static_cast<const T*>(seg == 0 ? w0 : (seg == 1 ? w1 : w2));
  const int kb = w * KW + G * KL;
  const int r0 = blockIdx.y * kLinRows;  // first activation row of this workgroup
  const bool row_ok = r0 + c < a.M;

  // ---- every global load first: weight row n0 + c and activation row c over k(G, ...), the
  // LayerNorm parameters of those k, and the epilogue operands of thread (m, n0 + cc) ----------
  // LayerNorm parameters are preloaded with the rest, except for fp32 at 16 wavefronts (K = 2048,
  // 128 registers per lane) where they are read after the statistics, 16 bytes at a time.
  constexpr bool PRE = LN && (BF || kLinWaves < 16);
  uint32_t wv[NWD], xv[NWD], lgv[PRE ? NWD : 1], lbv[PRE ? NWD : 1];
  auto sw = [](int r) { return (r / RPB) & (CPR - 1); };  // chunk swizzle of row r
  unsigned char* stage = sm_stage + w * kStageB;
  {
    const int n = n0 + c < a.seg_n ? n0 + c : a.seg_n - 1;  // clamp: the column is discarded
    if constexpr (STG_W) {
      // LDS slot (row r, chunk p) <- chunk p ^ sw(r) of the row's slice; rows past the layer
      // (or past M for activations) copy the last row and are discarded or zeroed on read.
      const T* wbase = W + (int64_t)n0 * a.K + w * KW;
#pragma unroll
      for (int s0 = 0; s0 < 16 * CPR; s0 += kWave) {
        const int sl = s0 + lane, r = sl / CPR, p = sl - r * CPR;
        const int nr = n0 + r < a.seg_n ? r : a.seg_n - 1 - n0;
        if (r < cw) stage_load16(wbase, (uint32_t)(nr * K * (int)sizeof(T) + 16 * (p ^ sw(r))), stage + 16 * s0);
      }
      if constexpr (STG_X) {
        const int64_t xr0 = __builtin_amdgcn_readfirstlane((int)lin_x_row(a, r0));  // < M * sel_group
        const T* xbase = static_cast<const T*>(a.x) + xr0 * a.x_stride + w * KW;
#pragma unroll
        for (int s0 = 0; s0 < 16 * CPR; s0 += kWave) {
          const int sl = s0 + lane, r = sl / CPR, p = sl - r * CPR;
          const int64_t xr = lin_x_row(a, r0 + r < a.M ? r0 + r : a.M - 1) - xr0;
          stage_load16(xbase, (uint32_t)(xr * a.x_stride * (int64_t)sizeof(T) + 16 * (p ^ sw(r))),
                       stage + 16 * RB + 16 * s0);
        }
      } else {
        load_words(xv, static_cast<const T*>(a.x) + (row_ok ? lin_x_row(a, r0 + c) : 0) * a.x_stride + kb, row_ok);
      }
    } else {
      load_words(wv, W + (int64_t)n * a.K + kb, c < cw);
      load_words(xv, static_cast<const T*>(a.x) + (row_ok ? lin_x_row(a, r0 + c) : 0) * a.x_stride + kb, row_ok);
    }
    if constexpr (PRE) {
      load_words(lgv, static_cast<const T*>(a.ln_w) + kb, true);
      load_words(lbv, static_cast<const T*>(a.ln_b) + kb, true);
    }
  }
  // F2: thread j < n2 owns output j of the second layer; its 16 weights w2[j][n0 .. n0 + 16) and,
  // in workgroup 0, the residual rows and bias it adds, are loaded now with everything else.
  float w2v[F2 ? 16 : 1], r2v[F2 ? kLinRows : 1];
  float b2v = 0.f;
  if constexpr (F2) {
    const int j = (int)threadIdx.x < a.n2 ? (int)threadIdx.x : a.n2 - 1;
    const f32x4* wp = reinterpret_cast<const f32x4*>(static_cast<const float*>(a.w2) + (int64_t)j * a.seg_n + n0);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const f32x4 t = wp[e];
      w2v[4 * e] = t[0]; w2v[4 * e + 1] = t[1]; w2v[4 * e + 2] = t[2]; w2v[4 * e + 3] = t[3];
    }
#pragma unroll
    for (int m2 = 0; m2 < kLinRows; ++m2) r2v[m2] = 0.f;
    if (blockIdx.x == 0) {
      if (a.b2 != nullptr) b2v = static_cast<const float*>(a.b2)[j];
      if (a.res2 != nullptr) {
#pragma unroll
        for (int m2 = 0; m2 < kLinRows; ++m2)
          if (m2 < a.M) r2v[m2] = static_cast<const float*>(a.res2)[(int64_t)m2 * a.res2_stride + j];
      }
    }
  }
  const int ml = (threadIdx.x >> a.cw_log2) & 15;  // epilogue thread (row ml, column cc) of the tile
  const int m = r0 + ml;
  const int cc = threadIdx.x & (cw - 1);
  const int n = n0 + cc;
  const bool live = (int)threadIdx.x < (kLinRows << a.cw_log2) && m < a.M && n < a.seg_n;
  float bias_v = 0.f, res_v = 0.f;
  if (live) {
    if (a.b[seg] != nullptr) bias_v = Elem<T>::load(static_cast<const T*>(a.b[seg]) + n);
    if (a.res != nullptr) res_v = Elem<T>::load(static_cast<const T*>(a.res) + (int64_t)m * a.res_stride + seg * a.seg_n + n);
  }

  if constexpr (STG_W) {
    // Every load of the wavefront has landed after vmcnt(0) (the tracked ones issued with them
    // are small); lane (G, c) then reads row c, chunks G * NWD / 4 .. of its wavefront's slice.
    vm_wait<0>();
#pragma unroll
    for (int t = 0; t < NWD / 4; ++t) {
      const int q = G * (NWD / 4) + t;
      const u32x4 z = {0u, 0u, 0u, 0u};
      const u32x4 wq = c < cw ? *reinterpret_cast<const u32x4*>(stage + c * RB + 16 * (q ^ sw(c))) : z;
#pragma unroll
      for (int e = 0; e < 4; ++e) wv[4 * t + e] = wq[e];
      if constexpr (STG_X) {
        const u32x4 xq = row_ok ? *reinterpret_cast<const u32x4*>(stage + 16 * RB + c * RB + 16 * (q ^ sw(c))) : z;
#pragma unroll
        for (int e = 0; e < 4; ++e) xv[4 * t + e] = xq[e];
      }
    }
  }

  // ---- LayerNorm of row c from the loaded slices: the row is spread over the 4 lane groups of
  // each wavefront, so the sums reduce with two permlane swaps and one LDS exchange ------------
  if constexpr (LN) {
    float xf[KL];
#pragma unroll
    for (int e = 0; e < KL; ++e) xf[e] = LinT<T>::get(xv, e);
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < KL; ++e) s += xf[e];
    s = sum_xor32(sum_xor16(s));
    if (G == 0) sm_red[0][w][c] = s;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int ww = 0; ww < kLinWaves; ++ww) tot += sm_red[0][ww][c];
    const float mean = tot / K;
    float q = 0.f;
#pragma unroll
    for (int e = 0; e < KL; ++e) q = fmaf(xf[e] - mean, xf[e] - mean, q);
    q = sum_xor32(sum_xor16(q));
    if (G == 0) sm_red[1][w][c] = q;
    __syncthreads();
    float var = 0.f;
#pragma unroll
    for (int ww = 0; ww < kLinWaves; ++ww) var += sm_red[1][ww][c];
    const float rstd = 1.f / sqrtf(var / K + a.ln_eps);
    constexpr int CH = NWD % 4 == 0 ? 4 : 2;  // words per parameter load
    constexpr int EPW = LinT<T>::EPW;
#pragma unroll
    for (int i0 = 0; i0 < NWD; i0 += CH) {
      uint32_t gw[CH], bw[CH];
      if constexpr (PRE) {
#pragma unroll
        for (int i = 0; i < CH; ++i) {
          gw[i] = lgv[i0 + i];
          bw[i] = lbv[i0 + i];
        }
      } else {
        load_words(gw, static_cast<const T*>(a.ln_w) + kb + i0 * EPW, true);
        load_words(bw, static_cast<const T*>(a.ln_b) + kb + i0 * EPW, true);
      }
#pragma unroll
      for (int e = 0; e < CH * EPW; ++e) {
        const int ee = i0 * EPW + e;
        xf[ee] = row_ok ? fmaf((xf[ee] - mean) * rstd, LinT<T>::get(gw, e), LinT<T>::get(bw, e)) : 0.f;
      }
    }
#pragma unroll
    for (int i = 0; i < NWD; ++i) {
      if constexpr (BF) xv[i] = pack_bf16x2(xf[2 * i], xf[2 * i + 1]);
      else xv[i] = __float_as_uint(xf[i]);
    }
  }

  // ---- D[m][n] += x[m][k] W[n][k] over this wavefront's K range (4 independent chains) ---------
  f32x4 acc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  if constexpr (BF) {
#pragma unroll
    for (int s = 0; s < KL / 4; ++s) {
      const s16x4 av = __builtin_bit_cast(s16x4, (u32x2{xv[2 * s], xv[2 * s + 1]}));
      const s16x4 bv = __builtin_bit_cast(s16x4, (u32x2{wv[2 * s], wv[2 * s + 1]}));
      acc[s & 3] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(av, bv, acc[s & 3], 0, 0, 0);
    }
  } else {
#pragma unroll
    for (int s = 0; s < KL; ++s)
      acc[s & 3] = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(xv[s]), __uint_as_float(wv[s]), acc[s & 3], 0, 0, 0);
  }
  const f32x4 d = (acc[0] + acc[1]) + (acc[2] + acc[3]);
  // lane (G, c) holds D[4G + i][c]: rows 4G..4G+3 of output column n0 + c
#pragma unroll
  for (int i = 0; i < 4; ++i) sm_part[w][4 * G + i][c] = d[i];
  __syncthreads();

  // ---- epilogue: one thread per (row, column) of the tile --------------------------------------
  if constexpr (F2) {
    // h[ml][cc] (bias and activation applied; zero past the rows and columns) into LDS, then thread
    // j folds the 16 columns into output j of every row and adds it to out2.
    if ((int)threadIdx.x < (kLinRows << a.cw_log2)) {
      float v = 0.f;
      if (live) {
#pragma unroll
        for (int ww = 0; ww < kLinWaves; ++ww) v += sm_part[ww][ml][cc];
        v += bias_v;
        if (a.act == 1) v = 0.5f * v * (1.f + erff(v * 0.70710678118654752f));
      }
      sm_h[ml][cc] = v;
    }
    __syncthreads();
    if ((int)threadIdx.x >= a.n2) return;
    float* o2 = static_cast<float*>(a.out2) + threadIdx.x;
#pragma unroll
    for (int m2 = 0; m2 < kLinRows; ++m2) {
      if (m2 >= a.M) break;
      float v = r2v[m2] + b2v;
#pragma unroll
      for (int cc2 = 0; cc2 < 16; ++cc2) v = fmaf(sm_h[m2][cc2], w2v[cc2], v);
      atomicAdd(o2 + (int64_t)m2 * a.out2_stride, v);
    }
    return;
  }
  const bool keyed = a.token_keys != nullptr;  // uniform
  if (!live && (!keyed || (int)threadIdx.x >= (kLinRows << a.cw_log2))) return;  // whole wavefronts past the tile
  float v = 0.f;
  if (live) {
#pragma unroll
    for (int ww = 0; ww < kLinWaves; ++ww) v += sm_part[ww][ml][cc];
    v += bias_v;
    if (a.act == 1) v = 0.5f * v * (1.f + erff(v * 0.70710678118654752f));
  }
  if (keyed) {
    // The row's cw threads are consecutive lanes: reduce their keys, one atomic per row.
    unsigned long long key = ~0ull;
    if (live) {
      float vr = v + res_v;
      if constexpr (BF) vr = bf16_to_f32(f32_to_bf16(vr));
      key = token_key(vr, n);
    }
    for (int off = 1; off < cw; off <<= 1) {
      const unsigned long long o = __shfl_xor(key, off);
      key = o < key ? o : key;
    }
    if (cc == 0 && m < a.M)
      __hip_atomic_fetch_min(a.token_keys + m * a.keys_stride, key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (!live) return;
  }
  lin_store<T>(a, seg, m, n, v, res_v);
}

// ---------------------------------------------------------------------------------------------
// Tiled kernel for steps of more than 16 rows. One workgroup of 4 wavefronts owns a 32-row x
// (16 * NT)-column output tile, so each weight column slice is read once per 32 rows (the
// 16-row kernel reads it once per 16 and, beyond a few hundred rows, runs in several rounds of
// workgroups). The wavefronts split K; each copies its K range, in chunks of one 128-byte row
// slice (32 fp32 or 64 bf16 values), into a private LDS ring with LDS-direct loads (one
// instruction copies 8 row slices, 16 bytes per lane): the whole range at once when that leaves
// room for two workgroups per compute unit, else through a two-stage ring, so no wavefront waits
// for another inside the loop. Row slices are stored with their
// 16-byte chunks XOR-swizzled by row, so the 16 rows of an operand read hit every bank group
// once. Operands and MFMAs follow the 16-row kernel (the same contiguous k-slot map; 16x16x4
// fp32 or 16x16x16 bf16, fp32 accumulation), two row tiles by NT column tiles per wavefront.
// LayerNorm: with the whole K range staged the row statistics come from the staged rows, each
// wavefront summing its K range of all 32 rows, combined in LDS; otherwise from a pass over the
// rows in memory that overlaps the ring's first loads. Either way the mean first, then the biased
// variance from the squared deviations (two passes, as torch does); every A value is then
// normalised (and, for bf16, rounded to bf16) as it is read. The wavefronts' partial tiles are summed in
// LDS and the epilogue (bias, GELU, residual, K/V scatter) runs one thread per output element.
// ---------------------------------------------------------------------------------------------
constexpr int kTileRows = 32;
constexpr int kTileWaves = 4;

template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

template <typename T, int K, int NT>
struct TileShape {
  static constexpr int BK = 128 / (int)sizeof(T);           // K per chunk
  static constexpr int NCH = K / kTileWaves / BK;           // chunks per wavefront
  static constexpr int STAGE = (kTileRows + 16 * NT) * 128; // bytes per chunk (A and B slices)
  // The whole K range staged when that leaves room for two workgroups per compute unit, else a
  // two-stage ring (the loads of the next chunk in flight while one is folded).
  static constexpr bool FULL = NCH * STAGE * kTileWaves <= 80 * 1024;
  static constexpr int STAGES = FULL ? NCH : 2;
};

template <typename T, int K, bool LN, int NT>
__global__ __launch_bounds__(kTileWaves * kWave) void tile_linear_kernel(const LinArgs a) {
  using Sh = TileShape<T, K, NT>;
  constexpr bool BF = sizeof(T) == 2;
  constexpr int EPW = LinT<T>::EPW;                 // values per 32-bit word
  constexpr int BK = Sh::BK;
  constexpr int KL = BK / 4;                        // contiguous k per lane per chunk
  constexpr int NWD = KL / EPW;                     // 8 words
  constexpr int KW = K / kTileWaves;                // K range of one wavefront
  constexpr int NCH = Sh::NCH;
  constexpr int STAGES = Sh::STAGES;
  constexpr int BN = 16 * NT;
  constexpr int A_BYTES = kTileRows * 128;
  constexpr int STAGE = Sh::STAGE;
  constexpr int RING = STAGES * STAGE;
  constexpr int EPT = kTileRows * BN / (kTileWaves * kWave);  // epilogue elements per thread
  constexpr int LOADS = (kTileRows + BN) / 8;                 // LDS-direct loads per chunk
  static_assert(KW % BK == 0 && NCH >= 1, "K must be a multiple of 4 row slices");
  static_assert(!LN || K <= 1024, "LayerNorm tiles take K <= 1024");
  static_assert(kTileWaves * RING >= kTileWaves * kTileRows * (BN + 1) * 4, "reduction buffer");

  __shared__ __attribute__((aligned(16))) unsigned char sm[kTileWaves * RING];
  __shared__ float sm_part[kTileWaves][kTileRows];
  __shared__ float sm_stat[kTileRows][2];

  const int lane = threadIdx.x & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int G = lane >> 4;
  const int c = lane & 15;

  int segn = a.seg_n;
  const void *w0 = a.w[0], *w1 = a.w[1], *w2 = a.w[2];
  asm volatile("" : "+s"(segn), "+s"(w0), "+s"(w1), "+s"(w2)
               : "s"(a.x), "s"(a.x_stride), "s"(a.M), "s"(a.ln_w), "s"(a.ln_b), "s"(a.res), "s"(a.res_stride),
                 "s"(a.b[0]), "s"(a.b[1]), "s"(a.b[2]));
  const int tiles_per_seg = segn / BN;
  const int seg = blockIdx.x / tiles_per_seg;
  const int n0 = (blockIdx.x - seg * tiles_per_seg) * BN;
  const T* W = static_cast<const T*>(seg == 0 ? w0 : (seg == 1 ? w1 : w2));
  const T* X = static_cast<const T*>(a.x);
  const int r0 = blockIdx.y * kTileRows;
  const int kw0 = w * KW;
  auto sw = [](int r) { return (r >> 1) & 7; };  // chunk swizzle of row slice r

  unsigned char* ring = sm + w * RING;
  auto issue = [&](int ch) {
    unsigned char* st = ring + (ch % STAGES) * STAGE;
    const uint32_t kb = (uint32_t)(kw0 + ch * BK) * (uint32_t)sizeof(T);
    const int r = lane >> 3, pc = lane & 7;
#pragma unroll
    for (int j = 0; j < kTileRows / 8; ++j) {
      const int rr = 8 * j + r;
      const int xr = r0 + rr < a.M ? r0 + rr : a.M - 1;
      stage_load16(X, (uint32_t)(xr * a.x_stride * (int64_t)sizeof(T)) + kb + 16 * (pc ^ sw(rr)), st + 1024 * j);
    }
#pragma unroll
    for (int j = 0; j < BN / 8; ++j) {
      const int rr = 8 * j + r;
      stage_load16(W, (uint32_t)((n0 + rr) * K * (int)sizeof(T)) + kb + 16 * (pc ^ sw(rr)), st + A_BYTES + 1024 * j);
    }
  };
  // The ring's first chunks go out first; everything else overlaps them.
#pragma unroll
  for (int ch = 0; ch < STAGES; ++ch) issue(ch);

  // ---- loads that do not depend on the loop: LayerNorm parameters of this lane's k values,
  // and the epilogue's bias and residual values -------------------------------------------------
  uint32_t gw[LN ? NCH * NWD : 1], bw[LN ? NCH * NWD : 1];
  if constexpr (LN) {
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
      const int kk = kw0 + ch * BK + G * KL;
      load_words(*reinterpret_cast<uint32_t(*)[NWD]>(gw + ch * NWD), static_cast<const T*>(a.ln_w) + kk, true);
      load_words(*reinterpret_cast<uint32_t(*)[NWD]>(bw + ch * NWD), static_cast<const T*>(a.ln_b) + kk, true);
    }
  }
  float bias_e[EPT], res_e[EPT];
#pragma unroll
  for (int i = 0; i < EPT; ++i) {
    const int e = threadIdx.x + i * kTileWaves * kWave;
    const int m = r0 + e / BN, n = n0 + e % BN;
    bias_e[i] = a.b[seg] != nullptr ? Elem<T>::load(static_cast<const T*>(a.b[seg]) + n) : 0.f;
    res_e[i] = (a.res != nullptr && m < a.M)
                   ? Elem<T>::load(static_cast<const T*>(a.res) + (int64_t)m * a.res_stride + seg * segn + n) : 0.f;
  }

  // ---- LayerNorm statistics. Whole K staged: from the staged rows, lane l summing row l / 2,
  // half h = l % 2 of every chunk's 128-byte slice (4 of its 8 16-byte pieces), over this
  // wavefront's K range. Otherwise: a pass over the rows in memory (wavefront w takes rows
  // 8w .. 8w + 7, all 64 lanes along each row), while the ring's first chunks are in flight. ----
  float mu[2] = {0.f, 0.f}, rs[2] = {0.f, 0.f};
  if constexpr (LN && !Sh::FULL) {
    // wavefront w takes rows 8w .. 8w + 7 with 8 lanes per row (lane 8i + j: row i, 16-byte
    // pieces 8t + j of it), so every load instruction reads 128 contiguous bytes per row and a
    // row's sums close with three DPP steps instead of a wavefront-wide reduction per row
    constexpr int PL = K * (int)sizeof(T) / 128;  // 16-byte pieces per lane
    constexpr int PH = PL < 16 ? PL : 16;          // pieces held at once (fp32 K 1024 reads twice)
    constexpr int NH = PL / PH;
    const int ri = lane >> 3, pj = lane & 7;
    const int r = r0 + 8 * w + ri;
    const u32x4* xp = reinterpret_cast<const u32x4*>(X + (int64_t)(r < a.M ? r : a.M - 1) * a.x_stride);
    u32x4 xr[PH];
    float part[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int hh = 0; hh < NH; ++hh) {
#pragma unroll
      for (int t = 0; t < PH; ++t) xr[t] = xp[8 * (hh * PH + t) + pj];
#pragma unroll
      for (int t = 0; t < PH; ++t) {
        const uint32_t qw[4] = {xr[t][0], xr[t][1], xr[t][2], xr[t][3]};
#pragma unroll
        for (int e = 0; e < 4 * EPW; ++e) part[e & 3] += LinT<T>::get(qw, e);
      }
    }
    const float mean = group_sum<8>((part[0] + part[1]) + (part[2] + part[3])) / K;
#pragma unroll
    for (int e = 0; e < 4; ++e) part[e] = 0.f;
#pragma unroll
    for (int hh = 0; hh < NH; ++hh) {
      if (NH > 1) {
#pragma unroll
        for (int t = 0; t < PH; ++t) xr[t] = xp[8 * (hh * PH + t) + pj];
      }
#pragma unroll
      for (int t = 0; t < PH; ++t) {
        const uint32_t qw[4] = {xr[t][0], xr[t][1], xr[t][2], xr[t][3]};
#pragma unroll
        for (int e = 0; e < 4 * EPW; ++e) {
          const float d = LinT<T>::get(qw, e) - mean;
          part[e & 3] = fmaf(d, d, part[e & 3]);
        }
      }
    }
    const float var = group_sum<8>((part[0] + part[1]) + (part[2] + part[3])) / K;
    if (pj == 0) {
      sm_stat[8 * w + ri][0] = mean;
      sm_stat[8 * w + ri][1] = 1.f / sqrtf(var + a.ln_eps);
    }
    __syncthreads();
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      mu[rt] = sm_stat[16 * rt + c][0];
      rs[rt] = sm_stat[16 * rt + c][1];
    }
  }
  if constexpr (LN && Sh::FULL) {
    vm_wait<0>();
    const int sr = lane >> 1, sh = lane & 1;
    auto row_pass = [&](float center, bool square) {
      float acc_s = 0.f;
#pragma unroll
      for (int ch = 0; ch < NCH; ++ch) {
        const unsigned char* st = ring + ch * STAGE + sr * 128;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const u32x4 q = *reinterpret_cast<const u32x4*>(st + 16 * ((4 * sh + t) ^ sw(sr)));
          const uint32_t qw[4] = {q[0], q[1], q[2], q[3]};
#pragma unroll
          for (int e = 0; e < 4 * EPW; ++e) {
            const float d = LinT<T>::get(qw, e) - center;
            acc_s = square ? fmaf(d, d, acc_s) : acc_s + d;
          }
        }
      }
      return acc_s + __shfl_xor(acc_s, 1);
    };
    float part = row_pass(0.f, false);
    if (sh == 0) sm_part[w][sr] = part;
    __syncthreads();
    float mean = 0.f;
#pragma unroll
    for (int ww = 0; ww < kTileWaves; ++ww) mean += sm_part[ww][sr];
    mean /= K;
    __syncthreads();
    part = row_pass(mean, true);
    if (sh == 0) sm_part[w][sr] = part;
    __syncthreads();
    if (w == 0 && sh == 0) {
      float var = 0.f;
#pragma unroll
      for (int ww = 0; ww < kTileWaves; ++ww) var += sm_part[ww][sr];
      sm_stat[sr][0] = mean;
      sm_stat[sr][1] = 1.f / sqrtf(var / K + a.ln_eps);
    }
    __syncthreads();
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      mu[rt] = sm_stat[16 * rt + c][0];
      rs[rt] = sm_stat[16 * rt + c][1];
    }
  }

  f32x4 acc[2][NT];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int ct = 0; ct < NT; ++ct) acc[rt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};

  static_for<0, NCH>([&](auto chc) {
    constexpr int ch = decltype(chc)::value;
    // chunk ch has landed once at most the loads of the chunks issued after it are outstanding
    constexpr int last_issued = (ch + STAGES - 1) < (NCH - 1) ? (ch + STAGES - 1) : (NCH - 1);
    if constexpr (!(LN && Sh::FULL)) vm_wait<(last_issued - ch) * LOADS>();
    const unsigned char* st = ring + (ch % STAGES) * STAGE;
    uint32_t av[2][NWD], bv[NT][NWD];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      const int rr = 16 * rt + c;
#pragma unroll
      for (int t = 0; t < NWD / 4; ++t) {
        const u32x4 q = *reinterpret_cast<const u32x4*>(st + rr * 128 + 16 * ((2 * G + t) ^ sw(rr)));
        av[rt][4 * t] = q[0]; av[rt][4 * t + 1] = q[1]; av[rt][4 * t + 2] = q[2]; av[rt][4 * t + 3] = q[3];
      }
    }
#pragma unroll
    for (int ct = 0; ct < NT; ++ct) {
      const int rr = 16 * ct + c;
#pragma unroll
      for (int t = 0; t < NWD / 4; ++t) {
        const u32x4 q = *reinterpret_cast<const u32x4*>(st + A_BYTES + rr * 128 + 16 * ((2 * G + t) ^ sw(rr)));
        bv[ct][4 * t] = q[0]; bv[ct][4 * t + 1] = q[1]; bv[ct][4 * t + 2] = q[2]; bv[ct][4 * t + 3] = q[3];
      }
    }
    if constexpr (LN) {
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        float xf[KL];
#pragma unroll
        for (int e = 0; e < KL; ++e)  // (rows past M hold row M - 1 and are never stored)
          xf[e] = fmaf((LinT<T>::get(av[rt], e) - mu[rt]) * rs[rt], LinT<T>::get(gw + ch * NWD, e),
                       LinT<T>::get(bw + ch * NWD, e));
#pragma unroll
        for (int i = 0; i < NWD; ++i) {
          if constexpr (BF) av[rt][i] = pack_bf16x2(xf[2 * i], xf[2 * i + 1]);
          else av[rt][i] = __float_as_uint(xf[i]);
        }
      }
    }
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int ct = 0; ct < NT; ++ct) {
        if constexpr (BF) {
#pragma unroll
          for (int s4 = 0; s4 < KL / 4; ++s4) {
            const s16x4 x4 = __builtin_bit_cast(s16x4, (u32x2{av[rt][2 * s4], av[rt][2 * s4 + 1]}));
            const s16x4 w4 = __builtin_bit_cast(s16x4, (u32x2{bv[ct][2 * s4], bv[ct][2 * s4 + 1]}));
            acc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(x4, w4, acc[rt][ct], 0, 0, 0);
          }
        } else {
#pragma unroll
          for (int s1 = 0; s1 < KL; ++s1)
            acc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(av[rt][s1]), __uint_as_float(bv[ct][s1]),
                                                               acc[rt][ct], 0, 0, 0);
        }
      }
    // refill this chunk's stage with chunk ch + STAGES once its reads have returned
    if constexpr (ch + STAGES < NCH) {
      lds_read_wait();
      issue(ch + STAGES);
    }
  });

  // ---- sum the wavefronts' partial tiles in LDS (the rings are free once every wavefront is
  // past its loop), then one thread per output element -----------------------------------------
  __syncthreads();
  float* red = reinterpret_cast<float*>(sm);
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int ct = 0; ct < NT; ++ct)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[(w * kTileRows + 16 * rt + 4 * G + i) * (BN + 1) + 16 * ct + c] = acc[rt][ct][i];
  __syncthreads();
#pragma unroll
  for (int i = 0; i < EPT; ++i) {
    const int e = threadIdx.x + i * kTileWaves * kWave;
    const int ml = e / BN, col = e % BN;
    const int m = r0 + ml;
    if (m >= a.M) continue;
    float v = bias_e[i];
#pragma unroll
    for (int ww = 0; ww < kTileWaves; ++ww) v += red[(ww * kTileRows + ml) * (BN + 1) + col];
    if (a.act == 1) v = 0.5f * v * (1.f + erff(v * 0.70710678118654752f));
    lin_store<T>(a, seg, m, n0 + col, v, res_e[i]);
  }
}

#ifndef PA_LIN_FORCE_CW_LOG2
#define PA_LIN_FORCE_CW_LOG2 0
#endif

// Column tile width: the widest of 16, 8, 4 columns whose grid still has 192 workgroups with a
// LayerNorm prologue (each workgroup normalises its rows again) or 128 without (else 4), so
// narrow layers spread their weight stream over more compute units.
static int lin_cw_log2(const LinArgs& a) {
  if (PA_LIN_FORCE_CW_LOG2) return PA_LIN_FORCE_CW_LOG2;
  const int64_t target = a.ln_w != nullptr ? 192 : 128;
  const int64_t row_tiles = (a.M + kLinRows - 1) / kLinRows;
  for (int l2 = 4; l2 > 2; --l2) {
    const int64_t tiles = (int64_t)a.nseg * ((a.seg_n + (1 << l2) - 1) >> l2) * row_tiles;
    if (tiles >= target) return l2;
  }
  return 2;
}

// The weight / activation slices go through LDS (see small_linear_kernel);
// PAGED_HIP_LINEAR_STAGING=regs turns that off (tests compare both).
static bool lin_stage_in_lds() {
  const char* env = getenv("PAGED_HIP_LINEAR_STAGING");
  return !(env != nullptr && strcmp(env, "regs") == 0);
}

// Kernel for a call: the tiled kernel above 16 rows where it applies (PAGED_HIP_LINEAR_KERNEL =
// small / tiled forces one of them where both apply; tests use it to cover both).
static bool tile_linear_applies(const LinArgs& a) {
  if (a.row_sel != nullptr || a.token_keys != nullptr) return false;
  if (!(a.K == 256 || a.K == 512 || a.K == 1024 || a.K == 2048)) return false;
  if (a.ln_w != nullptr && a.K > 1024) return false;
  if (a.seg_n % 16 != 0) return false;
  return (int64_t)a.M * a.x_stride * (a.bf16 ? 2 : 4) < (1LL << 31);
}

// Measured in graph replay on MI355X (d_model 512, d_ff 2048; 16-row / tiled kernel, us): fc2
// (K 2048) fp32 8.0 / 7.6 at 32 rows, 16.1 / 8.1 at 256; bf16 3.8 / 4.3 at 64, 4.5 / 4.4 at 128,
// 7.2 / 4.7 at 256. K 512 with LayerNorm: q/k/v fp32 6.7 / 6.8 at 64 rows, 9.3 / 9.2 at 128, 13.4 /
// 11.8 at 192; fc1 + GELU fp32 6.5 / 6.5 at 64, 11.1 / 8.1 at 128, bf16 7.5 / 6.4 at 128 (q/k/v
// bf16 6.3 / 6.8 at 128, 8.6 / 8.0 at 192). K 512 without: out_proj 3.7 / 3.8 at 128 rows, 4.4 /
// 3.9 at 192.
static bool use_tile_linear(const LinArgs& a) {
  if (!tile_linear_applies(a)) return false;
  const char* env = getenv("PAGED_HIP_LINEAR_KERNEL");
  if (env != nullptr && strcmp(env, "small") == 0) return false;
  if (env != nullptr && strcmp(env, "tiled") == 0) return true;
  if (a.K >= 1024) return a.M >= (a.bf16 ? 128 : 32);
  return a.M >= (a.ln_w != nullptr ? 96 : 192);
}

// Column tile width. 32 columns with a LayerNorm prologue, which each workgroup runs for its
// rows and then spreads over twice the columns; without one, 32 only when that still gives two
// workgroups per compute unit. Graph replay on MI355X, d_model 512, 16 / 32 columns, us: LayerNorm
// + q/k/v fp32 9.1 / 8.4 at 128 rows, 11.5 / 11.9 at 256, 19.2 / 17.2 at 512; LayerNorm + fc1 fp32
// 14.2 / 11.5 at 256, bf16 10.3 / 7.6; out_proj fp32 3.9 / 5.3 at 256, 5.1 / 5.4 at 512; fc2 (K
// 2048) fp32 8.1 / 11.9 at 256, 12.3 / 12.9 at 512. PAGED_HIP_TILE_COLUMNS=16 / 32 forces a width.
static int launch_tile_linear(const LinArgs& a, hipStream_t stream) {
  const int64_t row_tiles = (a.M + kTileRows - 1) / kTileRows;
  const int64_t tiles32 = (int64_t)a.nseg * (a.seg_n / 32) * row_tiles;
  bool nt2 = a.seg_n % 32 == 0 && (a.ln_w != nullptr || tiles32 >= 2 * (int64_t)pa_host::device_cu_count());
  if (const char* env = getenv("PAGED_HIP_TILE_COLUMNS")) {
    if (strcmp(env, "16") == 0) nt2 = false;
    if (strcmp(env, "32") == 0) nt2 = a.seg_n % 32 == 0;
  }
  const int bn = nt2 ? 32 : 16;
  const dim3 grid((unsigned)(a.nseg * (a.seg_n / bn)), (unsigned)row_tiles);
  const dim3 block(kTileWaves * kWave);
  const bool ln = a.ln_w != nullptr;
#define PA_TILE_LAUNCH(TT, KK, LNF)                                                   \
  if (nt2) tile_linear_kernel<TT, KK, LNF, 2><<<grid, block, 0, stream>>>(a);         \
  else tile_linear_kernel<TT, KK, LNF, 1><<<grid, block, 0, stream>>>(a);
#define PA_TILE_K(TT)                                                                 \
  switch (a.K) {                                                                      \
    case 256: if (ln) { PA_TILE_LAUNCH(TT, 256, true) } else { PA_TILE_LAUNCH(TT, 256, false) } break; \
    case 512: if (ln) { PA_TILE_LAUNCH(TT, 512, true) } else { PA_TILE_LAUNCH(TT, 512, false) } break; \
    case 1024: if (ln) { PA_TILE_LAUNCH(TT, 1024, true) } else { PA_TILE_LAUNCH(TT, 1024, false) } break; \
    case 2048: PA_TILE_LAUNCH(TT, 2048, false) break;                                 \
  }
  if (a.bf16) { PA_TILE_K(uint16_t) } else { PA_TILE_K(float) }
#undef PA_TILE_K
#undef PA_TILE_LAUNCH
  PA_CHECK_LAUNCH("tiled linear kernel");
  return PA_OK;
}

static int launch_small_linear(LinArgs a, hipStream_t stream) {
  if (use_tile_linear(a)) return launch_tile_linear(a, stream);
  a.cw_log2 = lin_cw_log2(a);
  const int64_t tiles = (int64_t)a.nseg * ((a.seg_n + (1 << a.cw_log2) - 1) >> a.cw_log2);
  if (tiles > 0x7fffffffLL) PA_FAIL(PA_ERR_INVALID_ARGUMENT, "grid too large");
  const dim3 grid((unsigned)tiles, (unsigned)((a.M + kLinRows - 1) / kLinRows));
  const bool ln = a.ln_w != nullptr;
  // (the staged activation offsets are 32-bit: the rows one tile may read must span < 2 GiB)
  const int64_t x_rows = a.row_sel != nullptr ? (int64_t)a.M * a.sel_group : a.M;  // all tiles' rows
  const bool stg = lin_stage_in_lds() && x_rows * a.x_stride * (a.bf16 ? 2 : 4) < (1LL << 31);
#define PA_LIN_LAUNCH(KK, LNF, TT)                                                                        \
  if (stg) small_linear_kernel<KK, LNF, TT, true><<<grid, lin_waves<KK>() * kWave, 0, stream>>>(a);       \
  else small_linear_kernel<KK, LNF, TT, false><<<grid, lin_waves<KK>() * kWave, 0, stream>>>(a);
#define PA_LIN_CASE(KK)                                                                                   \
  case KK:                                                                                                \
    if (a.bf16) {                                                                                         \
      if (ln) { PA_LIN_LAUNCH(KK, true, uint16_t) } else { PA_LIN_LAUNCH(KK, false, uint16_t) }           \
    } else {                                                                                              \
      if (ln) { PA_LIN_LAUNCH(KK, true, float) } else { PA_LIN_LAUNCH(KK, false, float) }                 \
    }                                                                                                     \
    break;
  switch (a.K) {
    PA_LIN_CASE(128)
    PA_LIN_CASE(256)
    PA_LIN_CASE(512)
    PA_LIN_CASE(1024)
    PA_LIN_CASE(2048)
    default: PA_FAIL(PA_ERR_UNSUPPORTED, "small linear: in_features must be 128, 256, 512, 1024 or 2048, got %d", a.K);
  }
#undef PA_LIN_CASE
#undef PA_LIN_LAUNCH
  PA_CHECK_LAUNCH("small linear kernel");
  return PA_OK;
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// LayerNorm + first layer + activation + second layer in one launch (fp32, at most 16 rows): one
// workgroup per 16 columns of the first layer, each adding its share of the second layer to out2.
static int launch_mlp_rows(LinArgs a, hipStream_t stream) {
  a.cw_log2 = 4;
  const dim3 grid((unsigned)(a.seg_n / 16), 1u);
  const bool stg = lin_stage_in_lds();
#define PA_MLP_CASE(KK)                                                                              \
  case KK:                                                                                           \
    if (stg) small_linear_kernel<KK, true, float, true, true><<<grid, lin_waves<KK>() * kWave, 0, stream>>>(a); \
    else small_linear_kernel<KK, true, float, false, true><<<grid, lin_waves<KK>() * kWave, 0, stream>>>(a);    \
    break;
  switch (a.K) {
    PA_MLP_CASE(128)
    PA_MLP_CASE(256)
    PA_MLP_CASE(512)
    default: PA_FAIL(PA_ERR_UNSUPPORTED, "mlp rows: d_model must be 128, 256 or 512, got %d", a.K);
  }
#undef PA_MLP_CASE
  PA_CHECK_LAUNCH("mlp rows kernel");
  return PA_OK;
}

// Token + position embedding of a [B, T] step: row b*T + t = tok[ids[b, t]] + pos[min(p0[b] + t,
// max_pos - 1)]; an id outside the vocabulary gives a zero token row. One workgroup per row;
// 16-byte vectors (4 fp32 or 8 bf16 values), the sum in fp32, rounded once for bf16.
template <typename T>
__global__ __launch_bounds__(256) void embed_rows_kernel(const int64_t* ids, const int64_t* pos0, int32_t T_len,
                                                        const T* tok, int64_t vocab, const T* pos_tab,
                                                        int32_t max_pos, int32_t d, T* out, int64_t out_stride) {
  constexpr int EPV = 16 / sizeof(T);
  const int row = blockIdx.x;
  const int b = row / T_len, t = row - b * T_len;
  const int64_t id = ids[row];
  int64_t p = pos0[b] + t;
  p = p < max_pos - 1 ? p : max_pos - 1;
  p = p > 0 ? p : 0;
  const bool ok = id >= 0 && id < vocab;
  const u32x4* tr = reinterpret_cast<const u32x4*>(tok + (ok ? id : 0) * d);
  const u32x4* pr = reinterpret_cast<const u32x4*>(pos_tab + p * d);
  u32x4* o = reinterpret_cast<u32x4*>(out + (int64_t)row * out_stride);
  for (int k = threadIdx.x; k < d / EPV; k += 256) {
    const u32x4 tv = ok ? tr[k] : u32x4{0u, 0u, 0u, 0u};
    const u32x4 pv = pr[k];
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (sizeof(T) == 4) {
        r[i] = __float_as_uint(__uint_as_float(tv[i]) + __uint_as_float(pv[i]));
      } else {
        const float lo = bf16_to_f32((uint16_t)(tv[i] & 0xffffu)) + bf16_to_f32((uint16_t)(pv[i] & 0xffffu));
        const float hi = bf16_to_f32((uint16_t)(tv[i] >> 16)) + bf16_to_f32((uint16_t)(pv[i] >> 16));
        r[i] = (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
      }
    }
    o[k] = r;
  }
}

}  // namespace pa

using namespace pa;

// Activations, weights, biases, LayerNorm parameters and outputs share one element type (dtype).
static bool lin_dtype_ok(int dtype) { return dtype == PA_DTYPE_F32 || dtype == PA_DTYPE_BF16; }
static int elems_per_16b(int dtype) { return dtype == PA_DTYPE_BF16 ? 8 : 4; }

extern "C" int pa_linear_rows(const void* x, int64_t x_stride, int32_t rows, int32_t in_features,
                              const void* weight, const void* bias, int32_t out_features,
                              const void* ln_weight, const void* ln_bias, float ln_eps,
                              int32_t activation, const void* residual, int64_t residual_stride,
                              void* out, int64_t out_stride, void* out_copy, int64_t out_copy_stride,
                              int dtype, void* stream) {
  pa_host::clear_error();
  PA_CHECK_ARG(rows >= 0 && rows <= kLinMaxRows, "rows must be in [0, %d], got %d", kLinMaxRows, rows);
  PA_CHECK_ARG(out_features > 0 && in_features > 0, "bad sizes: in=%d out=%d", in_features, out_features);
  PA_CHECK_ARG(activation == 0 || activation == 1, "bad activation %d", activation);
  PA_CHECK_ARG(lin_dtype_ok(dtype), "bad dtype %d", dtype);
  if (rows == 0) return PA_OK;
  PA_CHECK_ARG(x && weight && out, "null x/weight/out");
  PA_CHECK_ARG((ln_weight == nullptr) == (ln_bias == nullptr), "LayerNorm needs both weight and bias");
  const int vec = elems_per_16b(dtype);
  PA_CHECK_ARG(aligned16(x) && aligned16(weight) && x_stride % vec == 0 && (!ln_weight || (aligned16(ln_weight) &&
               aligned16(ln_bias))), "x, weight and LayerNorm parameters must be 16-byte aligned, x_stride a multiple of %d", vec);
  PA_CHECK_ARG(x_stride >= in_features && out_stride >= out_features &&
               (residual == nullptr || residual_stride >= out_features) &&
               (out_copy == nullptr || out_copy_stride >= out_features), "row strides smaller than the rows");
  LinArgs a{};
  a.x = x; a.x_stride = x_stride; a.M = rows; a.K = in_features;
  a.ln_w = ln_weight; a.ln_b = ln_bias; a.ln_eps = ln_eps;
  a.w[0] = weight; a.b[0] = bias; a.seg_n = out_features; a.nseg = 1;
  a.act = activation; a.res = residual; a.res_stride = residual_stride;
  a.out = out; a.out_stride = out_stride; a.bf16 = dtype == PA_DTYPE_BF16;
  a.out_copy = out_copy; a.out_copy_stride = out_copy_stride;
  return launch_small_linear(a, static_cast<hipStream_t>(stream));
}

extern "C" int pa_linear_select_rows(const void* x, int64_t x_stride, int32_t groups, int32_t group_rows,
                                     const int32_t* row_index, int32_t in_features, const void* weight,
                                     const void* bias, int32_t out_features, const void* ln_weight,
                                     const void* ln_bias, float ln_eps, int32_t activation, void* out,
                                     int64_t out_stride, uint64_t* token_keys, int64_t token_keys_stride,
                                     int dtype, void* stream) {
  pa_host::clear_error();
  PA_CHECK_ARG(groups >= 0 && groups <= kLinMaxRows, "groups must be in [0, %d], got %d", kLinMaxRows, groups);
  PA_CHECK_ARG(group_rows > 0, "group_rows must be positive, got %d", group_rows);
  PA_CHECK_ARG(out_features > 0 && in_features > 0, "bad sizes: in=%d out=%d", in_features, out_features);
  PA_CHECK_ARG(activation == 0 || activation == 1, "bad activation %d", activation);
  PA_CHECK_ARG(lin_dtype_ok(dtype), "bad dtype %d", dtype);
  if (groups == 0) return PA_OK;
  PA_CHECK_ARG(x && weight && out && row_index, "null x/weight/out/row_index");
  PA_CHECK_ARG((ln_weight == nullptr) == (ln_bias == nullptr), "LayerNorm needs both weight and bias");
  const int vec = elems_per_16b(dtype);
  PA_CHECK_ARG(aligned16(x) && aligned16(weight) && x_stride % vec == 0 && (!ln_weight || (aligned16(ln_weight) &&
               aligned16(ln_bias))), "x, weight and LayerNorm parameters must be 16-byte aligned, x_stride a multiple of %d", vec);
  PA_CHECK_ARG(x_stride >= in_features && out_stride >= out_features, "row strides smaller than the rows");
  LinArgs a{};
  a.x = x; a.x_stride = x_stride; a.M = groups; a.K = in_features;
  a.ln_w = ln_weight; a.ln_b = ln_bias; a.ln_eps = ln_eps;
  a.w[0] = weight; a.b[0] = bias; a.seg_n = out_features; a.nseg = 1;
  a.act = activation; a.res = nullptr; a.res_stride = 0;
  a.out = out; a.out_stride = out_stride; a.bf16 = dtype == PA_DTYPE_BF16;
  a.row_sel = row_index; a.sel_group = group_rows;
  PA_CHECK_ARG((reinterpret_cast<uintptr_t>(token_keys) & 7) == 0, "token_keys must be 8-byte aligned");
  PA_CHECK_ARG(token_keys == nullptr || token_keys_stride >= 1, "token_keys_stride must be >= 1, got %lld",
               (long long)token_keys_stride);
  a.token_keys = reinterpret_cast<unsigned long long*>(token_keys);
  a.keys_stride = token_keys_stride;
  return launch_small_linear(a, static_cast<hipStream_t>(stream));
}

extern "C" int pa_mlp_rows(const void* x, int64_t x_stride, int32_t rows, int32_t d_model,
                           const void* ln_weight, const void* ln_bias, float ln_eps,
                           const void* fc1_weight, const void* fc1_bias, int32_t d_ff, int32_t activation,
                           const void* fc2_weight, const void* fc2_bias,
                           const void* residual, int64_t residual_stride,
                           void* out, int64_t out_stride, int dtype, void* stream) {
  pa_host::clear_error();
  PA_CHECK_ARG(dtype == PA_DTYPE_F32, "mlp rows: dtype must be fp32, got %d", dtype);
  PA_CHECK_ARG(rows >= 0 && rows <= kLinRows, "mlp rows: rows must be in [0, %d], got %d", kLinRows, rows);
  PA_CHECK_ARG(d_model > 0 && d_ff > 0 && d_ff % 16 == 0, "bad sizes: d_model=%d d_ff=%d (d_ff a multiple of 16)",
               d_model, d_ff);
  PA_CHECK_ARG(activation == 0 || activation == 1, "bad activation %d", activation);
  if (rows == 0) return PA_OK;
  PA_CHECK_ARG(x && ln_weight && ln_bias && fc1_weight && fc2_weight && out, "null pointer argument");
  PA_CHECK_ARG(aligned16(x) && aligned16(fc1_weight) && aligned16(fc2_weight) && aligned16(ln_weight) &&
               aligned16(ln_bias) && x_stride % 4 == 0,
               "x, weights and LayerNorm parameters must be 16-byte aligned, x_stride a multiple of 4");
  PA_CHECK_ARG(x_stride >= d_model && out_stride >= d_model && (residual == nullptr || residual_stride >= d_model),
               "row strides smaller than the rows");
  LinArgs a{};
  a.x = x; a.x_stride = x_stride; a.M = rows; a.K = d_model;
  a.ln_w = ln_weight; a.ln_b = ln_bias; a.ln_eps = ln_eps;
  a.w[0] = fc1_weight; a.b[0] = fc1_bias; a.seg_n = d_ff; a.nseg = 1;
  a.act = activation; a.res = nullptr; a.res_stride = 0;
  a.out = nullptr; a.out_stride = 0; a.bf16 = 0;
  a.w2 = fc2_weight; a.b2 = fc2_bias; a.res2 = residual; a.res2_stride = residual_stride;
  a.out2 = out; a.out2_stride = out_stride; a.n2 = d_model;
  return launch_mlp_rows(a, static_cast<hipStream_t>(stream));
}

extern "C" int pa_qkv_append(const void* x, int64_t x_stride, int32_t rows, int32_t d_model,
                             const void* ln_weight, const void* ln_bias, float ln_eps,
                             const void* wq, const void* bq, const void* wk, const void* bk,
                             const void* wv, const void* bv,
                             void* q_out, int64_t q_stride,
                             void* k_pool, void* v_pool, int pool_dtype, int64_t num_blocks,
                             const int32_t* slot_mapping, int32_t num_heads, int32_t head_dim,
                             int32_t block_size, int dtype, void* stream) {
  pa_host::clear_error();
  PA_CHECK_ARG(rows >= 0 && rows <= kLinMaxRows, "rows must be in [0, %d], got %d", kLinMaxRows, rows);
  PA_CHECK_ARG(num_heads > 0 && head_dim > 0 && block_size > 0 && d_model == num_heads * head_dim,
               "d_model must equal num_heads * head_dim");
  PA_CHECK_ARG(pool_dtype == PA_DTYPE_F32 || pool_dtype == PA_DTYPE_BF16, "bad pool dtype %d", pool_dtype);
  PA_CHECK_ARG(lin_dtype_ok(dtype), "bad dtype %d", dtype);
  if (rows == 0) return PA_OK;
  PA_CHECK_ARG(x && wq && wk && wv && q_out && k_pool && v_pool && slot_mapping, "null pointer argument");
  PA_CHECK_ARG((ln_weight == nullptr) == (ln_bias == nullptr), "LayerNorm needs both weight and bias");
  const int vec = elems_per_16b(dtype);
  PA_CHECK_ARG(aligned16(x) && aligned16(wq) && aligned16(wk) && aligned16(wv) && x_stride % vec == 0 &&
               (!ln_weight || (aligned16(ln_weight) && aligned16(ln_bias))),
               "x, weights and LayerNorm parameters must be 16-byte aligned, x_stride a multiple of %d", vec);
  PA_CHECK_ARG(x_stride >= d_model && q_stride >= d_model, "row strides smaller than the rows");
  LinArgs a{};
  a.x = x; a.x_stride = x_stride; a.M = rows; a.K = d_model;
  a.ln_w = ln_weight; a.ln_b = ln_bias; a.ln_eps = ln_eps;
  a.w[0] = wq; a.w[1] = wk; a.w[2] = wv; a.b[0] = bq; a.b[1] = bk; a.b[2] = bv;
  a.seg_n = d_model; a.nseg = 3;
  a.act = 0; a.res = nullptr; a.res_stride = 0;
  a.out = q_out; a.out_stride = q_stride; a.bf16 = dtype == PA_DTYPE_BF16;
  a.k_pool = k_pool; a.v_pool = v_pool; a.pool_bf16 = pool_dtype == PA_DTYPE_BF16; a.num_blocks = num_blocks;
  a.slots = slot_mapping; a.H = num_heads; a.Hd = head_dim; a.bs = block_size;
  return launch_small_linear(a, static_cast<hipStream_t>(stream));
}

extern "C" int pa_embed_rows(const int64_t* ids, const int64_t* pos_start, int32_t batch, int32_t query_len,
                             const void* token_table, int64_t vocab, const void* pos_table, int32_t max_pos,
                             int32_t d_model, void* out, int64_t out_stride, int dtype, void* stream) {
  pa_host::clear_error();
  PA_CHECK_ARG(lin_dtype_ok(dtype), "bad dtype %d", dtype);
  const int vec = elems_per_16b(dtype);
  PA_CHECK_ARG(batch >= 0 && query_len >= 0 && vocab > 0 && max_pos > 0 && d_model > 0 && d_model % vec == 0,
               "bad sizes: batch=%d query_len=%d vocab=%lld max_pos=%d d_model=%d", batch, query_len,
               (long long)vocab, max_pos, d_model);
  const int64_t rows = (int64_t)batch * query_len;
  if (rows == 0) return PA_OK;
  PA_CHECK_ARG(ids && pos_start && token_table && pos_table && out, "null pointer argument");
  PA_CHECK_ARG(aligned16(token_table) && aligned16(pos_table) && aligned16(out) && out_stride % vec == 0 &&
               out_stride >= d_model, "tables and out must be 16-byte aligned, out_stride a multiple of %d", vec);
  if (rows > 0x7fffffffLL) PA_FAIL(PA_ERR_INVALID_ARGUMENT, "grid too large");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == PA_DTYPE_BF16)
    embed_rows_kernel<uint16_t><<<dim3((unsigned)rows), dim3(256), 0, st>>>(
        ids, pos_start, query_len, static_cast<const uint16_t*>(token_table), vocab,
        static_cast<const uint16_t*>(pos_table), max_pos, d_model, static_cast<uint16_t*>(out), out_stride);
  else
    embed_rows_kernel<float><<<dim3((unsigned)rows), dim3(256), 0, st>>>(
        ids, pos_start, query_len, static_cast<const float*>(token_table), vocab,
        static_cast<const float*>(pos_table), max_pos, d_model, static_cast<float*>(out), out_stride);
  PA_CHECK_LAUNCH("embedding kernel");
  return PA_OK;
}
