// Shared device helpers and host error plumbing for libpaged_hip (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "paged_hip.h"

namespace pa {

constexpr int kWave = 64;
constexpr int kXcds = 8;  // MI355X: 8 accelerator dies, each with its own L2; workgroup x runs on die x % 8
constexpr float kLog2e = 1.4426950408889634f;
// Finite "minus infinity" for running maxima: exp2(kNegBig - x) is 0 for any real x, and
// exp2(kNegBig - kNegBig) is 1, so an empty state merges without producing NaN.
constexpr float kNegBig = -1.0e30f;

// ---------------------------------------------------------------------------------------------
// Element conversions
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// fp32 -> bf16, round to nearest even; NaN becomes the canonical quiet NaN 0x7fc0.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)0x7fc0u;
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// Two fp32 values to packed bf16 (round to nearest even) with gfx950's v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

template <typename T> struct Elem;
template <> struct Elem<float> {
  __device__ static __forceinline__ float load(const float* p) { return *p; }
  __device__ static __forceinline__ void store(float* p, float v) { *p = v; }
};
template <> struct Elem<uint16_t> {
  __device__ static __forceinline__ float load(const uint16_t* p) { return bf16_to_f32(*p); }
  __device__ static __forceinline__ void store(uint16_t* p, float v) { *p = f32_to_bf16(v); }
};

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// Unpack one 16-byte vector into EPL floats.
template <typename T> struct Vec16;
template <> struct Vec16<float> {
  static constexpr int EPL = 4;
  __device__ static __forceinline__ void unpack(const u32x4& v, float* f) {
    f[0] = __uint_as_float(v[0]); f[1] = __uint_as_float(v[1]);
    f[2] = __uint_as_float(v[2]); f[3] = __uint_as_float(v[3]);
  }
};
template <> struct Vec16<uint16_t> {
  static constexpr int EPL = 8;
  __device__ static __forceinline__ void unpack(const u32x4& v, float* f) {
    f[0] = bf16_lo(v[0]); f[1] = bf16_hi(v[0]); f[2] = bf16_lo(v[1]); f[3] = bf16_hi(v[1]);
    f[4] = bf16_lo(v[2]); f[5] = bf16_hi(v[2]); f[6] = bf16_lo(v[3]); f[7] = bf16_hi(v[3]);
  }
};

// ---------------------------------------------------------------------------------------------
// Cross-lane reductions. DPP row ops stay inside a 16-lane row:
//   0xB1 = quad_perm [1,0,3,2] (xor 1), 0x4E = quad_perm [2,3,0,1] (xor 2),
//   0x141 = row_half_mirror (lane i <-> 7-i within 8), 0x140 = row_mirror (i <-> 15-i within 16).
// After xor1 and xor2 every lane of a quad holds the quad total, so the two mirrors then add the
// other quad / the other half-row. Widths 32 and 64 finish with cross-row shuffles.
// ---------------------------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

template <int W>
__device__ __forceinline__ float group_sum(float x) {
  static_assert(W == 4 || W == 8 || W == 16 || W == 32 || W == 64, "group width");
  x += dpp<0xB1>(x);
  x += dpp<0x4E>(x);
  if constexpr (W >= 8) x += dpp<0x141>(x);
  if constexpr (W >= 16) x += dpp<0x140>(x);
  if constexpr (W >= 32) x += __shfl_xor(x, 16);
  if constexpr (W >= 64) x += __shfl_xor(x, 32);
  return x;
}

template <int W>
__device__ __forceinline__ float group_max(float x) {
  static_assert(W == 4 || W == 8 || W == 16 || W == 32 || W == 64, "group width");
  x = fmaxf(x, dpp<0xB1>(x));
  x = fmaxf(x, dpp<0x4E>(x));
  if constexpr (W >= 8) x = fmaxf(x, dpp<0x141>(x));
  if constexpr (W >= 16) x = fmaxf(x, dpp<0x140>(x));
  if constexpr (W >= 32) x = fmaxf(x, __shfl_xor(x, 16));
  if constexpr (W >= 64) x = fmaxf(x, __shfl_xor(x, 32));
  return x;
}

__device__ __forceinline__ float wave_sum(float x) { return group_sum<64>(x); }
__device__ __forceinline__ float wave_max(float x) { return group_max<64>(x); }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// One LDS-direct load (global_load_lds_dwordx4): lane L reads the 16 bytes at base + voff
// (bytes) and writes them to LDS at lds + 16L; base and lds are wavefront-uniform. Inline
// assembly, so the compiler neither tracks it (the caller waits with vm_wait) nor moves memory
// accesses across it.
__device__ __forceinline__ void stage_load16(const void* base, uint32_t voff, const void* lds) {
  const uint32_t m0 = (uint32_t)(size_t)(const __attribute__((address_space(3))) void*)lds;
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "{m0}"(m0) : "memory");
}
// Wait until at most N vector memory loads of this wavefront are outstanding.
template <int N>
__device__ __forceinline__ void vm_wait() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Wait until this wavefront's LDS reads have returned. The compiler waits for an LDS read only
// where its value is used, which may be after a later LDS-direct load was issued; a ring stage is
// refilled only after this wait, so the refill cannot overwrite bytes a pending read still takes.
__device__ __forceinline__ void lds_read_wait() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

// Number of keys query row i may attend (src/kernels/reference_paged_attention.py:33-42):
// t <= (L - C) + i and t < L.
__device__ __forceinline__ int valid_keys(int L, int C, int i) {
  int n = L - C + 1 + i;
  n = n < L ? n : L;
  return n > 0 ? n : 0;
}

}  // namespace pa

// ---------------------------------------------------------------------------------------------
// Host-side error plumbing
// ---------------------------------------------------------------------------------------------
namespace pa_host {
void set_error(const char* fmt, ...);
void clear_error();
int device_cu_count();  // compute units of the current device (cached per device)
}  // namespace pa_host

#define PA_FAIL(code, ...)                \
  do {                                    \
    ::pa_host::set_error(__VA_ARGS__);    \
    return (code);                        \
  } while (0)

#define PA_CHECK_ARG(cond, ...)                                       \
  do {                                                                \
    if (!(cond)) PA_FAIL(PA_ERR_INVALID_ARGUMENT, __VA_ARGS__);       \
  } while (0)

#define PA_CHECK_LAUNCH(what)                                                          \
  do {                                                                                 \
    hipError_t e__ = hipGetLastError();                                                \
    if (e__ != hipSuccess) PA_FAIL(PA_ERR_HIP, "%s: %s", what, hipGetErrorString(e__)); \
  } while (0)
