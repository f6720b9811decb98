// Shared device helpers for the gfx950 kernels (wave64, CDNA4).
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

namespace orion {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;

// bf16 bits -> f32 is an exact widening (the reference's `half` crate does
// the same, crates/orion-models/src/loader.rs:85-92).
__device__ __host__ inline float bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
}

// f32 -> bf16, round to nearest even; NaN stays a quiet NaN.
__device__ __host__ inline uint16_t f32_to_bf16(float f) {
  uint32_t u;
  __builtin_memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// The two bf16 halves of a packed dword, widened exactly.
__device__ inline float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ inline float bf16hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// DPP lane exchange inside a row of 16 lanes.  Controls: quad_perm [1,0,3,2]
// (xor 1), quad_perm [2,3,0,1] (xor 2), row_half_mirror (i <-> 7-i within 8),
// row_mirror (i <-> 15-i within 16).  After the xor-1/xor-2 steps a quad holds
// one value, so the mirrors pair each lane with a lane of the other half.
template <int CTRL>
__device__ inline float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}
constexpr int kDppXor1 = 0xB1;
constexpr int kDppXor2 = 0x4E;
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppMirror = 0x140;

// Sum over groups of N consecutive lanes (N in 1..64, power of two); every
// lane of a group ends with the group total.
template <int N>
__device__ inline float group_sum(float v) {
  if constexpr (N >= 2) v += dpp<kDppXor1>(v);
  if constexpr (N >= 4) v += dpp<kDppXor2>(v);
  if constexpr (N >= 8) v += dpp<kDppHalfMirror>(v);
  if constexpr (N >= 16) v += dpp<kDppMirror>(v);
  if constexpr (N >= 32) v += __shfl_xor(v, 16);
  if constexpr (N >= 64) v += __shfl_xor(v, 32);
  return v;
}

template <int N>
__device__ inline float group_max(float v) {
  if constexpr (N >= 2) v = fmaxf(v, dpp<kDppXor1>(v));
  if constexpr (N >= 4) v = fmaxf(v, dpp<kDppXor2>(v));
  if constexpr (N >= 8) v = fmaxf(v, dpp<kDppHalfMirror>(v));
  if constexpr (N >= 16) v = fmaxf(v, dpp<kDppMirror>(v));
  if constexpr (N >= 32) v = fmaxf(v, __shfl_xor(v, 16));
  if constexpr (N >= 64) v = fmaxf(v, __shfl_xor(v, 32));
  return v;
}

__device__ inline float wave_sum(float v) { return group_sum<64>(v); }
__device__ inline float wave_max(float v) { return group_max<64>(v); }

__device__ inline double wave_sum_f64(double v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// Orders LDS traffic between the lanes of one wave: every LDS write issued
// before the call is visible to every lane's LDS read after it.  The fences
// are wavefront-scope (a wave's LDS operations execute in order, so no
// hardware wait is needed); they stop the compiler from moving memory
// operations across the exchange point, which wave_barrier alone does not.
__device__ inline void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Two f32 -> packed (hi, lo) bf16 pairs by truncation: hi = top 16 bits,
// lo = top 16 bits of (x - hi), which is exact in f32.  hi + lo keeps x to
// ~2^-16 relative; 4 VALU ops per pair.  For finite inputs.
__device__ inline void split2_trunc(float x0, float x1, uint32_t& hi, uint32_t& lo) {
  const uint32_t b0 = __float_as_uint(x0), b1 = __float_as_uint(x1);
  hi = __builtin_amdgcn_perm(b1, b0, 0x07060302u);
  const float r0 = x0 - __uint_as_float(b0 & 0xffff0000u);
  const float r1 = x1 - __uint_as_float(b1 & 0xffff0000u);
  lo = __builtin_amdgcn_perm(__float_as_uint(r1), __float_as_uint(r0), 0x07060302u);
}

// split2_trunc for one value: hi = the top 16 bits of x, lo = the top 16
// bits of x - hi (exact in f32).  The subtraction must not contract with a
// product that computed x (fma(a, b, -hi) gives the remainder of the exact
// product, not of the rounded value an f32 store holds), hence the pragma.
__device__ inline void split1_trunc(float x, uint16_t& hi, uint16_t& lo) {
#pragma clang fp contract(off)
  const uint32_t b = __float_as_uint(x);
  hi = (uint16_t)(b >> 16);
  lo = (uint16_t)(__float_as_uint(x - __uint_as_float(b & 0xffff0000u)) >> 16);
}

// Split an f32 into hi + lo bf16 terms: hi = rne(x), lo = rne(x - hi).
// x - hi is exact in f32, so hi + lo carries ~16 significant bits of x.
__device__ inline void split_bf16(float x, uint16_t& hi, uint16_t& lo) {
  hi = f32_to_bf16(x);
  lo = f32_to_bf16(x - bf16_to_f32(hi));
}

// global_load_lds_dwordx4: the wave's 64 lanes each fetch 16 bytes from their
// own global address and the hardware stores them to LDS at lds_wave_base +
// 16 * lane (lds_wave_base must be wave-uniform).  Written as inline asm so
// the compiler's wait-count tracking does not treat every later LDS read as
// a possible reader of the in-flight copy; the kernel orders these copies
// itself (vmcnt(0) then a workgroup barrier before the tile is read).
// Nothing else in the kernels that use it touches M0.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ inline void lds_load16(const void* src, uint32_t lds_wave_base) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off"
               :
               : "s"(lds_wave_base), "v"(src)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// s_waitcnt vmcnt(0) (expcnt and lgkmcnt left at their maxima).
__device__ inline void wait_vmem_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }

}  // namespace orion
