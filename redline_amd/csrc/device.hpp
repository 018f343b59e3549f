// Device-side building blocks for the gfx950 kernels: 128-bit vector types,
// fp16 <-> fp32 conversion of 8-element packets, wave64 reductions.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace rlk {

// Native clang vector types map to single 128-bit global_load/store_dwordx4.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef int8_t i8x8 __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;

__device__ __forceinline__ f32x8 unpack8(u32x4 v) {
  return __builtin_convertvector(__builtin_bit_cast(f16x8, v), f32x8);
}

// Round-to-nearest-even fp32 -> fp16 of 8 values, packed into 16 bytes.
__device__ __forceinline__ u32x4 pack8(f32x8 f) {
  return __builtin_bit_cast(u32x4, __builtin_convertvector(f, f16x8));
}

// x rounded to fp16 and back (the rounding points of the fp16 activations).
__device__ __forceinline__ f32x8 round_f16(f32x8 f) {
  return __builtin_convertvector(__builtin_convertvector(f, f16x8), f32x8);
}

__device__ __forceinline__ float round_f16(float f) {
  return static_cast<float>(static_cast<_Float16>(f));
}

// silu(g) rounded to fp16 (elementwise.cu:77): the SwiGLU gate before it
// multiplies up.  exp and the division use the hardware's fast exp2 /
// reciprocal: the result is rounded to fp16 right after, far coarser than
// their error.
__device__ __forceinline__ float silu_f16(float g) {
  return round_f16(__fdividef(g, 1.0f + __expf(-g)));
}

// Butterfly reductions over all 64 lanes of a wavefront; every lane gets the result.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// Max over aligned groups of G consecutive lanes (G a power of two <= 64).
template <int G>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int o = G / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

__device__ __forceinline__ u32x4 load16(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ void store16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }

// 16-byte access with a compile-time cache policy: kNT selects the
// non-temporal (streaming) variant for data touched exactly once, which keeps
// it from displacing reused lines and measurably raises HBM throughput of
// large streaming launches on gfx950.
template <bool kNT>
__device__ __forceinline__ u32x4 ld16(const u32x4* p) {
  if constexpr (kNT) return __builtin_nontemporal_load(p);
  return *p;
}
template <bool kNT>
__device__ __forceinline__ void st16(u32x4* p, u32x4 v) {
  if constexpr (kNT) {
    __builtin_nontemporal_store(v, p);
  } else {
    *p = v;
  }
}
template <bool kNT>
__device__ __forceinline__ void st8(u32x2* p, u32x2 v) {
  if constexpr (kNT) {
    __builtin_nontemporal_store(v, p);
  } else {
    *p = v;
  }
}

}  // namespace rlk
