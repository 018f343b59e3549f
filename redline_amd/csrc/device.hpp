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
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
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

// ---- cross-lane reductions without LDS.  Inside rows of 16 lanes they use
// DPP (quad_perm, row_half_mirror, row_mirror); across rows the gfx950
// v_permlane16/32_swap VALU instructions.  __shfl_xor by 16 or 32 would
// compile to ds_bpermute, an LDS round trip per step.

// v as read from the lane that DPP control CTRL selects (within rows of 16).
// Every control used here selects a valid lane of the same row, so no "old"
// value is involved (mov_dpp with bound_ctrl: no zeroing of the destination
// before a plain DPP move).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF,
                                                             0xF, true));
}

// Sum / max over aligned groups of N lanes (N = 2, 4, 8 or 16), every lane
// receiving the result.
template <int N>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (N >= 2) v += dpp<0xB1>(v);    // quad_perm [1,0,3,2]: pairs
  if constexpr (N >= 4) v += dpp<0x4E>(v);    // quad_perm [2,3,0,1]: quads
  if constexpr (N >= 8) v += dpp<0x141>(v);   // row_half_mirror: groups of 8
  if constexpr (N >= 16) v += dpp<0x140>(v);  // row_mirror: groups of 16
  return v;
}
template <int N>
__device__ __forceinline__ float group_max(float v) {
  if constexpr (N >= 2) v = fmaxf(v, dpp<0xB1>(v));
  if constexpr (N >= 4) v = fmaxf(v, dpp<0x4E>(v));
  if constexpr (N >= 8) v = fmaxf(v, dpp<0x141>(v));
  if constexpr (N >= 16) v = fmaxf(v, dpp<0x140>(v));
  return v;
}

// One v_permlane16_swap_b32 (k32 false) or v_permlane32_swap_b32 (k32 true)
// on a and b: the odd rows (16 lanes) or the upper half (32 lanes) of a trade
// places with the even rows or lower half of b.  The instruction writes both
// operands; the compiler's builtin exposes only one of them, so it is issued
// as asm on two in/out operands, after the two wait states a VALU write needs
// before a permlane read.
template <bool k32>
__device__ __forceinline__ void swap_rows_pair(float& a, float& b) {
  unsigned x = __builtin_bit_cast(unsigned, a), y = __builtin_bit_cast(unsigned, b);
  if constexpr (k32) {
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(x), "+v"(y));
  } else {
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(x), "+v"(y));
  }
  a = __builtin_bit_cast(float, x);
  b = __builtin_bit_cast(float, y);
}
// A swap of the rows of v with a copy of itself: the two registers then hold
// v and its partner (16 or 32 lanes apart), in some order.
template <bool k32>
__device__ __forceinline__ void swap_rows(float v, float& a, float& b) {
  a = v;
  b = v;
  swap_rows_pair<k32>(a, b);
}
template <bool k32>
__device__ __forceinline__ float rows_sum(float v) {
  float a, b;
  swap_rows<k32>(v, a, b);
  return a + b;
}
template <bool k32>
__device__ __forceinline__ float rows_max(float v) {
  float a, b;
  swap_rows<k32>(v, a, b);
  return fmaxf(a, b);
}

// Sum over all 64 lanes of a wavefront; every lane gets the result.
__device__ __forceinline__ float wave_sum(float v) {
  return rows_sum<true>(rows_sum<false>(group_sum<16>(v)));
}

// 8 int8 codes to fp16, exactly: each code + 128 (the sign bit flipped)
// becomes the low byte of an fp16 whose high byte is 0x64, i.e. the value
// 1024 + code + 128 (fp16 spacing is 1 on [1024, 2048)); one packed fp16
// subtract of 1152 leaves the code.  2 XORs + 4 byte permutes + 4 packed
// subtracts for 8 codes.  The _biased form stops before the subtract
// (1152 + code, exactly), for callers that remove the constant once from a
// sum instead of once per code.
__device__ __forceinline__ f16x8 int8x8_to_f16_biased(u32x2 r) {
  const uint32_t lo = r.x ^ 0x80808080u, hi = r.y ^ 0x80808080u;
  // v_perm_b32 selectors: bytes 0-3 of the second source, 4 = byte 0 of the
  // first (0x64)
  const u32x4 w = {__builtin_amdgcn_perm(0x64646464u, lo, 0x04010400u),
                   __builtin_amdgcn_perm(0x64646464u, lo, 0x04030402u),
                   __builtin_amdgcn_perm(0x64646464u, hi, 0x04010400u),
                   __builtin_amdgcn_perm(0x64646464u, hi, 0x04030402u)};
  return __builtin_bit_cast(f16x8, w);
}
__device__ __forceinline__ f16x8 int8x8_to_f16(u32x2 r) {
  return int8x8_to_f16_biased(r) - static_cast<_Float16>(1152);
}

// The codes of two rows, paired by element: out[x] = {a[x], b[x]} as exact
// fp16 values, ready for v_dot2 over the two rows.  The bytes are first
// interleaved (a0 b0 a1 b1 ...) by one permute per 4 codes, then each pair
// gets the 0x64 high bytes as in int8x8_to_f16: 4 XORs + 4 + 8 byte permutes
// + 8 packed subtracts for 16 codes, with no repacking of converted halves.
__device__ __forceinline__ void int8x8_pairs_to_f16x2(u32x2 a, u32x2 b, f16x2 (&out)[8]) {
  const uint32_t w[4] = {a.x ^ 0x80808080u, b.x ^ 0x80808080u, a.y ^ 0x80808080u,
                         b.y ^ 0x80808080u};
#pragma unroll
  for (int d = 0; d < 2; ++d) {
    // selectors 0-3 pick from the second source (a), 4-7 from the first (b)
    const uint32_t lo = __builtin_amdgcn_perm(w[2 * d + 1], w[2 * d], 0x05010400u);
    const uint32_t hi = __builtin_amdgcn_perm(w[2 * d + 1], w[2 * d], 0x07030602u);
    const uint32_t t[4] = {__builtin_amdgcn_perm(0x64646464u, lo, 0x04010400u),
                           __builtin_amdgcn_perm(0x64646464u, lo, 0x04030402u),
                           __builtin_amdgcn_perm(0x64646464u, hi, 0x04010400u),
                           __builtin_amdgcn_perm(0x64646464u, hi, 0x04030402u)};
#pragma unroll
    for (int i = 0; i < 4; ++i)
      out[4 * d + i] = __builtin_bit_cast(f16x2, t[i]) - static_cast<_Float16>(1152);
  }
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
