// Rotary position embedding fused with the paged KV-cache write, for gfx950.
//
// Work decomposition (wave64-first):
//   * a head of D = 128 (64) elements holds D/2 rotation pairs (i, i + D/2);
//     each lane owns 8 consecutive pairs, so a head is LPH = D/16 lanes and
//     every lane moves its data with two 16-byte loads and two 16-byte stores
//     (8 lanes of a D = 128 head write a full 256-byte cache row, coalesced);
//   * one wave64 therefore covers 64/LPH heads of a token at once; WPT waves
//     work on the same token, and the (token, head-group) loop walks the
//     q, k, v heads of the row;
//   * cos/sin for the lane's 8 pairs are loaded once per token (two float4
//     each) and stay in registers for every head the lane visits — the
//     register path needs no LDS staging;
//   * INT8: the per-(token, head) absmax is a 3-step xor butterfly across the
//     head's 8 lanes, no LDS and no barrier.
// Numerics follow src/cuda/kernels/rope_kv.cu:44-84 (Neil456/Redline): the
// rotation is evaluated in fp32 and rounded to fp16; INT8 uses
// scale = amax / 127 (amax over the fp16-rounded values; 1 when amax is 0),
// inv = 1 / scale, code = round-half-even(clamp(x * inv, -127, 127)).
// Contraction into FMA is disabled in the rotation so that the rounding of
// every intermediate is fixed by the source, and the INT8 codes are a
// deterministic function of the inputs.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "device.hpp"
#include "redline_amd/rlk.h"
#include "status.hpp"

namespace rlk {
namespace {

struct RopeArgs {
  _Float16* qkv;
  const int32_t* positions;
  const int32_t* slots;
  const float* cos_t;
  const float* sin_t;
  void* k;
  void* v;
  void* k_scale;  // float[cells], or fp16[cells] when scale16
  void* v_scale;
  const _Float16* bias;  // [heads * D] added before the rotation, or null
  int scale16;
  int num_tokens;
  int hq;
  int hkv;
  int block_size;
};

// Token-level metadata of one row: the cell coordinates of its KV slot and
// the lane's 8 cos / sin values (two float4 of each).
template <int D>
struct TokenMeta {
  f32x8 c, s;
  int slot, blk, off;
};

template <int D>
__device__ __forceinline__ TokenMeta<D> token_meta(const RopeArgs& a, int pos, int slot, int p0) {
  constexpr int kHalf = D / 2;
  TokenMeta<D> m;
  const float* cp = a.cos_t + static_cast<int64_t>(pos) * kHalf + p0;
  const float* sp = a.sin_t + static_cast<int64_t>(pos) * kHalf + p0;
  const f32x4 c0 = *reinterpret_cast<const f32x4*>(cp), c1 = *reinterpret_cast<const f32x4*>(cp + 4);
  const f32x4 s0 = *reinterpret_cast<const f32x4*>(sp), s1 = *reinterpret_cast<const f32x4*>(sp + 4);
  m.c = f32x8{c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
  m.s = f32x8{s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
  m.slot = slot;
  m.blk = 0;
  m.off = 0;
  if (slot >= 0) {
    m.blk = slot / a.block_size;
    m.off = slot - m.blk * a.block_size;
  }
  return m;
}

// The extension's QKV bias: fp16(x + b) per element.  The exact sum of two
// fp16 values fits a double, and its rounding to fp16 equals the rounding of
// the fp32 sum (an fp32 rounding happens only when the operands' exponents
// differ by more than 13, and then the smaller is below a quarter of the
// larger's fp16 spacing), so one packed fp16 add per pair of elements gives
// fp16(float(x) + float(b)) exactly.
__device__ __forceinline__ u32x4 add_bias(u32x4 v, u32x4 b) {
  return __builtin_bit_cast(u32x4, __builtin_bit_cast(f16x8, v) + __builtin_bit_cast(f16x8, b));
}

// One head h of a token row: the lane's 8 pairs (v0 = elements p0..p0+7,
// v1 = the partners D/2 later) are biased, rotated (q, k) and stored back in
// place (q) or into the KV cell of the token's slot (k, v; FP16 or INT8 with
// the per-(token, head) scale).  Every lane of the head's group calls it.
template <int D, bool kInt8>
__device__ __forceinline__ void rope_head(const RopeArgs& a, _Float16* hp, int h, int p0,
                                          u32x4 v0, u32x4 v1, const TokenMeta<D>& m) {
#pragma clang fp contract(off)
  constexpr bool NT = true;  // streaming accesses of whole lines: measured faster at every batch size
  constexpr int kHalf = D / 2;
  constexpr int kLPH = kHalf / 8;
  f32x8 x0 = unpack8(v0);
  f32x8 x1 = unpack8(v1);
  if (h < a.hq + a.hkv) {  // q and k heads rotate; v passes through
    const f32x8 y0 = x0 * m.c - x1 * m.s;
    const f32x8 y1 = x1 * m.c + x0 * m.s;
    x0 = round_f16(y0);
    x1 = round_f16(y1);
  }
  if (h < a.hq) {  // query: back in place
    st16<NT>(reinterpret_cast<u32x4*>(hp + p0), pack8(x0));
    st16<NT>(reinterpret_cast<u32x4*>(hp + kHalf + p0), pack8(x1));
    return;
  }
  if (m.slot < 0) return;
  const bool is_v = h >= a.hq + a.hkv;
  const int kvh = is_v ? h - a.hq - a.hkv : h - a.hq;
  const int64_t cell = (static_cast<int64_t>(m.blk) * a.hkv + kvh) * a.block_size + m.off;
  if constexpr (!kInt8) {
    _Float16* dst = static_cast<_Float16*>(is_v ? a.v : a.k) + cell * D;
    st16<NT>(reinterpret_cast<u32x4*>(dst + p0), pack8(x0));
    st16<NT>(reinterpret_cast<u32x4*>(dst + kHalf + p0), pack8(x1));
  } else {
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fmaxf(__builtin_fabsf(x0[j]), __builtin_fabsf(x1[j])));
    amax = group_max<kLPH>(amax);
    float scale = amax > 0.f ? amax / 127.f : 1.f;
    if (a.scale16) scale = round_f16(scale);  // extension: quantise against the stored fp16 scale
    const float inv = 1.f / scale;
    i8x8 q0, q1;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      q0[j] = static_cast<int8_t>(__builtin_rintf(fminf(fmaxf(x0[j] * inv, -127.f), 127.f)));
      q1[j] = static_cast<int8_t>(__builtin_rintf(fminf(fmaxf(x1[j] * inv, -127.f), 127.f)));
    }
    // An INT8 cell row of D = 128 is one 128-byte line, written as two
    // 64-byte halves (the rotation pairs i and i + D/2 sit in different
    // halves).  Ordinary stores let L2 join the halves before the line goes
    // to HBM; with the streaming hint each half went out on its own (C4:
    // 63.7 against 59.4 us per call).
    int8_t* dst = static_cast<int8_t*>(is_v ? a.v : a.k) + cell * D;
    st8<false>(reinterpret_cast<u32x2*>(dst + p0), __builtin_bit_cast(u32x2, q0));
    st8<false>(reinterpret_cast<u32x2*>(dst + kHalf + p0), __builtin_bit_cast(u32x2, q1));
    if (p0 == 0) {
      void* sp = is_v ? a.v_scale : a.k_scale;
      if (a.scale16) {
        static_cast<_Float16*>(sp)[cell] = static_cast<_Float16>(scale);
      } else {
        static_cast<float*>(sp)[cell] = scale;
      }
    }
  }
}

// The heads of token t that wave `wave` of `nwaves` covers: head group hg =
// wave * heads_per_wave + lane / LPH, then every nwaves * heads_per_wave-th
// head after it.
template <int D, bool kInt8>
__device__ __forceinline__ void rope_token(const RopeArgs& a, int64_t t, int wave, int nwaves,
                                           int lane) {
  constexpr bool NT = true;
  constexpr int kHalf = D / 2;
  constexpr int kLPH = kHalf / 8;            // lanes per head
  constexpr int kHeadsPerWave = kWave / kLPH;
  const int groups = kHeadsPerWave * nwaves;  // heads of one token in flight
  const int hg = wave * kHeadsPerWave + lane / kLPH;
  const int p0 = (lane % kLPH) * 8;  // first pair index owned by this lane
  const int heads = a.hq + 2 * a.hkv;
  _Float16* row = a.qkv + t * heads * D;
  // The activations do not depend on the metadata: issue their loads for the
  // first head before the positions -> cos/sin and slot -> cell chain, so the
  // two latencies overlap instead of adding up.
  u32x4 v0 = {0, 0, 0, 0}, v1 = {0, 0, 0, 0};
  if (hg < heads) {
    v0 = ld16<NT>(reinterpret_cast<const u32x4*>(row + hg * D + p0));
    v1 = ld16<NT>(reinterpret_cast<const u32x4*>(row + hg * D + kHalf + p0));
  }
  const TokenMeta<D> m = token_meta<D>(a, a.positions[t], a.slots[t], p0);
  for (int h = hg; h < heads; h += groups) {  // all lanes of a head share h
    _Float16* hp = row + h * D;
    if (h != hg) {
      v0 = ld16<NT>(reinterpret_cast<const u32x4*>(hp + p0));
      v1 = ld16<NT>(reinterpret_cast<const u32x4*>(hp + kHalf + p0));
    }
    if (a.bias != nullptr) {  // extension: QKV bias
      v0 = add_bias(v0, *reinterpret_cast<const u32x4*>(a.bias + h * D + p0));
      v1 = add_bias(v1, *reinterpret_cast<const u32x4*>(a.bias + h * D + kHalf + p0));
    }
    rope_head<D, kInt8>(a, hp, h, p0, v0, v1, m);
  }
}

// With a QKV bias: K tokens per workgroup, one head per lane group (the
// heads fit the workgroup's waves), so each lane loads its head's bias once
// and keeps it for the K tokens.  The bias costs what the activation loads
// do in the load path -- a load instruction of a wave touches 8 lines, one
// per head -- though every byte of it hits in cache: without the bias loads
// the C5 call takes 49.4 us, with them 52.2.  Two tokens per workgroup halve
// them but lose more elsewhere (52.9 us).
template <int D, bool kInt8, int WPT, int K>
__global__ __launch_bounds__(kWave * WPT) void rope_kv_bias_kernel(RopeArgs a) {
  constexpr bool NT = true;
  constexpr int kHalf = D / 2;
  constexpr int kLPH = kHalf / 8;
  constexpr int kHeadsPerWave = kWave / kLPH;
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int h = wave * kHeadsPerWave + lane / kLPH;
  const int p0 = (lane % kLPH) * 8;
  const int heads = a.hq + 2 * a.hkv;
  if (h >= heads) return;  // whole heads: every lane of a head leaves together
  const u32x4 b0 = *reinterpret_cast<const u32x4*>(a.bias + h * D + p0);
  const u32x4 b1 = *reinterpret_cast<const u32x4*>(a.bias + h * D + kHalf + p0);
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * K;
  const int nt = static_cast<int>(min(static_cast<int64_t>(K), a.num_tokens - t0));
  // every token's loads first (distinct rows: the in-place q stores of one
  // token cannot alias the next token's loads), then the tokens in order
  u32x4 v[K][2];
  TokenMeta<D> m[K];
#pragma unroll
  for (int j = 0; j < K; ++j) {
    if (j < nt) {
      const u32x4* hp = reinterpret_cast<const u32x4*>(a.qkv + ((t0 + j) * heads + h) * D);
      v[j][0] = ld16<NT>(reinterpret_cast<const u32x4*>(reinterpret_cast<const _Float16*>(hp) + p0));
      v[j][1] = ld16<NT>(reinterpret_cast<const u32x4*>(reinterpret_cast<const _Float16*>(hp) + kHalf + p0));
      m[j] = token_meta<D>(a, a.positions[t0 + j], a.slots[t0 + j], p0);
    }
  }
#pragma unroll
  for (int j = 0; j < K; ++j) {
    if (j < nt)
      rope_head<D, kInt8>(a, a.qkv + ((t0 + j) * heads + h) * D, h, p0, add_bias(v[j][0], b0),
                          add_bias(v[j][1], b1), m[j]);
  }
}

// One token per workgroup of WPT waves.
template <int D, bool kInt8, int WPT>
__global__ __launch_bounds__(kWave * WPT) void rope_kv_kernel(RopeArgs a) {
  rope_token<D, kInt8>(a, blockIdx.x, threadIdx.x / kWave, WPT, threadIdx.x % kWave);
}

template <int D, bool kInt8>
void launch_d(const RopeArgs& a, int wpt, hipStream_t stream) {
  switch (wpt) {
    case 1: rope_kv_kernel<D, kInt8, 1><<<a.num_tokens, 1 * kWave, 0, stream>>>(a); break;
    case 2: rope_kv_kernel<D, kInt8, 2><<<a.num_tokens, 2 * kWave, 0, stream>>>(a); break;
    case 3: rope_kv_kernel<D, kInt8, 3><<<a.num_tokens, 3 * kWave, 0, stream>>>(a); break;
    case 4: rope_kv_kernel<D, kInt8, 4><<<a.num_tokens, 4 * kWave, 0, stream>>>(a); break;
    case 5: rope_kv_kernel<D, kInt8, 5><<<a.num_tokens, 5 * kWave, 0, stream>>>(a); break;
    case 6: rope_kv_kernel<D, kInt8, 6><<<a.num_tokens, 6 * kWave, 0, stream>>>(a); break;
    case 7: rope_kv_kernel<D, kInt8, 7><<<a.num_tokens, 7 * kWave, 0, stream>>>(a); break;
    default: rope_kv_kernel<D, kInt8, 8><<<a.num_tokens, 8 * kWave, 0, stream>>>(a); break;
  }
}

template <int D>
void launch_dt(const RopeArgs& a, bool int8, int wpt, hipStream_t stream) {
  int8 ? launch_d<D, true>(a, wpt, stream) : launch_d<D, false>(a, wpt, stream);
}

}  // namespace
}  // namespace rlk

using namespace rlk;

namespace {

int rope_launch(uint16_t* qkv, const int32_t* positions, const int32_t* slot_mapping,
                int num_tokens, int num_heads, const float* cos_table, const float* sin_table,
                const rlk_kv_layer_view* kv, const uint16_t* bias, int scale16,
                hipStream_t stream, const char* what) {
  if (num_tokens <= 0) return RLK_OK;
  if (kv == nullptr) return fail(RLK_EINVAL, "%s: null KV layer view", what);
  if (kv->head_dim != 64 && kv->head_dim != 128)
    return fail(RLK_EUNSUPPORTED, "unsupported head_dim %d (supported: 64, 128)", kv->head_dim);
  if (kv->dtype != RLK_KV_FP16 && kv->dtype != RLK_KV_INT8)
    return fail(RLK_EINVAL, "%s: unknown KV dtype %d", what, kv->dtype);
  if (num_heads < 0 || kv->num_kv_heads < 0 || kv->block_size <= 0)
    return fail(RLK_EINVAL, "%s: bad head counts (%d, %d) or block size %d", what, num_heads,
                kv->num_kv_heads, kv->block_size);
  if (qkv == nullptr || positions == nullptr || slot_mapping == nullptr || cos_table == nullptr ||
      sin_table == nullptr || kv->k == nullptr || kv->v == nullptr ||
      (kv->dtype == RLK_KV_INT8 && (kv->k_scale == nullptr || kv->v_scale == nullptr)))
    return fail(RLK_EINVAL, "%s: null pointer argument", what);
  RopeArgs a;
  a.qkv = reinterpret_cast<_Float16*>(qkv);
  a.positions = positions;
  a.slots = slot_mapping;
  a.cos_t = cos_table;
  a.sin_t = sin_table;
  a.k = kv->k;
  a.v = kv->v;
  a.k_scale = kv->k_scale;
  a.v_scale = kv->v_scale;
  a.bias = reinterpret_cast<const _Float16*>(bias);
  a.scale16 = scale16;
  a.num_tokens = num_tokens;
  a.hq = num_heads;
  a.hkv = kv->num_kv_heads;
  a.block_size = kv->block_size;
  // One token per workgroup of `wpt` waves; a wave covers 64 / (D / 16)
  // heads of the token at once, so wpt = ceil(heads / heads_per_wave) (at most
  // 8) handles every head of the token in one pass: 6 waves for Llama-3.1-8B
  // (48 heads of 128), 5 for Qwen2-7B (36 heads).
  const int heads = num_heads + 2 * kv->num_kv_heads;
  const int heads_per_wave = kWave / (kv->head_dim / 16);
  int wpt = (heads + heads_per_wave - 1) / heads_per_wave;
  // With a bias and every head in one pass: rope_kv_bias_kernel, one token
  // per workgroup (RLK_TUNE_ROPE_BIAS_TOK: 2 tokens, or 0 for the general
  // kernel; C5: 52.2 us against 52.9 and 52.6)
  const int kb = tune_knob(kRopeBiasTok, 1);
  if (bias != nullptr && kb > 0 && wpt <= 8 && tune_knob(kRopeWpt, 0) == 0) {
    const bool i8 = kv->dtype == RLK_KV_INT8;
    auto go = [&](auto kernel, int k) {
      kernel<<<(num_tokens + k - 1) / k, wpt * kWave, 0, stream>>>(a);
    };
#define RLK_ROPE_BIAS_CASE(W)                                                                   \
  case W:                                                                                       \
    if (kv->head_dim == 128) {                                                                  \
      if (kb >= 2) i8 ? go(rope_kv_bias_kernel<128, true, W, 2>, 2) : go(rope_kv_bias_kernel<128, false, W, 2>, 2); \
      else i8 ? go(rope_kv_bias_kernel<128, true, W, 1>, 1) : go(rope_kv_bias_kernel<128, false, W, 1>, 1); \
    } else {                                                                                    \
      if (kb >= 2) i8 ? go(rope_kv_bias_kernel<64, true, W, 2>, 2) : go(rope_kv_bias_kernel<64, false, W, 2>, 2); \
      else i8 ? go(rope_kv_bias_kernel<64, true, W, 1>, 1) : go(rope_kv_bias_kernel<64, false, W, 1>, 1); \
    }                                                                                           \
    return launch_status(what);
    switch (wpt) {
      RLK_ROPE_BIAS_CASE(1)
      RLK_ROPE_BIAS_CASE(2)
      RLK_ROPE_BIAS_CASE(3)
      RLK_ROPE_BIAS_CASE(4)
      RLK_ROPE_BIAS_CASE(5)
      RLK_ROPE_BIAS_CASE(6)
      RLK_ROPE_BIAS_CASE(7)
      RLK_ROPE_BIAS_CASE(8)
      default: break;
    }
#undef RLK_ROPE_BIAS_CASE
  }
  wpt = tune_knob(kRopeWpt, wpt < 1 ? 1 : (wpt > 8 ? 8 : wpt));
  if (wpt < 1) wpt = 1;
  if (wpt > 8) wpt = 8;
  const bool int8 = kv->dtype == RLK_KV_INT8;
  if (kv->head_dim == 128) {
    launch_dt<128>(a, int8, wpt, stream);
  } else {
    launch_dt<64>(a, int8, wpt, stream);
  }
  return launch_status(what);
}

}  // namespace

extern "C" int rlk_rope_and_write_kv(uint16_t* qkv, const int32_t* positions,
                                     const int32_t* slot_mapping, int num_tokens, int num_heads,
                                     const float* cos_table, const float* sin_table,
                                     const rlk_kv_layer_view* kv, hipStream_t stream) {
  return rope_launch(qkv, positions, slot_mapping, num_tokens, num_heads, cos_table, sin_table,
                     kv, nullptr, 0, stream, "rope_and_write_kv");
}

extern "C" int rlk_rope_and_write_kv_ex(uint16_t* qkv, const int32_t* positions,
                                        const int32_t* slot_mapping, int num_tokens,
                                        int num_heads, const float* cos_table,
                                        const float* sin_table, const rlk_kv_layer_view* kv,
                                        const rlk_rope_kv_options* options, hipStream_t stream) {
  const uint16_t* bias = options != nullptr ? options->qkv_bias : nullptr;
  const int scale_dtype = options != nullptr ? options->scale_dtype : RLK_SCALE_F32;
  if (scale_dtype != RLK_SCALE_F32 && scale_dtype != RLK_SCALE_F16)
    return fail(RLK_EINVAL, "rope_and_write_kv_ex: unknown scale dtype %d", scale_dtype);
  return rope_launch(qkv, positions, slot_mapping, num_tokens, num_heads, cos_table, sin_table,
                     kv, bias, scale_dtype == RLK_SCALE_F16, stream, "rope_and_write_kv_ex");
}
