// Paged decode attention over the block-structured KV cache, for gfx950.
//
// Flash-decoding split-K with the reference's work decomposition and
// workspace layout (src/cuda/kernels/attention.cu:70-210 in Neil456/Redline):
// a workgroup handles one (decode item, kv head, 256-key partition) and all G
// query heads of that kv head's GQA group, so every K/V byte is read once per
// group; partitions are merged by a small reduction kernel when a context
// spans more than one.
//
// The in-workgroup mapping is wave64-first (8 waves per workgroup, 32 keys
// each):
//   * every key of the partition is resolved once to its cache cell (block
//     table lookup) into LDS, so K/V addresses are one LDS read each;
//   * q . k runs on the matrix cores (v_mfma_f32_16x16x32_f16, K as the A
//     operand, the G heads of the group as B columns); the keys are numbered
//     so that each lane receives scores of keys its own row of 16 lanes uses
//     in P . V, and the softmax runs once per (key, head) on that output;
//   * P . V runs on the matrix cores too: V rows (8 elements per lane) are
//     the A operand in a dim order that keeps every element in the lane that
//     loaded it, and the softmax output is the B operand as it stands; the 8
//     waves' partial outputs are combined through LDS (a v_dot2 form of P . V
//     remains selectable);
//   * INT8 codes become exact fp16 values (1152 + code) through byte
//     permutes under an fp16 exponent, without conversion instructions; the
//     constant leaves the q . k and P . V sums through one more MFMA each,
//     whose A operand is -1152 everywhere.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cfloat>
#include <cstdint>
#include <mutex>
#include <type_traits>

#include "device.hpp"
#include "redline_amd/rlk.h"
#include "status.hpp"

namespace rlk {
namespace {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / kWave;
constexpr int kPart = RLK_DECODE_PARTITION_SIZE;  // keys per partition
constexpr int kRedPad = 4;  // floats of padding per row of the waves' partial outputs in LDS

struct AttnArgs {
  rlk_attention_params p;
  rlk_decode_attention_work w;
  int scale16;  // INT8 scales stored as fp16 (extension)
};



// the MFMA operand that takes the 1152 of the biased INT8 codes out of a sum
__device__ __forceinline__ f16x8 minus1152x8() {
  const _Float16 v = static_cast<_Float16>(-1152);
  return f16x8{v, v, v, v, v, v, v, v};
}

template <bool kInt8>
struct Row;

template <>
struct Row<false> {  // 8 fp16 elements, 16 bytes
  using Raw = u32x4;
  __device__ static Raw load(const void* base, uint32_t cell, int D, int e0) {
    return ld16<true>(reinterpret_cast<const u32x4*>(static_cast<const _Float16*>(base) + e0 +
                                                     static_cast<uint64_t>(cell) * D));
  }
  __device__ static f16x8 halves(Raw r) { return __builtin_bit_cast(f16x8, r); }
  __device__ static f32x8 floats(Raw r) { return unpack8(r); }
};

template <>
struct Row<true> {  // 8 int8 codes, 8 bytes
  using Raw = u32x2;
  __device__ static Raw load(const void* base, uint32_t cell, int D, int e0) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(
        static_cast<const int8_t*>(base) + e0 + static_cast<uint64_t>(cell) * D));
  }
  __device__ static f16x8 halves(Raw r) { return int8x8_to_f16(r); }
  __device__ static f32x8 floats(Raw r) {
    return __builtin_convertvector(__builtin_bit_cast(i8x8, r), f32x8);
  }
};

// The 64 / N key slots of a wave (lanes l, l + N, l + 2N, ...) combined,
// every lane receiving the result: slots 16 and 32 lanes apart through the
// permlane row swaps, slots 8 apart (N = 8) through a DPP rotation by 8
// within each row of 16.
__device__ __forceinline__ float ror8(float v) { return dpp<0x128>(v); }  // row_ror:8
template <int N>
__device__ __forceinline__ float slots_sum(float v) {
  if constexpr (N == 8) v += ror8(v);
  return rows_sum<true>(rows_sum<false>(v));
}
template <int N>
__device__ __forceinline__ float slots_max(float v) {
  if constexpr (N == 8) v = fmaxf(v, ror8(v));
  return rows_max<true>(rows_max<false>(v));
}

// ---- one work unit = one (item, kv head, 256-key partition), processed by
// the 8 waves of a workgroup in stages.  A wave owns kPasses passes of kKPP
// keys, 32 consecutive keys in all (key j of pass u is (wave * kPasses + u) *
// kKPP + slot), so a matrix-core tile of 16 keys lies in one or two 16-key
// cache blocks and each K load instruction stays inside them (one address
// translation, few cache lines); the K rows of a unit and its V rows are two
// separate batches of loads, so the persistent form can keep one batch in
// flight while it computes with the other.

template <int D>
struct Geo {
  static constexpr int kLPK = D / 8;             // lanes per key row (16 or 8)
  static constexpr int kKPP = kWave / kLPK;      // keys per wave pass
  static constexpr int kPasses = kPart / (kKPP * kWaves);  // 8 or 4
};

// This thread's coordinates inside a unit.  With kPin the thread index passes
// through an empty asm (no instruction), so that the lane-dependent address
// arithmetic is re-derived per unit rather than hoisted out of the persistent
// loop and kept live across it: the FP16 form needs the registers (hoisted it
// spills), the INT8 form has them and saves the instructions.
struct LaneCoord {
  int tid, wave, slot, e0;
};
template <int D, bool kPin = true>
__device__ __forceinline__ LaneCoord lane_coord() {
  int tid = threadIdx.x;
  if constexpr (kPin) asm volatile("" : "+v"(tid));
  const int lane = tid % kWave;
  return {tid, __builtin_amdgcn_readfirstlane(tid / kWave), lane / Geo<D>::kLPK,
          (lane % Geo<D>::kLPK) * 8};
}
template <int D>
__device__ __forceinline__ int key_of(const LaneCoord& c, int pass) {
  return (c.wave * Geo<D>::kPasses + pass) * Geo<D>::kKPP + c.slot;
}

// The V rows of this thread's keys, in flight.
template <int D, bool kInt8>
struct RowBatch {
  typename Row<kInt8>::Raw r[Geo<D>::kPasses];
};

// Requests every row of this thread's keys of a unit whose first `n` keys
// are in context (cells: the unit's cache cells, in LDS).  Slots past the
// context re-read the last valid row (a cache hit) and are masked out later,
// which keeps every load unconditional: kClamp clamps the key to n - 1 here;
// without it the cells past the context already hold key n - 1's cell
// (write_cells with the unit's key count).
template <int D, bool kInt8, bool kClamp>
__device__ __forceinline__ void issue_rows(RowBatch<D, kInt8>& rb, const void* base,
                                           const int* cells, int n, const LaneCoord& c) {
  // keeps the last reads of the registers being refilled before the loads
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int u = 0; u < Geo<D>::kPasses; ++u)
    rb.r[u] = Row<kInt8>::load(base, cells[kClamp ? min(key_of<D>(c, u), n - 1) : key_of<D>(c, u)], D, c.e0);
  // keeps the scheduler from moving the batch next to its first use
  __builtin_amdgcn_sched_barrier(0);
}

// ---- q . k on the matrix cores.  For each of the wave's two tiles of 16 keys
// one v_mfma_f32_16x16x32_f16 per 32 dims multiplies K (A: 16 keys x 32
// dims) by q (B: 32 dims x 16 columns, column g = head g of the group, the
// columns past G zero).  Lane l supplies A row l % 16 and B column l % 16 at
// k-slot l / 16, and receives D rows 4 (l / 16) + i, column l % 16.
//
// The keys are numbered so that D lands where P . V needs it: tile t, row
// 4 rho + i is key (slot rho, pass 4t + i) for 16 lanes per key (D = 128) and
// (slot 2 rho + t, pass i) for 8 (D = 64).  Lane (rho, g) then holds head g's
// scores of keys its own row of 16 lanes consumes in P . V, and a DPP row
// broadcast of lane g hands head g's probability to the whole row.
template <int D>
__device__ __forceinline__ int mma_slot(int t, int r) {
  return Geo<D>::kLPK == 16 ? r / 4 : 2 * (r / 4) + t;
}
template <int D>
__device__ __forceinline__ int mma_pass(int t, int r) {
  return Geo<D>::kLPK == 16 ? 4 * t + r % 4 : r % 4;
}
template <int D>
__device__ __forceinline__ int mma_key(const LaneCoord& c, int t, int r) {
  return (c.wave * Geo<D>::kPasses + mma_pass<D>(t, r)) * Geo<D>::kKPP + mma_slot<D>(t, r);
}

// K rows of a unit in the matrix-core layout: per tile, lane (j, r) holds the
// 16-byte pieces [64 x + 16 j, +16) of key row r's bytes (x < kLoads), which
// are k-slot j of one (fp16) or two (int8, 8 codes each) MFMA steps.
template <int D, bool kInt8>
struct KBatch {
  static constexpr int kLoads = D * (kInt8 ? 1 : 2) / 64;
  u32x4 r[2][kLoads];
};

// dims of MFMA step `step` held at k-slot j
template <int D, bool kInt8>
__device__ __forceinline__ int step_dim(int step, int j) {
  return kInt8 ? 64 * (step / 2) + 16 * j + 8 * (step % 2) : 32 * step + 8 * j;
}

// FP16 K rows through whole-line loads: the two loads of one 128-byte line
// of the tile's 16 rows take 8 rows each -- lanes r < 8 fetch their own
// row's first half-line and row r + 8's second, lanes r >= 8 row r - 8's
// second half and their own first -- and keys_exchange hands each second
// half to its row's lane (DPP row_ror:8).  FP16: 104.3 -> 103.3 us at C2.
// The INT8 form, bound by its instruction stream, keeps the half-line loads
// (the exchange cost it 59.0 -> 59.8 us).  Ordinary loads either way: with
// the streaming hint the whole-line form took 111 / 68.6 us.
template <int D, bool kInt8>
constexpr bool kKeysFull = !kInt8 && D * 2 >= 128;

template <int D, bool kInt8, bool kClamp>
__device__ __forceinline__ void issue_keys(KBatch<D, kInt8>& kb, const void* base,
                                           const int* cells, int n, const LaneCoord& c) {
  __builtin_amdgcn_sched_barrier(0);  // as in issue_rows
  const int lane = c.tid % kWave, r = lane % 16, j = lane / 16;
  constexpr int kRowBytes = D * (kInt8 ? 1 : 2);
  if constexpr (kKeysFull<D, kInt8>) {
    const bool low = r < 8;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int k0 = mma_key<D>(c, t, low ? r : r - 8), k1 = mma_key<D>(c, t, low ? r + 8 : r);
      const uint32_t c0 = cells[kClamp ? min(k0, n - 1) : k0], c1 = cells[kClamp ? min(k1, n - 1) : k1];
      const char* r0 = static_cast<const char*>(base) + static_cast<uint64_t>(c0) * kRowBytes + 16 * j + (low ? 0 : 64);
      const char* r1 = static_cast<const char*>(base) + static_cast<uint64_t>(c1) * kRowBytes + 16 * j + (low ? 64 : 0);
#pragma unroll
      for (int L = 0; L < KBatch<D, kInt8>::kLoads / 2; ++L) {
        kb.r[t][2 * L] = *reinterpret_cast<const u32x4*>(r0 + 128 * L);
        kb.r[t][2 * L + 1] = *reinterpret_cast<const u32x4*>(r1 + 128 * L);
      }
    }
  } else {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int key = mma_key<D>(c, t, r);
      const uint32_t cell = cells[kClamp ? min(key, n - 1) : key];  // cells are >= 0
      const char* row = static_cast<const char*>(base) + 16 * j + static_cast<uint64_t>(cell) * kRowBytes;
      // Ordinary (temporal) loads: an instruction takes 64 bytes of each of
      // 16 rows, half of a cache line, and the next one takes the other
      // half; with the streaming hint the second half was fetched again
      // (INT8: 75.5 -> 62.0 us with ordinary loads).
#pragma unroll
      for (int x = 0; x < KBatch<D, kInt8>::kLoads; ++x)
        kb.r[t][x] = *reinterpret_cast<const u32x4*>(row + 64 * x);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
}

// The K rows in the matrix-core layout (lane (j, r): pieces [64 x + 16 j,
// +16) of row r) from the whole-line loads of issue_keys.
template <int D, bool kInt8>
__device__ __forceinline__ KBatch<D, kInt8> keys_exchange(const KBatch<D, kInt8>& kb, const LaneCoord& c) {
  if constexpr (!kKeysFull<D, kInt8>) {
    return kb;
  } else {
    const bool low = (c.tid % 16) < 8;
    KBatch<D, kInt8> out;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int L = 0; L < KBatch<D, kInt8>::kLoads / 2; ++L)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t a = kb.r[t][2 * L][e], b = kb.r[t][2 * L + 1][e];
          out.r[t][2 * L][e] = low ? a : b;
          out.r[t][2 * L + 1][e] = static_cast<uint32_t>(
              __builtin_amdgcn_mov_dpp(static_cast<int>(low ? b : a), 0x128, 0xF, 0xF, false));  // row_ror:8
        }
    return out;
  }
}

// v of lane `g` of each row of 16, to the whole row (DPP row_newbcast)
__device__ __forceinline__ float row_bcast(float v, int g) {
  switch (g) {
    case 0: return dpp<0x150>(v);
    case 1: return dpp<0x151>(v);
    case 2: return dpp<0x152>(v);
    case 3: return dpp<0x153>(v);
    case 4: return dpp<0x154>(v);
    case 5: return dpp<0x155>(v);
    case 6: return dpp<0x156>(v);
    default: return dpp<0x157>(v);
  }
}

// What the softmax hands to P . V: fp16 pairs of probabilities per pass pair
// and head for the v_dot2 form, or the B operand of the MFMA form (this
// lane's 8 keys for its head column).
template <int D, int G, bool kMma>
struct PvOperand {
  f16x2 pp[Geo<D>::kPasses / 2][G];
};
template <int D, int G>
struct PvOperand<D, G, true> {
  f16x8 b;
};

// Scores s = scale * (q_g . k) * k_scale on the matrix cores, then the
// softmax over the wave's keys per head: p = exp(s - m_g) (0 past the
// context), with the wave's max m and sum l per head stored to stat[wave]
// (flash-decoding inside the workgroup; the waves are combined at the
// output).  The probabilities leave in the P . V layout, passes 2h and 2h + 1
// of this lane's key slot as fp16 pairs per head: the operands of
// v_dot2_f32_f16.  `then` runs once the K rows are consumed (the persistent
// form requests the next unit's K rows into the same registers there).
template <int D, int G, bool kInt8, bool kMma, class Then>
__device__ __forceinline__ void wave_softmax(const KBatch<D, kInt8>& kb_in, const _Float16* qs,
                                            const float* ksc, const float* vsc, float scale, int n,
                                            const LaneCoord& c, PvOperand<D, G, kMma>& po,
                                            float (&stat)[kWaves][G][2], bool carry, float& cf,
                                            Then then) {
  constexpr int kSteps = D / 32, kP = Geo<D>::kPasses;
  const int lane = c.tid % kWave, g = lane % 16, rho = lane / 16;
  // q of one MFMA step at a time (B: column g = head g), so only one step's
  // operand is live.  INT8: A holds 1152 + code (int8x8_to_f16_biased), so
  // the scores also collect -1152 * sum_d q[g][d], one MFMA per step with
  // A = -1152 everywhere (the same for every key row), added at the end,
  // instead of a subtract per pair of codes
  f32x4 acc0 = {0.f, 0.f, 0.f, 0.f};
  f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
  const KBatch<D, kInt8> kr = keys_exchange<D, kInt8>(kb_in, c);
#pragma unroll
  for (int st = 0; st < kSteps; ++st) {
    f16x8 qb = {0, 0, 0, 0, 0, 0, 0, 0};
    if (g < G) qb = *reinterpret_cast<const f16x8*>(qs + g * D + step_dim<D, kInt8>(st, rho));
    if constexpr (kInt8) acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(minus1152x8(), qb, acc0, 0, 0, 0);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      f16x8 a;
      if constexpr (kInt8) {
        const u32x4 w = kr.r[t][st / 2];
        a = int8x8_to_f16_biased(st % 2 ? u32x2{w.z, w.w} : u32x2{w.x, w.y});
      } else {
        a = __builtin_bit_cast(f16x8, kr.r[t][st]);
      }
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qb, acc[t], 0, 0, 0);
    }
  }
  if constexpr (kInt8) {
    acc[0] += acc0;
    acc[1] += acc0;
  }
  then();
  // INT8: the k scales of the lane's keys, from LDS, already multiplied by
  // the softmax scale (scale * k_scale, the same product as scale * ks here)
  auto ks = [&](int x) { return kInt8 ? ksc[mma_key<D>(c, x / 4, 4 * rho + x % 4)] : scale; };
  float e[2][4], m, l;
  // keys past the context are masked only in a unit that has such keys
  // (uniform branch: a full unit skips the compares and selects)
  auto softmax = [&](auto masked) {
    constexpr bool kMasked = decltype(masked)::value;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        e[t][i] = !kMasked || mma_key<D>(c, t, 4 * rho + i) < n ? acc[t][i] * ks(4 * t + i) : -FLT_MAX;
    m = e[0][0];
#pragma unroll
    for (int x = 1; x < 8; ++x) m = fmaxf(m, e[x / 4][x % 4]);
    m = rows_max<true>(rows_max<false>(m));
    if (carry) {  // uniform: continue from the wave's (m, l) of the previous partition
      const float m1 = g < G ? stat[c.wave][g][0] : m;
      const float mm = fmaxf(m, m1);
      cf = __expf(m1 - mm);
      m = mm;
    }
    l = 0.f;
#pragma unroll
    for (int x = 0; x < 8; ++x) {
      const float v = !kMasked || mma_key<D>(c, x / 4, 4 * rho + x % 4) < n ? __expf(e[x / 4][x % 4] - m) : 0.f;
      e[x / 4][x % 4] = v;
      l += v;
    }
  };
  if (n >= kPart) softmax(std::false_type{});
  else softmax(std::true_type{});
  l = rows_sum<true>(rows_sum<false>(l));
  if (carry && g < G) l += stat[c.wave][g][1] * cf;
  if (rho == 0 && g < G) {
    stat[c.wave][g][0] = m;
    stat[c.wave][g][1] = l;
  }
  if constexpr (kMma) {
    // B operand of the P . V MFMA (K = 32 keys x N = 16 head columns): lane
    // (rho, g) supplies k = 8 rho + 4 t + i, the scores it holds, times the
    // key's INT8 v scale
    f16x8 b;
#pragma unroll
    for (int x = 0; x < 8; ++x) {
      float v = e[x / 4][x % 4];
      if constexpr (kInt8) v *= vsc[mma_key<D>(c, x / 4, 4 * rho + x % 4)];
      b[x] = static_cast<_Float16>(v);
    }
    po.b = b;
    return;
  } else {
  auto& pp = po.pp;
  (void)vsc;
  // to the P . V layout: pass u of this lane's key slot is (t, i) = (u / 4,
  // u % 4) of its row (D = 128), or (t, i) = (half of the row, u) (D = 64)
#pragma unroll
  for (int h = 0; h < kP / 2; ++h)
#pragma unroll
    for (int gg = 0; gg < G; ++gg) {
      float pr[2];
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int u = 2 * h + k;
        if constexpr (Geo<D>::kLPK == 16) {
          pr[k] = row_bcast(e[u / 4][u % 4], gg);
        } else {
          const float x0 = row_bcast(e[0][u], gg), x1 = row_bcast(e[1][u], gg);
          pr[k] = (lane % 16) < 8 ? x0 : x1;
        }
      }
      pp[h][gg] = f16x2{static_cast<_Float16>(pr[0]), static_cast<_Float16>(pr[1])};
    }
  }
}

// P . V for this thread's 8 output dims and G heads, fp32 accumulation of
// v_dot2_f32_f16 over pairs of keys; then the wave's key slots are summed and
// the wave's partial output written to red[wave].
//
// The slot sum is a transpose-reduction: one permlane16 swap of two values
// followed by one add leaves the sum over a pair of rows of the first value
// in even rows and of the second in odd rows, so each level halves the
// values a lane carries.  After the row-pair (16 lanes) and row-half (32
// lanes) levels, row r holds the wave-wide sum of flat value 4i + r
// (flat = g * 8 + x) as z[i].  With 8 lanes per key (D = 64) the two slots
// of a row are first summed by a DPP rotation.
// `then` runs once the V rows are consumed and the first level of the slot
// sum has halved the accumulators (the persistent form requests the next
// unit's V rows into the same registers there).
template <int D, int G, bool kInt8, class Then>
__device__ __forceinline__ void wave_pv(const RowBatch<D, kInt8>& vb, const float* vsc,
                                        const PvOperand<D, G, false>& po, const LaneCoord& c,
                                        float (&red)[kWaves][G][D + kRedPad], Then then) {
  constexpr int kP = Geo<D>::kPasses, kN = G * 8;
  const auto& pp = po.pp;
  float v[kN];
#pragma unroll
  for (int h = 0; h < kP / 2; ++h) {
    f16x2 vv[8];  // element x of the pass pair's two keys
    if constexpr (kInt8) {
      int8x8_pairs_to_f16x2(vb.r[2 * h], vb.r[2 * h + 1], vv);
    } else {
      const f16x8 va = Row<kInt8>::halves(vb.r[2 * h]), vb2 = Row<kInt8>::halves(vb.r[2 * h + 1]);
#pragma unroll
      for (int x = 0; x < 8; ++x) vv[x] = f16x2{va[x], vb2[x]};
    }
    f16x2 ph[G];
#pragma unroll
    for (int g = 0; g < G; ++g) ph[g] = pp[h][g];
    if constexpr (kInt8) {  // p * v_scale, per key
      const f16x2 vs = {static_cast<_Float16>(vsc[key_of<D>(c, 2 * h)]),
                        static_cast<_Float16>(vsc[key_of<D>(c, 2 * h + 1)])};
#pragma unroll
      for (int g = 0; g < G; ++g) ph[g] *= vs;
    }
#pragma unroll
    for (int x = 0; x < 8; ++x) {
#pragma unroll
      for (int g = 0; g < G; ++g)  // the first pair starts from 0 (no zeroed accumulator)
        v[g * 8 + x] = __builtin_amdgcn_fdot2(ph[g], vv[x], h == 0 ? 0.f : v[g * 8 + x], false);
    }
  }
  if constexpr (Geo<D>::kLPK == 8) {
#pragma unroll
    for (int i = 0; i < kN; ++i) v[i] += ror8(v[i]);
  }
  float w[kN / 2];
#pragma unroll
  for (int i = 0; i < kN / 2; ++i) {
    float a = v[2 * i], b = v[2 * i + 1];
    swap_rows_pair<false>(a, b);
    w[i] = a + b;
  }
  then();  // after the first level, with half the accumulators live
  float z[kN / 4];
#pragma unroll
  for (int i = 0; i < kN / 4; ++i) {
    float a = w[2 * i], b = w[2 * i + 1];
    swap_rows_pair<true>(a, b);
    z[i] = a + b;
  }
  const int lane = c.tid % kWave, r = lane / 16;
  if (Geo<D>::kLPK == 16 || lane % 16 < 8) {
#pragma unroll
    for (int i = 0; i < kN / 4; ++i) {
      const int f = 4 * i + r;
      red[c.wave][f / 8][c.e0 + f % 8] = z[i];
    }
  }
}

// INT8 codes of 8 keys (the 8 k-slots of an MFMA operand) at 4 dims to
// fp16: w[kk] holds key kk's codes of the 4 dims, sign bits already flipped
// (code + 128 in each byte); a[j][kk] = 1152 + code of dim j of key kk,
// exactly.  Bytes of keys (2p, 2p + 1) are interleaved by two permutes, then
// each pair gets the 0x64 high bytes (fp16 1024 + byte); the constant 1152
// is removed from the P . V sums (wave_pv_mma), not per code.
__device__ __forceinline__ void int8_cols_to_f16_biased(const uint32_t (&w)[8], f16x8 (&a)[4]) {
#pragma unroll
  for (int pr = 0; pr < 4; ++pr) {
    // selectors 0-3 pick from the second source, 4-7 from the first
    const uint32_t t01 = __builtin_amdgcn_perm(w[2 * pr + 1], w[2 * pr], 0x05010400u);
    const uint32_t t23 = __builtin_amdgcn_perm(w[2 * pr + 1], w[2 * pr], 0x07030602u);
    const uint32_t h[4] = {__builtin_amdgcn_perm(0x64646464u, t01, 0x04010400u),
                           __builtin_amdgcn_perm(0x64646464u, t01, 0x04030402u),
                           __builtin_amdgcn_perm(0x64646464u, t23, 0x04010400u),
                           __builtin_amdgcn_perm(0x64646464u, t23, 0x04030402u)};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f16x2 v = __builtin_bit_cast(f16x2, h[j]);
      a[j][2 * pr] = v[0];
      a[j][2 * pr + 1] = v[1];
    }
  }
}

// P . V on the matrix cores: per dim tile, one v_mfma_f32_16x16x32_f16 with V
// as A (16 dims x 32 keys: the wave's keys) and the probabilities as B (32
// keys x 16 head columns, from the softmax).  The dims of a tile are chosen
// so that every lane feeds A from rows it already holds: lane (rho, m)
// supplies A row m at k-slot rho, keys k = 8 rho + kk.
//   D = 128 (16 lanes per key row): lane m holds dims 8m .. 8m + 7 of its key
//     slot rho over the 8 passes kk; tile dt takes dim 8m + dt, i.e. element
//     dt of each of the lane's 8 rows -- no data leaves the lane.
//   D = 64 (8 lanes per key row): the k-slot's keys span slots 2 rho and
//     2 rho + 1 (passes 0..3 each), held by lanes m and m ^ 8; tile dt takes
//     dim 8 (m % 8) + 4 (m / 8) + dt, so each lane keeps half of its row
//     elements and receives the other slot's half from lane m ^ 8 (one DPP
//     row rotation by 8 per dword).
// Output: lane (rho, g) receives rows 4 rho + i of head column g, i.e. head
// g's partial output at the dims of rows 4 rho + i, written to red[wave] for
// g < G.  `then` runs once the V rows are consumed.
template <int D, int G, bool kInt8, bool kCarry, class Then>
__device__ __forceinline__ void wave_pv_mma(const RowBatch<D, kInt8>& vb, const PvOperand<D, G, true>& po,
                                            const LaneCoord& c, float (&red)[kWaves][G][D + kRedPad],
                                            float cf, Then then) {
  constexpr int kTiles = D / 16;
  const int lane = c.tid % kWave, rho = lane / 16, m = lane % 16;
  f16x8 a[kTiles];
  if constexpr (D == 128) {
    if constexpr (!kInt8) {
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        const f16x8 row = __builtin_bit_cast(f16x8, vb.r[kk]);
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) a[dt][kk] = row[dt];
      }
    } else {
#pragma unroll
      for (int half = 0; half < 2; ++half) {  // dims 4 half .. 4 half + 3 of the lane's 8
        uint32_t w[8];
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) w[kk] = vb.r[kk][half] ^ 0x80808080u;
        f16x8 q[4];
        int8_cols_to_f16_biased(w, q);
#pragma unroll
        for (int j = 0; j < 4; ++j) a[4 * half + j] = q[j];
      }
    }
  } else {  // D = 64: keep half the row elements, swap the other half with lane m ^ 8
    const bool t1 = m >= 8;  // this lane's key slot is 2 rho + 1 (k-slots 4..7)
    if constexpr (!kInt8) {
      u32x2 own[4], other[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const u32x4 r = vb.r[u];
        const u32x2 lo = {r.x, r.y}, hi = {r.z, r.w};
        own[u] = t1 ? hi : lo;
        const u32x2 send = t1 ? lo : hi;  // what the partner keeps
        other[u] = u32x2{static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(send.x), 0x128, 0xF, 0xF, false)),
                         static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(send.y), 0x128, 0xF, 0xF, false))};
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const f16x4 mine = __builtin_bit_cast(f16x4, own[u]), theirs = __builtin_bit_cast(f16x4, other[u]);
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
          a[dt][u] = t1 ? theirs[dt] : mine[dt];      // slot 2 rho, pass u
          a[dt][4 + u] = t1 ? mine[dt] : theirs[dt];  // slot 2 rho + 1, pass u
        }
      }
    } else {
      uint32_t w[8];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const u32x2 r = vb.r[u];
        const uint32_t own = t1 ? r.y : r.x, send = t1 ? r.x : r.y;
        const uint32_t other = static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(send), 0x128, 0xF, 0xF, false));
        w[u] = (t1 ? other : own) ^ 0x80808080u;
        w[4 + u] = (t1 ? own : other) ^ 0x80808080u;
      }
      int8_cols_to_f16_biased(w, a);
    }
  }
  // INT8: A holds 1152 + code, so every tile starts from -1152 * sum_k b[k][g]
  // (one MFMA with A = -1152 everywhere, the same for every dim row)
  f32x4 o0 = {0.f, 0.f, 0.f, 0.f};
  if constexpr (kInt8) o0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(minus1152x8(), po.b, o0, 0, 0, 0);
#pragma unroll
  for (int dt = 0; dt < kTiles; ++dt) {
    const f32x4 o = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[dt], po.b, o0, 0, 0, 0);
    if (m < G) {
      auto dim = [&](int i) {
        const int r = 4 * rho + i;
        return D == 128 ? 8 * r + dt : 8 * (r % 8) + 4 * (r / 8) + dt;
      };
      if constexpr (kCarry) {  // onto the run's partial so far, rescaled by e^(m_prev - M) (cf)
        float prev[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) prev[i] = red[c.wave][m][dim(i)];
#pragma unroll
        for (int i = 0; i < 4; ++i) red[c.wave][m][dim(i)] = fmaf(prev[i], cf, o[i]);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) red[c.wave][m][dim(i)] = o[i];
      }
    }
  }
  // The V registers are free once every tile is consumed: the next unit's
  // rows go out only now, so the operand tiles need not all be live beside
  // the refilled batch.
  then();
}

// Combines the waves of a unit: M = max m_w, L = sum e^(m_w - M) l_w,
// o = sum e^(m_w - M) o_w; written as the output row o / L (one partition)
// or as the unit's split-K partial row o with its (M, L) in slot `part`.  A
// unit that ran through partitions part .. part_end marks slots part + 1 ..
// part_end empty (sum -1, which no sum of exponentials takes; the merge skips
// them).  With D a multiple
// of 64 every lane of a wave serves the same head g, so the weights are
// computed once per wave: lane l takes wave l % 8's statistics, the max is a
// reduction over 8 lanes, and lanes 0-7 leave e^(m_w - M) and l_w in the
// wave's own LDS slots `wgt`, which the wave reads back (LDS accesses of one
// wave complete in order; no barrier).  The sums run in wave order as fmas,
// so every lane forms the same L and o as a per-lane loop over the waves.
template <int D, int G, bool kMark = false>
__device__ __forceinline__ void combine_waves(const AttnArgs& args, const float (&red)[kWaves][G][D + kRedPad],
                                              const float (&stat)[kWaves][G][2],
                                              float (&wgt)[kWaves][2][kWaves], int tid, int item,
                                              int token, int num_parts, int part, int kvh,
                                              int part_end = -1) {
  static_assert(kWaves == 8 && D % kWave == 0, "one head per wave, 8 waves per workgroup");
  const rlk_attention_params& p = args.p;
  const rlk_decode_attention_work& w = args.w;
  const int wave = tid / kWave, lane = tid % kWave;
  for (int i = tid; i < G * D; i += kThreads) {  // uniform over a wave
    const int g = i / D, d = i % D;
    const int ww = lane % kWaves;
    const float mw = stat[ww][g][0];
    const float M = group_max<kWaves>(mw);
    if (lane < kWaves) {
      wgt[wave][0][lane] = __expf(mw - M);
      wgt[wave][1][lane] = stat[lane][g][1];
    }
    float L = 0.f, o = 0.f;
#pragma unroll
    for (int v = 0; v < kWaves; ++v) {
      const float f = wgt[wave][0][v];
      L += f * wgt[wave][1][v];
      o += f * red[v][g][d];
    }
    const int h = kvh * G + g;
    if (num_parts == 1) {
      reinterpret_cast<_Float16*>(p.out)[static_cast<int64_t>(token) * p.num_heads * D + h * D + d] =
          static_cast<_Float16>(o / L);
    } else {  // the partition's partial, not divided by its sum L (the merge weighs it by e^(M - max))
      const int64_t row = (static_cast<int64_t>(item) * p.num_heads + h) * w.max_partitions + part;
      w.ws_out[row * D + d] = o;
      if (d == 0) {
        w.ws_max[row] = M;
        w.ws_sum[row] = L;
      }
      if constexpr (kMark)
        for (int j = 1 + d; j <= part_end - part; j += D) w.ws_sum[row + j] = -1.f;
    }
  }
}

// LDS of the unit stages.  cells and q are double-buffered in the persistent
// form (the next unit's are written while the current one computes).
template <int D, int G>
struct UnitLds {
  float red[kWaves][G][D + kRedPad];  // each wave's P . V partial
  float stat[kWaves][G][2];  // each wave's (max, sum) per head
  float wgt[kWaves][2][kWaves];  // per wave: the combine's e^(m_w - M) and l_w of every wave
  int cell[2][kPart];        // cache cell of each key of the partition
  float ksc[2][kPart];       // its INT8 k scale times the softmax scale, and v scale
  float vsc[2][kPart];
  alignas(16) _Float16 q[2][G * D];
};

// Cache cells of a partition's keys, from this thread's block-table entry
// `blk` for key min(tid, nkeys - 1) (threads tid < 256; blk < 0 past the
// table: nothing written); the key's INT8 scales are requested into ks / vs
// as raw bits (0 when there is no cell; scale_value converts them where they
// are written to LDS, so no wait follows the request).  With nkeys = the
// partition's keys in context, the keys past the context get the last key's
// cell and scales.
template <bool kInt8>
__device__ __forceinline__ void write_cells(int* cells, const AttnArgs& args, int tid, int blk,
                                            int part, int kvh, uint32_t& ks, uint32_t& vs,
                                            int nkeys = kPart) {
  const rlk_attention_params& p = args.p;
  ks = 0;
  vs = 0;
  if (tid < kPart && blk >= 0) {
    const int bs = p.kv.block_size;
    const int pos = part * kPart + min(tid, nkeys - 1);
    const int cell = (blk * p.kv.num_kv_heads + kvh) * bs + (pos - (pos / bs) * bs);
    cells[tid] = cell;
    if constexpr (kInt8) {
      if (args.scale16) {  // uniform
        ks = reinterpret_cast<const uint16_t*>(p.kv.k_scale)[cell];
        vs = reinterpret_cast<const uint16_t*>(p.kv.v_scale)[cell];
      } else {
        ks = reinterpret_cast<const uint32_t*>(p.kv.k_scale)[cell];
        vs = reinterpret_cast<const uint32_t*>(p.kv.v_scale)[cell];
      }
    }
  }
}

// An INT8 scale from its raw bits (fp16 in the low half with scale16).
__device__ __forceinline__ float scale_value(uint32_t raw, int scale16) {
  return scale16 ? static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(raw)))
                 : __builtin_bit_cast(float, raw);
}

// q of the G heads of a kv head: G * D fp16 contiguous in the token's row,
// one 16-byte piece per thread kPart <= tid < kPart + G * D / 8.
template <int D, int G>
__device__ __forceinline__ bool q_piece(int tid) {
  return tid >= kPart && tid < kPart + G * D / 8;
}
template <int D, int G>
__device__ __forceinline__ u32x4 load_q_piece(const rlk_attention_params& p, int tid, int token, int kvh) {
  const _Float16* q = reinterpret_cast<const _Float16*>(p.q) + static_cast<int64_t>(token) * p.q_stride +
                      kvh * G * D + (tid - kPart) * 8;
  return load16(q);
}

// Block-table entry of key min(tid, nkeys - 1) of a partition (threads
// tid < 256), or -1 past the table.  Table rows are padded with block 0, so every entry inside
// the row is a valid block.
__device__ __forceinline__ int table_entry(const rlk_attention_params& p, int tid, int seq, int part,
                                           int nkeys = kPart) {
  const int bi = (part * kPart + min(tid, nkeys - 1)) / p.kv.block_size;
  if (tid >= kPart || bi >= p.max_blocks_per_seq) return -1;
  return p.block_tables[static_cast<int64_t>(seq) * p.max_blocks_per_seq + bi];
}

// Persistent form.  Every workgroup first reads each decode item's token,
// sequence and context into LDS and prefix-sums the partitions per item; the
// work units -- only those inside a context -- are then split into contiguous
// ranges, one per workgroup.  With kSeg (the FP16 MFMA form) the units run
// (item, kv head, partition), partition fastest, so a range holds runs of
// consecutive partitions of one (item, kv head): each wave carries its (m, l)
// and partial output through a run (rescaled by e^(m_prev - M) at each
// partition), and the waves are combined once per run, into the workspace slot
// of its first partition; the run's other slots are marked empty.  The other
// forms run (item, partition, kv head), kv head fastest (a partition's block
// table entries and neighbouring K/V rows stay together), and combine every
// unit.  The INT8 scales of
// a partition's keys are fetched once, by the threads that resolve its cells,
// into LDS next to the cells.
//
// The partitions of a range are software-pipelined across their two row
// batches:
//   wait K(n) -> q . k -> request K(n+1) -> softmax -> wait V(n) -> P . V
//   -> request V(n+1) -> slot sums -> barrier -> combine (at a run's end),
//   write cells(n+2) -> barrier
// so each batch is requested as soon as its registers are free and one is
// always in flight while the other is consumed, in the registers a
// non-pipelined unit needs.  Cells and q of later partitions are staged in
// LDS (double-buffered), their block-table entries and q requested one ahead.
constexpr int kMaxItemsLds = 2048;

struct UnitPos {
  int item, part, kvh;
};

template <int D, int G, bool kInt8, bool kMma>
__global__ __launch_bounds__(kThreads, (G <= 4 ? 4 : 2)) void decode_attention_persistent(AttnArgs args) {
  constexpr bool kSeg = kMma && !kInt8;
  const rlk_attention_params& p = args.p;
  const rlk_decode_attention_work& w = args.w;
  __shared__ UnitLds<D, G> s;
  __shared__ int it_tok[kMaxItemsLds], it_seq[kMaxItemsLds], it_ctx[kMaxItemsLds];
  __shared__ int it_pfx[kMaxItemsLds + 1];  // partitions before item i
  __shared__ int wave_tot[kWaves];
  // Cells of the requests issued past a workgroup's last unit: all cell 0
  // (block 0 exists in every pool), so every lane re-reads one cached row.
  // Issuing them keeps the next unit's loads unconditional; a load issued
  // only on some path makes the compiler copy the batch registers at the
  // loop edge, and a copy waits for every load in flight.
  __shared__ int zero_cells[kPart];
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  if (tid < kPart) zero_cells[tid] = 0;
  const int items = w.num_items, hkv = p.kv.num_kv_heads;

  // Items are split into kThreads contiguous runs; each thread sums its run,
  // the runs are scanned across the workgroup, then each thread writes its
  // run's exclusive prefixes.
  const int per = (items + kThreads - 1) / kThreads;
  const int i0 = min(tid * per, items), i1 = min(i0 + per, items);
  int run = 0;
  for (int i = i0; i < i1; ++i) {
    const int tok = w.item_token[i];
    const int ctx = p.positions[tok] + 1;
    it_tok[i] = tok;
    it_seq[i] = w.item_seq[i];
    it_ctx[i] = ctx;
    run += min((ctx + kPart - 1) / kPart, w.max_partitions);
  }
  int incl = run;  // inclusive scan of runs inside the wave
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int v = __shfl_up(incl, o, kWave);
    if (lane >= o) incl += v;
  }
  if (lane == kWave - 1) wave_tot[wave] = incl;
  __syncthreads();
  int before = incl - run;
  for (int ww = 0; ww < wave; ++ww) before += wave_tot[ww];
  for (int i = i0; i < i1; ++i) {
    it_pfx[i] = before;
    before += min((it_ctx[i] + kPart - 1) / kPart, w.max_partitions);
  }
  if (tid == kThreads - 1) it_pfx[items] = before;
  __syncthreads();

  const int total = it_pfx[items] * hkv;
  const int chunk = (total + gridDim.x - 1) / gridDim.x;
  const int u0 = blockIdx.x * chunk, u1 = min(u0 + chunk, total);
  if (u0 >= u1) return;
  // first unit: binary search of its item (item i's units start at it_pfx[i] * hkv)
  const int pu = u0 / hkv;
  int lo = 0, hi = items - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) / 2;
    if (it_pfx[mid] <= pu) lo = mid; else hi = mid - 1;
  }
  auto keys_in = [&](const UnitPos& q) { return min(kPart, it_ctx[q.item] - q.part * kPart); };
  auto num_parts = [&](const UnitPos& q) {
    return min((it_ctx[q.item] + kPart - 1) / kPart, w.max_partitions);
  };
  auto advance = [&](UnitPos q) {
    if constexpr (kSeg) {  // partition fastest
      if (++q.part == it_pfx[q.item + 1] - it_pfx[q.item]) {
        q.part = 0;
        if (++q.kvh == hkv) {
          q.kvh = 0;
          ++q.item;
        }
      }
    } else {  // kv head fastest
      if (++q.kvh == hkv) {
        q.kvh = 0;
        if (++q.part == it_pfx[q.item + 1] - it_pfx[q.item]) {
          q.part = 0;
          ++q.item;
        }
      }
    }
    return q;
  };

  UnitPos cur;
  if constexpr (kSeg) {
    const int r = u0 - it_pfx[lo] * hkv, np = min((it_ctx[lo] + kPart - 1) / kPart, w.max_partitions);
    cur = {lo, r - (r / np) * np, r / np};
  } else {
    cur = {lo, pu - it_pfx[lo], u0 - pu * hkv};
  }
  UnitPos nxt = u0 + 1 < u1 ? advance(cur) : cur;
  // INT8 scales of key tid of unit n+1, requested in unit n-1 and written to
  // LDS in unit n (the cells of unit n+2 are written there too).
  // The first two units' block-table entries and the first q piece go out
  // together; unit 0's scales reach LDS only after its K/V rows are requested.
  uint32_t sk_next = 0, sv_next = 0, ks0, vs0;
  {
    const int blk0 = table_entry(p, tid, it_seq[cur.item], cur.part, keys_in(cur));
    const int blk1 = u0 + 1 < u1 ? table_entry(p, tid, it_seq[nxt.item], nxt.part, keys_in(nxt)) : -1;
    u32x4 q0 = {0, 0, 0, 0};
    if (q_piece<D, G>(tid)) q0 = load_q_piece<D, G>(p, tid, it_tok[cur.item], cur.kvh);
    write_cells<kInt8>(s.cell[0], args, tid, blk0, cur.part, cur.kvh, ks0, vs0, keys_in(cur));
    write_cells<kInt8>(s.cell[1], args, tid, blk1, nxt.part, nxt.kvh, sk_next, sv_next, keys_in(nxt));
    if (q_piece<D, G>(tid)) store16(s.q[0] + (tid - kPart) * 8, q0);
  }
  __syncthreads();

  KBatch<D, kInt8> kb;
  RowBatch<D, kInt8> vb;
  {
    const LaneCoord c = lane_coord<D, !kInt8>();
    issue_keys<D, kInt8, false>(kb, p.kv.k, s.cell[0], keys_in(cur), c);
    issue_rows<D, kInt8, false>(vb, p.kv.v, s.cell[0], keys_in(cur), c);
  }
  if constexpr (kInt8) {
    if (tid < kPart) {
      s.ksc[0][tid] = p.scale * scale_value(ks0, args.scale16);
      s.vsc[0][tid] = scale_value(vs0, args.scale16);
    }
    __syncthreads();
  }
  int run_first = cur.part;  // first partition of the current run
  bool carry = false;        // the previous unit belongs to the same run
  for (int u = u0; u < u1; ++u) {
    const int b = (u - u0) & 1;
    const bool has1 = u + 1 < u1, has2 = u + 2 < u1;
    const UnitPos nn = has2 ? advance(nxt) : nxt;
    const LaneCoord c = lane_coord<D, !kInt8>();
    // block-table entries of unit n+2 and the q piece of unit n+1, consumed
    // after the first barrier
    const int blk2 = has2 ? table_entry(p, c.tid, it_seq[nn.item], nn.part, keys_in(nn)) : -1;
    u32x4 qn = {0, 0, 0, 0};
    if (has1 && q_piece<D, G>(c.tid)) qn = load_q_piece<D, G>(p, c.tid, it_tok[nxt.item], nxt.kvh);
    // the run ends here unless the next unit is the next partition of this (item, kv head)
    const bool run_end = !kSeg || !has1 || nxt.item != cur.item || nxt.kvh != cur.kvh;

    PvOperand<D, G, kMma> po;
    float cf = 1.f;
    wave_softmax<D, G, kInt8, kMma>(kb, s.q[b], s.ksc[b], s.vsc[b], p.scale, keys_in(cur), c, po,
                                    s.stat, carry, cf, [&] {
      issue_keys<D, kInt8, false>(kb, p.kv.k, has1 ? s.cell[b ^ 1] : zero_cells, 0, c);
    });
    // q(n+1) goes to the buffer q(n-1) used: free since the barriers of unit n-1
    if (has1 && q_piece<D, G>(c.tid)) store16(s.q[b ^ 1] + (c.tid - kPart) * 8, qn);
    auto next_rows = [&] {
      issue_rows<D, kInt8, false>(vb, p.kv.v, has1 ? s.cell[b ^ 1] : zero_cells, 0, c);
    };
    if constexpr (kMma) {
      if (carry) {  // uniform
        wave_pv_mma<D, G, kInt8, true>(vb, po, c, s.red, cf, next_rows);
      } else {
        wave_pv_mma<D, G, kInt8, false>(vb, po, c, s.red, cf, next_rows);
      }
    } else {
      wave_pv<D, G, kInt8>(vb, s.vsc[b], po, c, s.red, next_rows);
    }
    __syncthreads();

    // scales(n+1) go to the buffers unit n-1 read (free since its barriers);
    // cells(n+2) to the buffer cells(n) used, free once every wave has
    // requested V(n), i.e. after this barrier
    if (kInt8 && has1 && c.tid < kPart) {
      s.ksc[b ^ 1][c.tid] = p.scale * scale_value(sk_next, args.scale16);
      s.vsc[b ^ 1][c.tid] = scale_value(sv_next, args.scale16);
    }
    if (has2) write_cells<kInt8>(s.cell[b], args, c.tid, blk2, nn.part, nn.kvh, sk_next, sv_next, keys_in(nn));
    if (run_end)  // uniform
      combine_waves<D, G, kSeg>(args, s.red, s.stat, s.wgt, c.tid, cur.item, it_tok[cur.item],
                                num_parts(cur), kSeg ? run_first : cur.part, cur.kvh, cur.part);
    __syncthreads();
    if constexpr (kSeg) {
      carry = !run_end;
      run_first = run_end ? nxt.part : run_first;
    }
    cur = nxt;
    nxt = nn;
  }
}

// Grid form: one workgroup per (partition, kv head, item), exiting at once
// when the partition lies past the item's context; the same stages, in order.
template <int D, int G, bool kInt8, bool kMma>
__global__ __launch_bounds__(kThreads, (G <= 4 ? 4 : 2)) void decode_attention_kernel(AttnArgs args) {
  const rlk_attention_params& p = args.p;
  const rlk_decode_attention_work& w = args.w;
  __shared__ UnitLds<D, G> s;
  const int part = blockIdx.x, kvh = blockIdx.y, item = blockIdx.z, tid = threadIdx.x;
  const int token = w.item_token[item];
  const int blk = table_entry(p, tid, w.item_seq[item], part);  // issued before the context is known
  const int ctx = p.positions[token] + 1;
  if (part >= (ctx + kPart - 1) / kPart) return;  // uniform over the workgroup (part < max_partitions)
  const int n = min(kPart, ctx - part * kPart);
  {
    uint32_t ks0, vs0;
    write_cells<kInt8>(s.cell[0], args, tid, blk, part, kvh, ks0, vs0);
    if (kInt8 && tid < kPart) {
      s.ksc[0][tid] = p.scale * scale_value(ks0, args.scale16);
      s.vsc[0][tid] = scale_value(vs0, args.scale16);
    }
  }
  if (q_piece<D, G>(tid)) store16(s.q[0] + (tid - kPart) * 8, load_q_piece<D, G>(p, tid, token, kvh));
  __syncthreads();
  const LaneCoord c = lane_coord<D>();
  KBatch<D, kInt8> kb;
  RowBatch<D, kInt8> vb;
  issue_keys<D, kInt8, true>(kb, p.kv.k, s.cell[0], n, c);
  issue_rows<D, kInt8, true>(vb, p.kv.v, s.cell[0], n, c);
  PvOperand<D, G, kMma> po;
  float cf = 1.f;
  wave_softmax<D, G, kInt8, kMma>(kb, s.q[0], s.ksc[0], s.vsc[0], p.scale, n, c, po, s.stat, false, cf,
                                  [] {});
  if constexpr (kMma) {
    wave_pv_mma<D, G, kInt8, false>(vb, po, c, s.red, cf, [] {});
  } else {
    wave_pv<D, G, kInt8>(vb, s.vsc[0], po, c, s.red, [] {});
  }
  __syncthreads();
  combine_waves<D, G>(args, s.red, s.stat, s.wgt, tid, item, token,
                      min((ctx + kPart - 1) / kPart, w.max_partitions), part, kvh);
}

// Merges the split-K partials of one (item, head), one lane per output dim
// (the merge rule of attention.cu:193-210).  A partition's partial row is
// sum_k e^(s_k - m_i) v_k, not divided by its sum l_i; the output is
// sum_i e^(m_i - M) row_i / sum_i e^(m_i - M) l_i with M = max_i m_i.  The
// workspace addresses depend only on the (item, head), so the statistics of
// the first D partitions and the first kEarly partial rows are requested
// before the context is known (token -> position is two dependent reads) and
// masked once the partition count is.  The next kLate rows then go out
// together, rows past the count re-reading the last one (weight 0), and the
// rest kUnroll at a time: up to kEarly + kLate partitions cost three memory
// round trips.  Entries past the count are never used (they may hold anything).
constexpr int kReduceMaxParts = 4096;  // weights kept in LDS (contexts up to 1M keys)

template <int D, bool kRuns>
__global__ __launch_bounds__(D) void decode_reduce_kernel(AttnArgs args) {
  // kRuns: slots absorbed by a persistent workgroup's run hold the sum -1
  // and take no part (weight marker -1, rows never accumulated); slot 0 is
  // always a run's own, so only it is requested before the slots' states
  // are known, and later rows past the count or of absorbed slots re-read it
  constexpr int kEarly = kRuns ? 1 : 4, kLate = kRuns ? 31 : 28;
  constexpr int kUnroll = 8;
  const rlk_attention_params& p = args.p;
  const rlk_decode_attention_work& w = args.w;
  __shared__ float wgt[kReduceMaxParts];
  __shared__ float part_red[D / kWave];
  const int item = blockIdx.x, h = blockIdx.y, d = threadIdx.x, lane = d % kWave, wv = d / kWave;
  const int mp = w.max_partitions;
  const int64_t base = (static_cast<int64_t>(item) * p.num_heads + h) * mp;
  const float* src = w.ws_out + base * D + d;
  const float m0 = d < mp ? w.ws_max[base + d] : -FLT_MAX;
  const float l0 = d < mp ? w.ws_sum[base + d] : 0.f;
  // every wave's view of slots 0..63 (wave 0's own l0)
  const float lw = kRuns && wv > 0 && lane < mp ? w.ws_sum[base + lane] : l0;
  float v0[kEarly];
#pragma unroll
  for (int u = 0; u < kEarly; ++u) v0[u] = u < mp ? src[static_cast<int64_t>(u) * D] : 0.f;
  const int token = w.item_token[item];
  const int ctx = p.positions[token] + 1;
  const int num_parts = min((ctx + kPart - 1) / kPart, mp);
  if (num_parts <= 1) return;  // uniform: written directly by the attention kernel
  // bit j: slot j < 64 holds a partial of its own
  const uint64_t own = kRuns ? __ballot(lane < num_parts && !(lw < 0.f)) : ~0ull;
  float v1[kLate];
#pragma unroll
  for (int u = 0; u < kLate; ++u) {
    const int j = min(kEarly + u, num_parts - 1);
    v1[u] = src[static_cast<int64_t>(kRuns && j < 64 && !((own >> j) & 1) ? 0 : j) * D];
  }

  float mx = d < num_parts && !(kRuns && l0 < 0.f) ? m0 : -FLT_MAX;
  for (int i = d + D; i < num_parts; i += D)
    if (!(kRuns && w.ws_sum[base + i] < 0.f)) mx = fmaxf(mx, w.ws_max[base + i]);
  mx = rows_max<true>(rows_max<false>(group_max<16>(mx)));
  if (lane == 0) part_red[wv] = mx;
  __syncthreads();
  mx = part_red[0];
#pragma unroll
  for (int i = 1; i < D / kWave; ++i) mx = fmaxf(mx, part_red[i]);
  __syncthreads();  // part_red is reused below
  float total = 0.f;
  if (d < num_parts) {
    const float f = __expf(m0 - mx);
    const bool absorbed = kRuns && l0 < 0.f;
    wgt[d] = absorbed ? -1.f : f;
    if (!absorbed) total = f * l0;
  }
  for (int i = d + D; i < num_parts; i += D) {
    const float li = w.ws_sum[base + i];
    const float f = __expf(w.ws_max[base + i] - mx);
    const bool absorbed = kRuns && li < 0.f;
    wgt[i] = absorbed ? -1.f : f;
    if (!absorbed) total += f * li;
  }
  total = wave_sum(total);
  if (lane == 0) part_red[wv] = total;
  __syncthreads();
  total = part_red[0];
#pragma unroll
  for (int i = 1; i < D / kWave; ++i) total += part_red[i];

  float o = 0.f;
#pragma unroll
  for (int u = 0; u < kEarly; ++u)
    if (u < num_parts && !(kRuns && wgt[u] == -1.f)) o += wgt[u] * v0[u];
#pragma unroll
  for (int u = 0; u < kLate; ++u)
    if (kEarly + u < num_parts && !(kRuns && wgt[kEarly + u] == -1.f)) o += wgt[kEarly + u] * v1[u];
  int i = kEarly + kLate;
  for (; i + kUnroll <= num_parts; i += kUnroll) {
    float v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) v[u] = src[static_cast<int64_t>(i + u) * D];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      if (!(kRuns && wgt[i + u] == -1.f)) o += wgt[i + u] * v[u];
  }
  for (; i < num_parts; ++i)
    if (!(kRuns && wgt[i] == -1.f)) o += wgt[i] * src[static_cast<int64_t>(i) * D];
  reinterpret_cast<_Float16*>(p.out)[static_cast<int64_t>(token) * p.num_heads * D + h * D + d] =
      static_cast<_Float16>(o / total);
}

// The persistent form (two workgroups per CU) serves batches of up to
// kMaxItemsLds decode items, the grid form larger ones.  RLK_TUNE_ATTN_PERSIST
// overrides: workgroups per CU for the persistent form, or 0 for the grid form.
// Returns whether the partials were written by runs (absorbed slots marked).
template <int D, int G, bool kMma>
bool launch_gm(const AttnArgs& a, bool int8, hipStream_t stream) {
  const int mode = tune_knob(kAttnPersist, 2);
  if (mode > 0 && a.w.num_items <= kMaxItemsLds) {
    const int64_t units = static_cast<int64_t>(a.w.num_items) * a.w.max_partitions * a.p.kv.num_kv_heads;
    const int blocks = static_cast<int>(std::min<int64_t>(units, static_cast<int64_t>(compute_units()) * mode));
    if (int8) {
      decode_attention_persistent<D, G, true, kMma><<<blocks, kThreads, 0, stream>>>(a);
    } else {
      decode_attention_persistent<D, G, false, kMma><<<blocks, kThreads, 0, stream>>>(a);
    }
    return kMma && !int8;
  }
  const dim3 grid(a.w.max_partitions, a.p.kv.num_kv_heads, a.w.num_items);
  if (int8) {
    decode_attention_kernel<D, G, true, kMma><<<grid, kThreads, 0, stream>>>(a);
  } else {
    decode_attention_kernel<D, G, false, kMma><<<grid, kThreads, 0, stream>>>(a);
  }
  return false;
}

// P . V on the matrix cores (the default: at C2 8% faster with an INT8 cache
// in the persistent form, 11% in the grid form, equal with FP16), or on
// v_dot2 (RLK_TUNE_ATTN_PV = 0).
template <int D, int G>
bool launch_g(const AttnArgs& a, bool int8, hipStream_t stream) {
  if (tune_knob(kAttnPv, 1) == 1) return launch_gm<D, G, true>(a, int8, stream);
  return launch_gm<D, G, false>(a, int8, stream);
}

template <int D>
bool launch_d(const AttnArgs& a, int G, bool int8, hipStream_t stream) {
  bool runs;
  switch (G) {
    case 1: runs = launch_g<D, 1>(a, int8, stream); break;
    case 2: runs = launch_g<D, 2>(a, int8, stream); break;
    case 3: runs = launch_g<D, 3>(a, int8, stream); break;
    case 4: runs = launch_g<D, 4>(a, int8, stream); break;
    case 5: runs = launch_g<D, 5>(a, int8, stream); break;
    case 6: runs = launch_g<D, 6>(a, int8, stream); break;
    case 7: runs = launch_g<D, 7>(a, int8, stream); break;
    case 8: runs = launch_g<D, 8>(a, int8, stream); break;
    default: return false;
  }
  if (a.w.max_partitions > 1) {
    const dim3 grid(a.w.num_items, a.p.num_heads);
    if (runs) {
      decode_reduce_kernel<D, true><<<grid, D, 0, stream>>>(a);
    } else {
      decode_reduce_kernel<D, false><<<grid, D, 0, stream>>>(a);
    }
  }
  return true;
}

}  // namespace
}  // namespace rlk

using namespace rlk;

namespace {

int attention_launch(const rlk_attention_params* p, const rlk_decode_attention_work* w,
                     int scale16, hipStream_t stream) {
  if (p == nullptr || w == nullptr)
    return fail(RLK_EINVAL, "paged_attention_decode: null params or work");
  if (w->num_items <= 0) return RLK_OK;
  const int hkv = p->kv.num_kv_heads;
  if (hkv <= 0 || p->num_heads <= 0 || p->num_heads % hkv != 0)
    return fail(RLK_EINVAL, "num_heads must be a multiple of num_kv_heads (%d, %d)", p->num_heads,
                hkv);
  if (p->kv.head_dim != 64 && p->kv.head_dim != 128)
    return fail(RLK_EUNSUPPORTED, "unsupported head_dim %d", p->kv.head_dim);
  if (p->kv.dtype != RLK_KV_FP16 && p->kv.dtype != RLK_KV_INT8)
    return fail(RLK_EINVAL, "paged_attention_decode: unknown KV dtype %d", p->kv.dtype);
  if (w->num_items > 65535 || p->kv.num_kv_heads > 65535)
    return fail(RLK_EINVAL, "paged_attention_decode: %d items exceed one launch; split the call",
                w->num_items);
  if (w->max_partitions < 1 || p->kv.block_size <= 0)
    return fail(RLK_EINVAL, "paged_attention_decode: bad max_partitions %d or block size %d",
                w->max_partitions, p->kv.block_size);
  if (w->max_partitions > kReduceMaxParts)
    return fail(RLK_EUNSUPPORTED, "paged_attention_decode: max_partitions %d exceeds %d",
                w->max_partitions, kReduceMaxParts);
  if (w->max_partitions > 1 && (w->ws_out == nullptr || w->ws_max == nullptr || w->ws_sum == nullptr))
    return fail(RLK_EINVAL, "paged_attention_decode: split-K workspace is required when "
                            "max_partitions > 1");
  if (p->q == nullptr || p->out == nullptr || p->block_tables == nullptr || p->positions == nullptr ||
      w->item_token == nullptr || w->item_seq == nullptr || p->kv.k == nullptr ||
      p->kv.v == nullptr ||
      (p->kv.dtype == RLK_KV_INT8 && (p->kv.k_scale == nullptr || p->kv.v_scale == nullptr)))
    return fail(RLK_EINVAL, "paged_attention_decode: null pointer argument");
  if (p->q_stride % 8 != 0 || (reinterpret_cast<uintptr_t>(p->q) & 15) != 0)
    return fail(RLK_EINVAL, "paged_attention_decode: q rows must be 16-byte aligned (q_stride %d)",
                p->q_stride);
  AttnArgs a;
  a.p = *p;
  a.w = *w;
  a.scale16 = scale16;
  const int G = p->num_heads / hkv;
  const bool int8 = p->kv.dtype == RLK_KV_INT8;
  const bool ok = p->kv.head_dim == 128 ? launch_d<128>(a, G, int8, stream)
                                        : launch_d<64>(a, G, int8, stream);
  if (!ok) return fail(RLK_EUNSUPPORTED, "unsupported GQA group size %d", G);
  return launch_status("paged_attention_decode");
}

}  // namespace

// ---- the no-allocation form.  Its split-K partials live in a file-scope
// device array, one copy per GPU, instead of a caller workspace.  In host
// code `scratch` names a host-side stand-in, not device memory: the device
// address of each GPU's copy comes from hipGetSymbolAddress, taken once per
// device (with that device current) on the first call there, and only that
// address is handed to kernels.
namespace {

static __device__ __align__(256) unsigned char scratch[RLK_DECODE_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices] = {};

// Device address of the current device's scratch array, or null (message set).
void* device_scratch() {
  int dev = -1;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    fail(RLK_EINVAL, "paged_attention_decode_noalloc: no usable current device (%s)",
         hipGetErrorString(e));
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch[dev] == nullptr) {
    void* ptr = nullptr;
    const hipError_t s = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (s != hipSuccess || ptr == nullptr) {
      fail(static_cast<int>(s), "paged_attention_decode_noalloc: hipGetSymbolAddress failed (%s)",
           hipGetErrorString(s));
      return nullptr;
    }
    g_scratch[dev] = ptr;
  }
  return g_scratch[dev];
}

}  // namespace

extern "C" int rlk_paged_attention_decode_noalloc(const rlk_attention_params* p,
                                                  const rlk_decode_attention_work* w,
                                                  hipStream_t stream) {
  if (p == nullptr || w == nullptr)
    return fail(RLK_EINVAL, "paged_attention_decode_noalloc: null params or work");
  if (w->num_items <= 0) return RLK_OK;
  if (w->max_partitions < 1 || p->num_heads <= 0 || p->kv.head_dim <= 0)
    return fail(RLK_EINVAL, "paged_attention_decode_noalloc: bad max_partitions %d, num_heads %d "
                            "or head_dim %d", w->max_partitions, p->num_heads, p->kv.head_dim);
  // One partition: the kernel writes the output rows directly and reads no
  // split-K scratch, so the array is not resolved at all.
  if (w->max_partitions == 1) {
    rlk_decode_attention_work ws = *w;
    ws.ws_out = nullptr;
    ws.ws_max = nullptr;
    ws.ws_sum = nullptr;
    return attention_launch(p, &ws, 0, stream);
  }
  // partials [items, heads, partitions, D] then max and sum [items, heads,
  // partitions], each region 256-byte aligned; no zeroing is needed (every
  // partition a merge reads is written first by the same call)
  const uint64_t rows = static_cast<uint64_t>(w->num_items) * p->num_heads * w->max_partitions;
  const uint64_t out_bytes = (rows * p->kv.head_dim * 4 + 255) / 256 * 256;
  const uint64_t stat_bytes = (rows * 4 + 255) / 256 * 256;
  const uint64_t need = out_bytes + 2 * stat_bytes;
  if (need > RLK_DECODE_SCRATCH_BYTES)
    return fail(RLK_EINVAL, "paged_attention_decode_noalloc: %d items x %d heads x %d partitions "
                            "need %llu bytes of split-K scratch, more than the %llu available; "
                            "split the call or pass a workspace to paged_attention_decode",
                w->num_items, p->num_heads, w->max_partitions,
                static_cast<unsigned long long>(need),
                static_cast<unsigned long long>(RLK_DECODE_SCRATCH_BYTES));
  char* base = static_cast<char*>(device_scratch());
  if (base == nullptr) return RLK_EINVAL;
  rlk_decode_attention_work ws = *w;
  ws.ws_out = reinterpret_cast<float*>(base);
  ws.ws_max = reinterpret_cast<float*>(base + out_bytes);
  ws.ws_sum = reinterpret_cast<float*>(base + out_bytes + stat_bytes);
  return attention_launch(p, &ws, 0, stream);
}

extern "C" int rlk_paged_attention_decode(const rlk_attention_params* p,
                                          const rlk_decode_attention_work* w,
                                          hipStream_t stream) {
  return attention_launch(p, w, 0, stream);
}

extern "C" int rlk_paged_attention_decode_ex(const rlk_attention_params* p,
                                             const rlk_decode_attention_work* w,
                                             const rlk_attention_options* o, hipStream_t stream) {
  const int scale_dtype = o != nullptr ? o->scale_dtype : RLK_SCALE_F32;
  if (scale_dtype != RLK_SCALE_F32 && scale_dtype != RLK_SCALE_F16)
    return fail(RLK_EINVAL, "paged_attention_decode_ex: unknown scale dtype %d", scale_dtype);
  return attention_launch(p, w, scale_dtype == RLK_SCALE_F16, stream);
}
