// Paged decode attention over the block-structured KV cache, for gfx950.
//
// Flash-decoding split-K with the reference's work decomposition and
// workspace layout (src/cuda/kernels/attention.cu:70-210 in Neil456/Redline):
// a workgroup handles one (decode item, kv head, 256-key partition) and all G
// query heads of that kv head's GQA group, so every K/V byte is read once per
// group; partitions are merged by a small reduction kernel when a context
// spans more than one.
//
// The in-workgroup mapping is wave64-first (8 waves per workgroup):
//   * every key of the partition is resolved once to its cache cell (block
//     table lookup) into LDS, so K/V addresses are one LDS read each;
//   * a K or V row of D elements is D/8 lanes x 8 elements: one 16-byte load
//     per lane for fp16 rows, one 8-byte load for int8 rows; a wave covers
//     64/(D/8) keys per pass and each wave requests all of its K and V rows
//     for the partition before consuming the first (loads past the context
//     re-read the last valid row and are masked, so none is conditional);
//   * q . k runs on fp16 pairs with v_dot2_f32_f16 (fp32 accumulate) and the
//     D/8 lanes of a key finish the dot with DPP row operations (quad_perm,
//     row_half_mirror, row_mirror): no LDS traffic; scores go to LDS;
//   * the softmax statistics of all G heads are reduced together (wave
//     butterflies, one LDS exchange);
//   * P . V keeps the row mapping, each lane accumulating its 8 output dims
//     for the G heads; key slots are folded with xor shuffles inside the wave
//     and across the 8 waves through LDS.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cfloat>
#include <cstdint>

#include "device.hpp"
#include "redline_amd/rlk.h"
#include "status.hpp"

namespace rlk {
namespace {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / kWave;
constexpr int kPart = RLK_DECODE_PARTITION_SIZE;  // keys per partition

struct AttnArgs {
  rlk_attention_params p;
  rlk_decode_attention_work w;

};

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8v __attribute__((ext_vector_type(8)));

template <bool kInt8>
struct Row;

template <>
struct Row<false> {  // 8 fp16 elements, 16 bytes
  using Raw = u32x4;
  __device__ static Raw load(const void* base, int64_t cell, int D, int e0) {
    return ld16<true>(reinterpret_cast<const u32x4*>(static_cast<const _Float16*>(base) + cell * D + e0));
  }
  __device__ static f16x8v halves(Raw r) { return __builtin_bit_cast(f16x8v, r); }
  __device__ static f32x8 floats(Raw r) { return unpack8(r); }
};

template <>
struct Row<true> {  // 8 int8 codes, 8 bytes
  using Raw = u32x2;
  __device__ static Raw load(const void* base, int64_t cell, int D, int e0) {
    return __builtin_nontemporal_load(
        reinterpret_cast<const u32x2*>(static_cast<const int8_t*>(base) + cell * D + e0));
  }
  // |code| <= 127 is exact in fp16
  __device__ static f16x8v halves(Raw r) {
    return __builtin_convertvector(__builtin_bit_cast(i8x8, r), f16x8v);
  }
  __device__ static f32x8 floats(Raw r) {
    return __builtin_convertvector(__builtin_bit_cast(i8x8, r), f32x8);
  }
};

// LDS of one work unit.
template <int D, int G>
struct UnitLds {
  float red[kWaves][G][D];   // each wave's P . V partial
  float stat[kWaves][G][2];  // each wave's (max, sum) per head
  int cell[kPart];           // cache cell of each key of the partition
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

// One work unit = one (item, kv head, 256-key partition), processed by the 8
// waves of the workgroup.  `blk` is this thread's block-table entry for key
// `tid` of the partition (threads tid < 256; -1 past the table).  Each wave
// owns kPasses passes of kKPP keys; all of its K and V rows are requested
// before the first is used, so a workgroup keeps its whole partition (256
// keys x 2 rows) in flight at once.  Starts and ends with every thread of the
// workgroup.
template <int D, int G, bool kInt8>
__device__ __forceinline__ void attend_unit(const AttnArgs& args, UnitLds<D, G>& lds, int item,
                                            int token, int ctx, int part, int kvh, int blk) {
  constexpr int kLPK = D / 8;             // lanes per key row (16 or 8)
  constexpr int kKPP = kWave / kLPK;      // keys per wave pass
  constexpr int kKPB = kKPP * kWaves;     // keys per workgroup pass
  constexpr int kPasses = kPart / kKPB;   // passes over a full partition (8 or 4)
  using R = Row<kInt8>;
  const rlk_attention_params& p = args.p;
  const rlk_decode_attention_work& w = args.w;
  float (&red)[kWaves][G][D] = lds.red;
  float (&stat)[kWaves][G][2] = lds.stat;
  int (&cell_s)[kPart] = lds.cell;
  // The thread index passes through an empty asm (no instruction) so that the
  // lane-dependent address arithmetic below is recomputed per unit instead of
  // being hoisted out of the persistent loop and kept live across it.
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave), lane = tid % kWave;
  // partitions of this context the caller's workspace holds (a smaller
  // max_partitions than the context needs truncates, and never writes past
  // the workspace rows)
  const int num_parts = min((ctx + kPart - 1) / kPart, w.max_partitions);
  const int start = part * kPart;
  const int n = min(kPart, ctx - start);
  const int slot = lane / kLPK;         // key slot of this lane within a wave pass
  const int e0 = (lane % kLPK) * 8;     // first element of the row owned by this lane

  // Every key of the partition resolved once to its cache cell (the block-
  // table entry `blk` comes from the caller); the K/V addresses below are
  // then one LDS read each.
  if (tid < kPart && blk >= 0) {
    const int bs = p.kv.block_size;
    const int pos = start + tid;
    cell_s[tid] = (blk * p.kv.num_kv_heads + kvh) * bs + (pos - (pos / bs) * bs);
  }
  // q of the G heads, this lane's 8 elements, kept in fp16 pairs for
  // v_dot2_f32_f16 (the softmax scale is applied to the fp32 dot).
  f16x8v q[G];
  {
    const _Float16* qrow = reinterpret_cast<const _Float16*>(p.q) +
                           static_cast<int64_t>(token) * p.q_stride + (kvh * G) * D + e0;
#pragma unroll
    for (int g = 0; g < G; ++g) q[g] = __builtin_bit_cast(f16x8v, load16(qrow + g * D));
  }
  __syncthreads();

  // Key j of pass u for this lane; slots past the context re-read the last
  // valid row (a cache hit) and are masked out of the results, which keeps
  // every load unconditional.
  auto key_of = [&](int pass) { return (pass * kWaves + wave) * kKPP + slot; };
  auto cell_of = [&](int j) -> int64_t { return cell_s[min(j, n - 1)]; };

  // ---- all K and V rows of this wave (and INT8 scales) in flight at once
  typename R::Raw kr[kPasses], vr[kPasses];
  float ksc[kPasses], vsc[kPasses];
#pragma unroll
  for (int u = 0; u < kPasses; ++u) {
    const int64_t cell = cell_of(key_of(u));
    kr[u] = R::load(p.kv.k, cell, D, e0);
    vr[u] = R::load(p.kv.v, cell, D, e0);
    ksc[u] = kInt8 ? p.kv.k_scale[cell] : 1.f;
    vsc[u] = kInt8 ? p.kv.v_scale[cell] : 1.f;
  }
  // Keep the scheduler from consuming a row right after its own load (which
  // would wait for each load in turn) and from converting V rows early.
  __builtin_amdgcn_sched_barrier(0);

  // ---- scores of this wave's keys, in registers: s = scale * (q_g . k_j) * k_scale_j
  // (every lane of a key holds its score after the DPP reduction)
  float sc[kPasses][G];
#pragma unroll
  for (int u = 0; u < kPasses; ++u) {
    const f16x8v k = R::halves(kr[u]);
    const bool valid = key_of(u) < n;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float d2 = 0.f;
#pragma unroll
      for (int x = 0; x < 8; x += 2) {
        const f16x2 a = {q[g][x], q[g][x + 1]};
        const f16x2 b = {k[x], k[x + 1]};
        d2 = __builtin_amdgcn_fdot2(a, b, d2, false);
      }
      const float dot = group_sum<kLPK>(d2);
      sc[u][g] = valid ? dot * (p.scale * ksc[u]) : -FLT_MAX;
    }
  }

  // ---- softmax over this wave's keys (flash-decoding inside the workgroup):
  // the wave's own max and sum, combined across waves at the output
  float mw[G], lw[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float v = sc[0][g];
#pragma unroll
    for (int u = 1; u < kPasses; ++u) v = fmaxf(v, sc[u][g]);
    mw[g] = slots_max<kLPK>(v);
  }
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float v = 0.f;
#pragma unroll
    for (int u = 0; u < kPasses; ++u) {
      const float e = key_of(u) < n ? __expf(sc[u][g] - mw[g]) : 0.f;
      sc[u][g] = e;  // the probability (unnormalised) replaces the score
      v += e;
    }
    lw[g] = slots_sum<kLPK>(v);
  }

  // ---- P . V: o[g][e0..e0+7] += (p_gj * v_scale_j) * v_j, then the key slots folded
  f32x8 acc[G];
#pragma unroll
  for (int g = 0; g < G; ++g) acc[g] = f32x8{0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int u = 0; u < kPasses; ++u) {
    const f32x8 v = R::floats(vr[u]);
#pragma unroll
    for (int g = 0; g < G; ++g) acc[g] += (sc[u][g] * vsc[u]) * v;
  }
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int x = 0; x < 8; ++x) acc[g][x] = slots_sum<kLPK>(acc[g][x]);
  if (slot == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int x = 0; x < 8; ++x) red[wave][g][e0 + x] = acc[g][x];
  }
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      stat[wave][g][0] = mw[g];
      stat[wave][g][1] = lw[g];
    }
  }
  __syncthreads();

  // ---- combine the waves: M = max m_w, L = sum e^(m_w - M) l_w,
  // o = sum e^(m_w - M) o_w / L
  for (int i = tid; i < G * D; i += kThreads) {
    const int g = i / D, d = i % D;
    float M = stat[0][g][0];
#pragma unroll
    for (int ww = 1; ww < kWaves; ++ww) M = fmaxf(M, stat[ww][g][0]);
    float L = 0.f, o = 0.f;
#pragma unroll
    for (int ww = 0; ww < kWaves; ++ww) {
      const float f = __expf(stat[ww][g][0] - M);
      L += f * stat[ww][g][1];
      o += f * red[ww][g][d];
    }
    o /= L;
    const int h = kvh * G + g;
    if (num_parts == 1) {
      reinterpret_cast<_Float16*>(p.out)[static_cast<int64_t>(token) * p.num_heads * D + h * D + d] =
          static_cast<_Float16>(o);
    } else {
      const int64_t row = (static_cast<int64_t>(item) * p.num_heads + h) * w.max_partitions + part;
      w.ws_out[row * D + d] = o;
      if (d == 0) {
        w.ws_max[row] = M;
        w.ws_sum[row] = L;
      }
    }
  }
  __syncthreads();  // the unit's LDS may be reused
}

// Block-table entry of key `tid` of a partition (threads tid < 256), or -1
// past the table.  Table rows are padded with block 0, so every entry inside
// the row is a valid block.
__device__ __forceinline__ int table_entry(const rlk_attention_params& p, int seq, int part) {
  const int tid = threadIdx.x;
  const int bi = (part * kPart + tid) / p.kv.block_size;
  if (tid >= kPart || bi >= p.max_blocks_per_seq) return -1;
  return p.block_tables[static_cast<int64_t>(seq) * p.max_blocks_per_seq + bi];
}

// Persistent form.  Every workgroup first reads each decode item's token,
// sequence and context into LDS and prefix-sums the partitions per item; the
// work units (item, partition, kv head) -- only those inside a context -- are
// then split into contiguous ranges, one per workgroup.  Kv head runs fastest,
// so one partition's block-table entries serve all kv heads, and the chain of
// dependent loads per unit is the K/V rows alone.  (Pipelining the next
// unit's rows into the current unit's registers was measured slower: it needs
// more than the 128 VGPRs that keep two workgroups per CU.)  The unit body
// re-derives its lane-dependent addresses per unit (see attend_unit), which
// keeps the loop within those 128 VGPRs.
constexpr int kMaxItemsLds = 2048;

template <int D, int G, bool kInt8>
__global__ __launch_bounds__(kThreads, (G <= 4 ? 4 : 2)) void decode_attention_persistent(AttnArgs args) {
  const rlk_attention_params& p = args.p;
  const rlk_decode_attention_work& w = args.w;
  __shared__ UnitLds<D, G> s;
  __shared__ int it_tok[kMaxItemsLds], it_seq[kMaxItemsLds], it_ctx[kMaxItemsLds];
  __shared__ int it_pfx[kMaxItemsLds + 1];  // partitions before item i
  __shared__ int wave_tot[kWaves];
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
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
  // first unit: binary search of its partition among the items
  int pu = u0 / hkv, kvh = u0 - pu * hkv;
  int lo = 0, hi = items - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) / 2;
    if (it_pfx[mid] <= pu) lo = mid; else hi = mid - 1;
  }
  int item = lo, part = pu - it_pfx[item];
  int blk = table_entry(p, it_seq[item], part);
  for (int u = u0; u < u1; ++u) {
    attend_unit<D, G, kInt8>(args, s, item, it_tok[item], it_ctx[item], part, kvh, blk);
    if (++kvh == hkv) {
      kvh = 0;
      if (++part == it_pfx[item + 1] - it_pfx[item]) {
        part = 0;
        ++item;
      }
      if (u + 1 < u1) blk = table_entry(p, it_seq[item], part);
    }
  }
}

// Grid form: one workgroup per (partition, kv head, item), exiting at once
// when the partition lies past the item's context.
template <int D, int G, bool kInt8>
__global__ __launch_bounds__(kThreads, (G <= 4 ? 4 : 2)) void decode_attention_kernel(AttnArgs args) {
  const rlk_attention_params& p = args.p;
  const rlk_decode_attention_work& w = args.w;
  __shared__ UnitLds<D, G> s;
  const int part = blockIdx.x, kvh = blockIdx.y, item = blockIdx.z;
  const int token = w.item_token[item];
  const int blk = table_entry(p, w.item_seq[item], part);  // issued before the context is known
  const int ctx = p.positions[token] + 1;
  if (part >= (ctx + kPart - 1) / kPart) return;  // uniform over the workgroup (part < max_partitions)
  attend_unit<D, G, kInt8>(args, s, item, token, ctx, part, kvh, blk);
}

// Merges the split-K partials of one (item, head), one lane per output dim
// (the merge rule of attention.cu:193-210).  Weight of partition i:
// exp(m_i - max_j m_j) * l_i.  The partition statistics are read by all lanes
// together and the weights kept in LDS; each lane then sums its dim over the
// partitions with kUnroll partial-row loads in flight.
constexpr int kReduceMaxParts = 4096;  // weights kept in LDS (contexts up to 1M keys)

template <int D>
__global__ __launch_bounds__(D) void decode_reduce_kernel(AttnArgs args) {
  constexpr int kUnroll = 8;
  const rlk_attention_params& p = args.p;
  const rlk_decode_attention_work& w = args.w;
  __shared__ float wgt[kReduceMaxParts];
  __shared__ float part_red[D / kWave];
  const int item = blockIdx.x, h = blockIdx.y, d = threadIdx.x, lane = d % kWave, wv = d / kWave;
  const int token = w.item_token[item];
  const int ctx = p.positions[token] + 1;
  const int num_parts = min((ctx + kPart - 1) / kPart, w.max_partitions);
  if (num_parts <= 1) return;  // uniform: written directly by the attention kernel
  const int64_t base = (static_cast<int64_t>(item) * p.num_heads + h) * w.max_partitions;

  float mx = -FLT_MAX;
  for (int i = d; i < num_parts; i += D) mx = fmaxf(mx, w.ws_max[base + i]);
  mx = rows_max<true>(rows_max<false>(group_max<16>(mx)));
  if (lane == 0) part_red[wv] = mx;
  __syncthreads();
  mx = part_red[0];
#pragma unroll
  for (int i = 1; i < D / kWave; ++i) mx = fmaxf(mx, part_red[i]);
  __syncthreads();  // part_red is reused below
  float total = 0.f;
  for (int i = d; i < num_parts; i += D) {
    const float g = __expf(w.ws_max[base + i] - mx) * w.ws_sum[base + i];
    wgt[i] = g;
    total += g;
  }
  total = wave_sum(total);
  if (lane == 0) part_red[wv] = total;
  __syncthreads();
  total = part_red[0];
#pragma unroll
  for (int i = 1; i < D / kWave; ++i) total += part_red[i];

  const float* src = w.ws_out + base * D + d;
  float o = 0.f;
  int i = 0;
  for (; i + kUnroll <= num_parts; i += kUnroll) {
    float v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) v[u] = src[static_cast<int64_t>(i + u) * D];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) o += wgt[i + u] * v[u];
  }
  for (; i < num_parts; ++i) o += wgt[i] * src[static_cast<int64_t>(i) * D];
  reinterpret_cast<_Float16*>(p.out)[static_cast<int64_t>(token) * p.num_heads * D + h * D + d] =
      static_cast<_Float16>(o / total);
}

// The persistent form (two workgroups per CU) serves batches of up to
// kMaxItemsLds decode items, the grid form larger ones.  RLK_TUNE_ATTN_PERSIST
// overrides: workgroups per CU for the persistent form, or 0 for the grid form.
template <int D, int G>
void launch_g(const AttnArgs& a, bool int8, hipStream_t stream) {
  const int mode = tune_knob("RLK_TUNE_ATTN_PERSIST", 2);
  if (mode > 0 && a.w.num_items <= kMaxItemsLds) {
    const int64_t units = static_cast<int64_t>(a.w.num_items) * a.w.max_partitions * a.p.kv.num_kv_heads;
    const int blocks = static_cast<int>(std::min<int64_t>(units, static_cast<int64_t>(compute_units()) * mode));
    if (int8) {
      decode_attention_persistent<D, G, true><<<blocks, kThreads, 0, stream>>>(a);
    } else {
      decode_attention_persistent<D, G, false><<<blocks, kThreads, 0, stream>>>(a);
    }
    return;
  }
  const dim3 grid(a.w.max_partitions, a.p.kv.num_kv_heads, a.w.num_items);
  if (int8) {
    decode_attention_kernel<D, G, true><<<grid, kThreads, 0, stream>>>(a);
  } else {
    decode_attention_kernel<D, G, false><<<grid, kThreads, 0, stream>>>(a);
  }
}

template <int D>
bool launch_d(const AttnArgs& a, int G, bool int8, hipStream_t stream) {
  switch (G) {
    case 1: launch_g<D, 1>(a, int8, stream); break;
    case 2: launch_g<D, 2>(a, int8, stream); break;
    case 3: launch_g<D, 3>(a, int8, stream); break;
    case 4: launch_g<D, 4>(a, int8, stream); break;
    case 5: launch_g<D, 5>(a, int8, stream); break;
    case 6: launch_g<D, 6>(a, int8, stream); break;
    case 7: launch_g<D, 7>(a, int8, stream); break;
    case 8: launch_g<D, 8>(a, int8, stream); break;
    default: return false;
  }
  if (a.w.max_partitions > 1)
    decode_reduce_kernel<D><<<dim3(a.w.num_items, a.p.num_heads), D, 0, stream>>>(a);
  return true;
}

}  // namespace
}  // namespace rlk

using namespace rlk;

extern "C" int rlk_paged_attention_decode(const rlk_attention_params* p,
                                          const rlk_decode_attention_work* w,
                                          hipStream_t stream) {
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
  AttnArgs a;
  a.p = *p;
  a.w = *w;
  const int G = p->num_heads / hkv;
  const bool int8 = p->kv.dtype == RLK_KV_INT8;
  const bool ok = p->kv.head_dim == 128 ? launch_d<128>(a, G, int8, stream)
                                        : launch_d<64>(a, G, int8, stream);
  if (!ok) return fail(RLK_EUNSUPPORTED, "unsupported GQA group size %d", G);
  return launch_status("paged_attention_decode");
}
