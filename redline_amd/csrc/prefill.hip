// Paged prefill attention over the block-structured KV cache, for gfx950.
//
// Causal (flash-attention style) attention for sequences that process several
// new tokens against cached + new keys, with the reference's work contract
// (src/cuda/kernels/attention.cu:210-360, launcher :399-408, entry :423-431 in
// Neil456/Redline): sequence seq_ids[z] has q_len new tokens at query rows
// q_start .. q_start + q_len - 1; new token i sits at position
// past + i = ctx_len - q_len + i and attends to positions [0, past + i].
//
// The mapping is wave64 and matrix-core first:
//   * a workgroup of 4 waves takes (sequence, 64 or 128 query rows, head); a
//     wave owns 16 or 32 query rows and keeps their q in registers as MFMA B
//     operands;
//   * K and V tiles of 64 keys are staged once per workgroup in LDS (K
//     row-major, V transposed), with the next tile's loads in flight while the
//     current one is computed; INT8 codes are dequantised on the way, to
//     fp16(float(code) * scale) as the reference's tile loader does;
//   * S^T = K Q^T on v_mfma_f32_16x16x32_f16: the output gives each lane one
//     query row (its column) and 16 keys of the tile, so the online softmax
//     (max, sum, rescale) is per lane with one cross-row reduction;
//   * O^T = V^T P^T on the same instruction: the probabilities a lane holds are
//     exactly its B operand (the keys of a 32-key step taken in the order the
//     S^T output hands them over), and the output again gives each lane its
//     own query row, so the running max and sum never leave the lane.
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cstdint>
#include <type_traits>

#include "device.hpp"
#include "redline_amd/rlk.h"
#include "status.hpp"

namespace rlk {
namespace {

typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

constexpr int kBK = 64;          // keys per tile
// Workgroup shape per head dim and cache dtype (measured at the C3-C5 shapes).
// The kernel waits on its K/V tile loads, which are in flight only while the
// previous tile is computed: more query rows per loaded tile (more waves per
// workgroup, QS 16-row query sets per wave) and more waves per SIMD both hide
// more of that.  8 waves per workgroup (256 query rows FP16, 128 INT8) beat 4
// by 20% (FP16, C5) and 16% (INT8, C4).  FP16: QS = 2 at two waves per SIMD
// beat QS = 1 at four by 6-8%; INT8 (dequantised during staging, which wants
// the more waves) the other way round.  Left to itself, the compiler took
// ~200 VGPRs at QS = 1 (two waves per SIMD), 20-35% slower than four.  D = 64
// keeps 4 waves: its V tile has only 256 staging items.
template <int D, bool kInt8>
struct PfShape {
  static constexpr int kQS = kInt8 ? 1 : 2;
  static constexpr int kWavesPerSimd = kInt8 ? 4 : 2;
  static constexpr int kWaves = D == 128 ? 8 : 4;  // waves per workgroup
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kBQ = kWaves * 16 * kQS;  // query rows per workgroup
};
// K row padding: 16 halves measured half the bank conflicts of 8 (rocprofv3
// SQ_LDS_BANK_CONFLICT); the V^T padding made no difference.
constexpr int kKPad = 16;        // halves of padding per K row
constexpr int kVPad = 8;         // halves of padding per V^T row

struct PrefillArgs {
  rlk_attention_params p;
  rlk_prefill_attention_work w;
  int scale16;  // INT8 scales stored as fp16 (extension)
};

template <int D, bool kInt8>
struct PfTile {
  // per thread: K chunks (8 dims of one key) and V chunk pairs (8 dims of two keys)
  static constexpr int kKChunks = kBK * D / 8 / PfShape<D, kInt8>::kThreads;
  static constexpr int kVPairs = kKChunks / 2;
  using Raw = typename std::conditional<kInt8, u32x2, u32x4>::type;
  Raw k[kKChunks];
  float ks[kKChunks];
  Raw v[kVPairs][2];
  float vs[kVPairs][2];
};

// Column of key k (0..63) in a V^T row: within each 32-key step, keys
// 4 q + e and 16 + 4 q + e (q, e = 0..3) sit at 8 q + e and 8 q + 4 + e, the
// order in which the P . V operands take them; a pair (k, k + 1) with k even
// stays adjacent.
__device__ __forceinline__ int vt_col(int k) {
  const int r = k % 32;
  return (k - r) + 8 * ((r % 16) / 4) + 4 * (r / 16) + r % 4;
}

// Physical column of V^T[row][col]: the 16-byte chunks of a row are XOR-ed
// with (row / 8) % 8.  A staging write puts each lane's key pair (one dword)
// into the row of one of its 8 dims, rows 8 apart across the 8-dim chunks of V:
// unswizzled, every lane of an instruction fell in one bank (rocprofv3: 76% of
// the LDS-active cycles were bank conflicts).  With the XOR, and the lanes of
// each 32-lane half covering 8 dim chunks x 4 key pairs whose columns are the
// 4 dwords of one chunk (vt_item), the 32 lanes hit 32 banks.  The P . V
// operand reads take 8 consecutive rows at one chunk per 128 bytes and stay
// conflict-free and 16-byte contiguous.
__device__ __forceinline__ int vt_phys(int row, int col) {
  return (((col >> 3) ^ ((row >> 3) & 7)) << 3) | (col & 7);
}

// Key pair kp (keys 2 kp, 2 kp + 1) and 8-dim chunk ch that thread tid stages
// in V round u: lane bits 0-2 (and bit 5 when D = 128) pick the chunk, bits
// 3-4 the offset {0, 1, 8, 9} within a group of key pairs (the 4 dwords of one
// V^T chunk), the rest the group; the 16 lanes of one key pair read its
// 256-byte (D = 128) row contiguously.
template <int D, int kThreads>
__device__ __forceinline__ void vt_item(int tid, int u, int& kp, int& ch) {
  const int l = tid & 63, wv = tid >> 6;
  int bi;
  if constexpr (D == 128 && kThreads == 512) {
    ch = ((l >> 5) << 3) | (l & 7);
    bi = wv;
    (void)u;
  } else if constexpr (D == 128) {
    ch = ((l >> 5) << 3) | (l & 7);
    bi = (wv << 1) | u;
  } else {
    ch = l & 7;
    bi = ((l >> 5) << 2) | wv;
  }
  constexpr int kOff[4] = {0, 1, 8, 9};
  kp = 2 * (bi & 3) + 16 * (bi >> 2) + kOff[(l >> 3) & 3];
}

template <bool kInt8>
__device__ __forceinline__ f16x8 dequant8(typename std::conditional<kInt8, u32x2, u32x4>::type r,
                                          float s) {
  if constexpr (kInt8) {
    // fp16(float(code) * scale), as attention.cu:266-274
    const uint32_t w[2] = {r.x, r.y};
    f16x8 h;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int code = static_cast<int8_t>((w[i / 4] >> (8 * (i % 4))) & 0xFF);
      h[i] = static_cast<_Float16>(static_cast<float>(code) * s);
    }
    return h;
  } else {
    (void)s;
    return __builtin_bit_cast(f16x8, r);
  }
}

// Online-softmax state of a wave's query rows (QS sets of 16), in raw-score
// units; the scale is folded into the exponent: e^((s - m) scale) = 2^(s c - m c),
// c = scale log2(e).  Lane (qd, c16) holds output dims 16 dt + 4 qd + e of row
// c16 of each set.
template <int D, int QS>
struct PfState {
  f32x4 o[QS][D / 16];
  float m_run[QS], l_run[QS];
  float c;
  __device__ explicit PfState(float scale) : c(scale * 1.44269504088896340736f) {
#pragma unroll
    for (int qs = 0; qs < QS; ++qs) {
      m_run[qs] = -FLT_MAX;
      l_run[qs] = 0.f;
#pragma unroll
      for (int dt = 0; dt < D / 16; ++dt) o[qs][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
  __device__ void store(const rlk_attention_params& p, int q0, const int (&qi)[QS], int q_len, int h,
                        int qd) const {
#pragma unroll
    for (int qs = 0; qs < QS; ++qs) {
      const float l = rows_sum<true>(rows_sum<false>(l_run[qs]));  // the 4 lanes of the row
      if (qi[qs] >= q_len) continue;
      const float inv = l > 0.f ? 1.f / l : 0.f;
      uint16_t* out = p.out + static_cast<size_t>(q0 + qi[qs]) * p.num_heads * D + h * D + 4 * qd;
#pragma unroll
      for (int dt = 0; dt < D / 16; ++dt) {
        const f16x4 r = {static_cast<_Float16>(o[qs][dt][0] * inv), static_cast<_Float16>(o[qs][dt][1] * inv),
                         static_cast<_Float16>(o[qs][dt][2] * inv), static_cast<_Float16>(o[qs][dt][3] * inv)};
        *reinterpret_cast<f16x4*>(out + 16 * dt) = r;
      }
    }
  }
};

// Online softmax of one 64-key tile: s holds raw scores (lane (qd, c16): keys
// k0 + 16 t + 4 qd + e of query row qi[qs]), turned into the probabilities
// pb (fp16, the B operands of the O^T steps); the running max and sum are
// updated, and alpha[qs] is the factor the output of query set qs takes (the
// function returns whether any lane's differs from 1: rescale_output).  Keys past a row's position get probability 0 where masked
// (kMask 1: always, 0: never, 2: as the runtime flag says; 2 keeps one copy
// of the code for kernels short of registers).
template <int kMask, int D, int QS>
__device__ __forceinline__ bool softmax_max(PfState<D, QS>& st, f32x4 (&s)[QS][4], int qs, float& alpha,
                                            int k0, const int (&qi)[QS], int q_len, int past, int qd,
                                            bool masked) {
  const float c = st.c;
  if (kMask == 1 || (kMask == 2 && masked)) {
    // keys k0 + 16 t + 4 qd + e <= past + qi: e <= lim - 16 t
    const int lim = qi[qs] < q_len ? past + qi[qs] - k0 - 4 * qd : -1000;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (16 * t + e > lim) s[qs][t][e] = -FLT_MAX;
  }
  float mt = -FLT_MAX;
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int e = 0; e < 4; ++e) mt = fmaxf(mt, s[qs][t][e]);
  mt = rows_max<true>(rows_max<false>(mt));  // the 4 lanes of this query row
  // The reference max moves only when the tile's max exceeds it by more
  // than 2^8 in probability: below that, probabilities up to 256 are exact
  // enough in fp16 and the output and sum need no rescale.
  const float m_new = fmaxf(st.m_run[qs], mt);
  const bool grew = (m_new - st.m_run[qs]) * c > 8.f;  // first valid tile: always
  // branch-free: 2^((-FLT_MAX - m) c) flushes to 0 for the first valid tile
  const float e = __builtin_amdgcn_exp2f((st.m_run[qs] - m_new) * c);
  alpha = grew ? e : 1.f;
  if (grew) st.m_run[qs] = m_new;
  return grew;
}

template <int D, int QS>
__device__ __forceinline__ void softmax_exp(PfState<D, QS>& st, f32x4 (&s)[QS][4], f16x8 (&pb)[QS][2],
                                            int qs, float alpha) {
  const float c = st.c, mc = st.m_run[qs] * c;
  float ts = 0.f;
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      s[qs][t][e] = __builtin_amdgcn_exp2f(fmaf(s[qs][t][e], c, -mc));  // masked: 2^-huge = 0
      ts += s[qs][t][e];
    }
  // the sum stays per lane (its keys of the row); store() adds the 4 lanes
  st.l_run[qs] = st.l_run[qs] * alpha + ts;
#pragma unroll
  for (int j = 0; j < 2; ++j)
    pb[qs][j] = f16x8{static_cast<_Float16>(s[qs][2 * j][0]), static_cast<_Float16>(s[qs][2 * j][1]),
                      static_cast<_Float16>(s[qs][2 * j][2]), static_cast<_Float16>(s[qs][2 * j][3]),
                      static_cast<_Float16>(s[qs][2 * j + 1][0]), static_cast<_Float16>(s[qs][2 * j + 1][1]),
                      static_cast<_Float16>(s[qs][2 * j + 1][2]), static_cast<_Float16>(s[qs][2 * j + 1][3])};
}

template <int kMask, int D, int QS>
__device__ __forceinline__ bool softmax_core(PfState<D, QS>& st, f32x4 (&s)[QS][4], f16x8 (&pb)[QS][2],
                                             float (&alpha)[QS], int k0, const int (&qi)[QS], int q_len,
                                             int past, int qd, bool masked = true) {
  bool any_grew = false;
#pragma unroll
  for (int qs = 0; qs < QS; ++qs) {
    any_grew |= softmax_max<kMask>(st, s, qs, alpha[qs], k0, qi, q_len, past, qd, masked);
    softmax_exp(st, s, pb, qs, alpha[qs]);
  }
  return __any(any_grew);
}

template <int D, int QS>
__device__ __forceinline__ void rescale_output(PfState<D, QS>& st, const float (&alpha)[QS]) {
#pragma unroll
  for (int qs = 0; qs < QS; ++qs)
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) st.o[qs][dt] *= alpha[qs];
}

// S^T of one tile for a wave's query sets: lane (qd, c16) gets the raw scores
// of keys 16 t + 4 qd + e of its rows; each K fragment feeds every query set.
// kfrag(t, ks): the A operand of subtile t (keys 16 t .. + 15 of the tile),
// step ks (dims 32 ks .. + 31): lane (qd, c16) gets key 16 t + c16, dims
// 32 ks + 8 qd .. + 7.
template <int D, int QS, class KFrag>
__device__ __forceinline__ void score_sub(f32x4 (&s)[QS][4], const f16x8 (&qb)[QS][D / 32], KFrag kfrag,
                                          int t) {
#pragma unroll
  for (int qs = 0; qs < QS; ++qs) s[qs][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < D / 32; ++ks) {
    const f16x8 ka = kfrag(t, ks);
#pragma unroll
    for (int qs = 0; qs < QS; ++qs)
      s[qs][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qb[qs][ks], s[qs][t], 0, 0, 0);
  }
}

template <int D, int QS, class KFrag>
__device__ __forceinline__ void score_tile(f32x4 (&s)[QS][4], const f16x8 (&qb)[QS][D / 32], KFrag kfrag) {
#pragma unroll
  for (int t = 0; t < 4; ++t) score_sub<D, QS>(s, qb, kfrag, t);
}

// The softmax of one tile (scores sc) interleaved with the scores of the
// next (into sn): 2 QS sections, each 4 / (2 QS) subtiles of MFMAs beside one
// phase of the softmax (max of set 0, exponentials of set 0, then set 1); the
// scheduling barriers keep each section's registers bounded.
template <int kMask, int D, int QS, class KFrag>
__device__ __forceinline__ bool softmax_beside_scores(PfState<D, QS>& st, f32x4 (&sc)[QS][4],
                                                      f16x8 (&pb)[QS][2], float (&alpha)[QS],
                                                      f32x4 (&sn)[QS][4], const f16x8 (&qb)[QS][D / 32],
                                                      KFrag kf, int k0, const int (&qi)[QS], int q_len,
                                                      int past, int qd) {
  static_assert(QS == 1 || QS == 2, "one or two query sets");
  bool grew = false;
  // QS phases of max and exponentials, spread over the 4 subtiles
  constexpr int kSubPerPhase = 4 / (2 * QS);
#pragma unroll
  for (int ph = 0; ph < 2 * QS; ++ph) {
#pragma unroll
    for (int i = 0; i < kSubPerPhase; ++i) score_sub<D, QS>(sn, qb, kf, ph * kSubPerPhase + i);
    const int qs = ph / 2;
    if (ph % 2 == 0) grew |= softmax_max<kMask>(st, sc, qs, alpha[qs], k0, qi, q_len, past, qd, true);
    else softmax_exp(st, sc, pb, qs, alpha[qs]);
    if (ph + 1 < 2 * QS) __builtin_amdgcn_sched_barrier(0);
  }
  return __any(grew);
}

// O^T += V^T P^T over two 32-key steps; step j takes keys 32 j + 4 qd + e
// (subtile 2 j) then 32 j + 16 + 4 qd + e (subtile 2 j + 1) in both operands.
// vfrag(j, dt) (j a compile-time constant): the A operand of step j, dim tile
// dt: lane (qd, c16) gets dim 16 dt + c16 of those keys.  vready(va) runs
// after a group of fragments is requested and before the MFMAs use them (a
// wait for reads the compiler does not track).
template <int D, int QS, class VFrag, class VReady>
__device__ __forceinline__ void value_tile(PfState<D, QS>& st, const f16x8 (&pb)[QS][2], VFrag vfrag,
                                           VReady vready) {
  // fragments are requested kGroup dim tiles at a time (fewer live registers)
  constexpr int kGroup = D == 128 ? 4 : D / 16;
  auto step = [&](auto jc) {
    constexpr int j = decltype(jc)::value;
#pragma unroll
    for (int g = 0; g < D / 16; g += kGroup) {
      f16x8 va[kGroup];
#pragma unroll
      for (int i = 0; i < kGroup; ++i) va[i] = vfrag(jc, g + i);
      vready(va);
#pragma unroll
      for (int i = 0; i < kGroup; ++i)
#pragma unroll
        for (int qs = 0; qs < QS; ++qs)
          st.o[qs][g + i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va[i], pb[qs][j], st.o[qs][g + i], 0, 0, 0);
    }
  };
  step(std::integral_constant<int, 0>{});
  step(std::integral_constant<int, 1>{});
}

// One 64-key tile for a wave's query rows (score_tile, softmax_core,
// value_tile).  kSplitMask: separate code for masked and unmasked tiles.
template <int D, int QS, bool kSplitMask, class KFrag, class VFrag, class VReady>
__device__ __forceinline__ void attend_tile(PfState<D, QS>& st, int k0, const f16x8 (&qb)[QS][D / 32],
                                            const int (&qi)[QS], int q_len, int past, int row0,
                                            int wave_rows, int qd, KFrag kfrag, VFrag vfrag,
                                            VReady vready) {
  f32x4 s[QS][4];
  score_tile<D, QS>(s, qb, kfrag);
  // masks only where the tile reaches past a row's position (the diagonal,
  // the context end) or the wave has rows past q_len
  f16x8 pb[QS][2];
  float alpha[QS];
  const bool masked = k0 + kBK - 1 > past + row0 || wave_rows < 16 * QS;
  bool grew;
  if constexpr (kSplitMask) {
    if (masked) grew = softmax_core<1>(st, s, pb, alpha, k0, qi, q_len, past, qd);
    else grew = softmax_core<0>(st, s, pb, alpha, k0, qi, q_len, past, qd);
  } else {
    grew = softmax_core<2>(st, s, pb, alpha, k0, qi, q_len, past, qd, masked);
  }
  if (grew) rescale_output(st, alpha);  // only when some row's reference max moved
  value_tile<D, QS>(st, pb, vfrag, vready);
}

template <int D, bool kInt8>
__global__ __launch_bounds__((PfShape<D, kInt8>::kThreads), (PfShape<D, kInt8>::kWavesPerSimd)) void
prefill_attention_kernel(PrefillArgs a) {
  using Tile = PfTile<D, kInt8>;
  constexpr int kQS = PfShape<D, kInt8>::kQS, kBQ = PfShape<D, kInt8>::kBQ;
  constexpr int kPfThreads = PfShape<D, kInt8>::kThreads;
  constexpr int kSteps = D / 32, kChunksPerRow = D / 8;
  constexpr int kWaveRows = 16 * kQS;
  __shared__ __attribute__((aligned(16))) _Float16 k_lds[kBK][D + kKPad];
  __shared__ __attribute__((aligned(16))) _Float16 vt_lds[D][kBK + kVPad];

  const rlk_attention_params& p = a.p;
  const rlk_prefill_attention_work& w = a.w;
  const int h = blockIdx.y;
  // sequences in reverse dispatch order: in a chunked-prefill batch the later
  // chunks usually sit deeper in their sequences (more keys), so the longest
  // workgroups start first
  const int seq = w.seq_ids[gridDim.z - 1 - blockIdx.z];
  const int q_len = w.q_len[seq];
  // query tiles in reverse dispatch order: the last rows have the most keys,
  // so the longest workgroups start first and the causal tail is short
  const int qt = (q_len + kBQ - 1) / kBQ - 1 - static_cast<int>(blockIdx.x);
  if (qt < 0) return;  // workgroup-uniform
  const int q0 = w.q_start[seq], ctx = w.ctx_len[seq];
  const int past = ctx - q_len;
  const int hkv = p.kv.num_kv_heads, bs = p.kv.block_size;
  const int kvh = h / (p.num_heads / hkv);
  const int32_t* table = p.block_tables + static_cast<size_t>(seq) * p.max_blocks_per_seq;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c16 = lane & 15, qd = lane >> 4;
  const int row0 = qt * kBQ + wave * kWaveRows;  // first query row of this wave
  const int kv_end = past + min(q_len, (qt + 1) * kBQ);
  const int wave_rows = min(q_len - row0, kWaveRows);
  const int wave_kv_end = wave_rows > 0 ? past + row0 + wave_rows : 0;
  // query set qs of this lane: row row0 + 16 qs + c16 (index among the new tokens)
  int qi[kQS];
#pragma unroll
  for (int qs = 0; qs < kQS; ++qs) qi[qs] = row0 + 16 * qs + c16;

  // q of this lane's rows as B operands: lane (qd, c16) holds dims 32 ks + 8 qd .. + 8
  f16x8 qb[kQS][kSteps];
#pragma unroll
  for (int qs = 0; qs < kQS; ++qs)
#pragma unroll
    for (int ks = 0; ks < kSteps; ++ks) {
      qb[qs][ks] = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
      if (qi[qs] < q_len)
        qb[qs][ks] = __builtin_bit_cast(
            f16x8, load16(p.q + static_cast<size_t>(q0 + qi[qs]) * p.q_stride + h * D + 32 * ks + 8 * qd));
    }

  const float* kscale32 = p.kv.k_scale;
  const float* vscale32 = p.kv.v_scale;
  auto cell_of = [&](int pos) {
    return (static_cast<size_t>(table[pos / bs]) * hkv + kvh) * bs + pos % bs;
  };
  auto scale_at = [&](const float* s32, size_t cell) {
    if (a.scale16)
      return static_cast<float>(__builtin_bit_cast(_Float16, reinterpret_cast<const uint16_t*>(s32)[cell]));
    return s32[cell];
  };
  auto load_row = [&](const void* base, size_t cell, int ch) {
    if constexpr (kInt8)
      return *reinterpret_cast<const u32x2*>(static_cast<const int8_t*>(base) + cell * D + ch * 8);
    else
      return load16(static_cast<const uint16_t*>(base) + cell * D + ch * 8);
  };
  auto zero_raw = []() {
    if constexpr (kInt8) return u32x2{0u, 0u};
    else return u32x4{0u, 0u, 0u, 0u};
  };

  // keys past kv_end are zero (never attended: they lie past every row's position)
  Tile st;
  auto stage_load = [&](int k0) {
#pragma unroll
    for (int u = 0; u < Tile::kKChunks; ++u) {
      const int i = tid + kPfThreads * u, r = i / kChunksPerRow, ch = i % kChunksPerRow;
      const int pos = k0 + r;
      st.k[u] = zero_raw();
      st.ks[u] = 0.f;
      if (pos < kv_end) {
        const size_t cell = cell_of(pos);
        st.k[u] = load_row(p.kv.k, cell, ch);
        if constexpr (kInt8) st.ks[u] = scale_at(kscale32, cell);
      }
    }
#pragma unroll
    for (int u = 0; u < Tile::kVPairs; ++u) {
      int kp, ch;
      vt_item<D, kPfThreads>(tid, u, kp, ch);
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        const int pos = k0 + 2 * kp + x;
        st.v[u][x] = zero_raw();
        st.vs[u][x] = 0.f;
        if (pos < kv_end) {
          const size_t cell = cell_of(pos);
          st.v[u][x] = load_row(p.kv.v, cell, ch);
          if constexpr (kInt8) st.vs[u][x] = scale_at(vscale32, cell);
        }
      }
    }
  };
  auto stage_store = [&]() {
#pragma unroll
    for (int u = 0; u < Tile::kKChunks; ++u) {
      const int i = tid + kPfThreads * u, r = i / kChunksPerRow, ch = i % kChunksPerRow;
      *reinterpret_cast<f16x8*>(&k_lds[r][ch * 8]) = dequant8<kInt8>(st.k[u], st.ks[u]);
    }
#pragma unroll
    for (int u = 0; u < Tile::kVPairs; ++u) {
      int kp, ch;
      vt_item<D, kPfThreads>(tid, u, kp, ch);
      const f16x8 v0 = dequant8<kInt8>(st.v[u][0], st.vs[u][0]);
      const f16x8 v1 = dequant8<kInt8>(st.v[u][1], st.vs[u][1]);
#pragma unroll
      for (int d = 0; d < 8; ++d) {  // V^T[dim][key pair], keys permuted within 32
        const f16x2 pr = {v0[d], v1[d]};
        *reinterpret_cast<f16x2*>(&vt_lds[ch * 8 + d][vt_phys(ch * 8 + d, vt_col(2 * kp))]) = pr;
      }
    }
  };

  PfState<D, kQS> stt(p.scale);
  auto compute = [&](int k0) {
    attend_tile<D, kQS, false>(
        stt, k0, qb, qi, q_len, past, row0, wave_rows, qd,
        [&](int t, int ks) {
          return *reinterpret_cast<const f16x8*>(&k_lds[16 * t + c16][32 * ks + 8 * qd]);
        },
        [&](int j, int dt) {
          return *reinterpret_cast<const f16x8*>(
              &vt_lds[16 * dt + c16][vt_phys(16 * dt + c16, 32 * j + 8 * qd)]);
        },
        [](auto&) {});
  };

  const int ntiles = (kv_end + kBK - 1) / kBK;
  stage_load(0);
  for (int t = 0; t < ntiles; ++t) {
    __syncthreads();  // the previous tile is consumed
    stage_store();
    __syncthreads();
    if (t + 1 < ntiles) stage_load((t + 1) * kBK);  // in flight during this tile
    if (t * kBK < wave_kv_end) compute(t * kBK);
  }

  stt.store(p, q0, qi, q_len, h, qd);
}

// Caches read by the load-to-LDS path (no register staging, no VGPRs held by
// loads in flight): four raw LDS stages, tiles t + 2 and t + 3 in flight while
// t and t + 1 are used.  Each wave instruction writes 1 KiB of LDS
// contiguously, 16 bytes per lane.
//   FP16: the raw stage is the MFMA operand image.  Its layouts are swizzled
//     on the source side: LDS chunk c (16 bytes) of key row r holds K chunk
//     c ^ kswz(r) and V chunk c ^ vswz(r).  The swizzles make every LDS read
//     conflict-free with 64 banks of 4 bytes: a 16-byte K read covers 16 key
//     rows at 16 distinct 16-byte slots of 256 bytes, and a transposing V
//     read (ds_read_tr16_b64, 8 bytes a lane) covers 8 key rows at 8 distinct
//     32-byte slots.
//   INT8: the raw stage holds the codes row-major and the 64 K and 64 V
//     scales (one dword per key, loaded by 4-byte load-to-LDS; fp16 scales
//     take the dword that holds them).  The workgroup dequantises tile t + 1
//     into one of two fp16 images of the FP16 layout, fp16(float(code) *
//     scale) as attention.cu:266-274, before the scores of t + 1 need it.
// The block table of the sequence is copied to LDS first so that the loop
// issues no other global load (whose wait would also drain the tiles in
// flight).
constexpr int kDmaStages = 4;
constexpr int kDmaTableCap = 4096;  // block-table entries staged in LDS

#define RLK_LDS __attribute__((address_space(3)))

// QS query sets of 16 rows per wave: 2 normally; 1 at D = 128 for grids too
// small to give every CU two workgroups (half the rows per workgroup).
template <int D, bool kInt8, int QS = 2>
struct PfDma {
  static constexpr int kQS = QS;
  static constexpr int kThreads = PfShape<D, false>::kThreads;
  static constexpr int kWaves = kThreads / 64;
  static constexpr int kBQ = kWaves * 16 * QS;
  static constexpr int kRowBytes = 2 * D;             // fp16 image
  static constexpr int kTileBytes = kBK * kRowBytes;  // one fp16 K or V tile
  static constexpr int kRawRow = kInt8 ? D : 2 * D;   // cache row
  static constexpr int kRawTile = kBK * kRawRow;
  static constexpr int kScaleOff = 2 * kRawTile;      // INT8: K scales, then V scales
  static constexpr int kStageBytes = 2 * kRawTile + (kInt8 ? 2 * 4 * kBK : 0);
  static constexpr int kImageOff = kDmaStages * kStageBytes;  // INT8: two fp16 images
  static constexpr int kImages = kInt8 ? 2 : 0;
  static constexpr int kTableOff = kImageOff + kImages * 2 * kTileBytes;
  static constexpr int kPieces = kRawTile / 1024 / kWaves;  // 1 KiB pieces per wave per tile (K or V)
  static_assert(kRawTile % (1024 * kWaves) == 0, "whole instructions per wave");
  static_assert(kPieces == 1 || kWaves * 1024 == 32 * kRawRow, "32 rows per round of pieces");
  // instructions a wave issues per tile (INT8: waves 0 and 1 also load the scales)
  static constexpr int kOps = 2 * kPieces;
  static constexpr int kOpsScales = kOps + (kInt8 ? 1 : 0);
  // row pitch 256 bytes (D = 128): 16 slots a row; 128 bytes (D = 64): a
  // 256-byte span holds rows r and r ^ 1
  __device__ static int kswz(int r) { return D == 128 ? r & 15 : (r >> 1) & 7; }
  __device__ static int vswz(int r) { return D == 128 ? (r & 7) << 1 : ((r >> 1) & 3) << 1; }
  static size_t lds_bytes(int table_entries) {
    return static_cast<size_t>(kTableOff) + 4 * ((table_entries + 3) & ~3);
  }
};

// s_waitcnt vmcnt(N): the compiler's own waits do not follow this kernel's
// ring (it puts none before the 16-byte LDS reads and drains every load in
// flight before the transposing reads), so the loop waits explicitly for the
// tile it needs and reads the transposed V through inline asm
template <int N>
__device__ __forceinline__ void wait_vmem() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

template <int D, bool kInt8, int QS>
__global__ __launch_bounds__((PfShape<D, false>::kThreads), (PfShape<D, false>::kWavesPerSimd)) void
prefill_dma_kernel(PrefillArgs a) {
  using G = PfDma<D, kInt8, QS>;
  constexpr int kQS = G::kQS, kBQ = G::kBQ;
  constexpr int kSteps = D / 32, kWaveRows = 16 * kQS;
  extern __shared__ __attribute__((aligned(1024))) unsigned char pf_lds[];
  int32_t* tab_lds = reinterpret_cast<int32_t*>(pf_lds + G::kTableOff);

  const rlk_attention_params& p = a.p;
  const rlk_prefill_attention_work& w = a.w;
  const int h = blockIdx.y;
  // sequences in reverse dispatch order: in a chunked-prefill batch the later
  // chunks usually sit deeper in their sequences (more keys), so the longest
  // workgroups start first
  const int seq = w.seq_ids[gridDim.z - 1 - blockIdx.z];
  const int q_len = w.q_len[seq];
  const int qt = (q_len + kBQ - 1) / kBQ - 1 - static_cast<int>(blockIdx.x);
  if (qt < 0) return;  // workgroup-uniform
  const int q0 = w.q_start[seq], ctx = w.ctx_len[seq];
  const int past = ctx - q_len;
  const int hkv = p.kv.num_kv_heads, bs = p.kv.block_size;
  const int kvh = h / (p.num_heads / hkv);
  const int32_t* table = p.block_tables + static_cast<size_t>(seq) * p.max_blocks_per_seq;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c16 = lane & 15, qd = lane >> 4;
  const int row0 = qt * kBQ + wave * kWaveRows;
  const int kv_end = past + min(q_len, (qt + 1) * kBQ);
  const int wave_rows = min(q_len - row0, kWaveRows);
  const int wave_kv_end = wave_rows > 0 ? past + row0 + wave_rows : 0;
  int qi[kQS];
#pragma unroll
  for (int qs = 0; qs < kQS; ++qs) qi[qs] = row0 + 16 * qs + c16;

  f16x8 qb[kQS][kSteps];
#pragma unroll
  for (int qs = 0; qs < kQS; ++qs)
#pragma unroll
    for (int ks = 0; ks < kSteps; ++ks) {
      qb[qs][ks] = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
      if (qi[qs] < q_len)
        qb[qs][ks] = __builtin_bit_cast(
            f16x8, load16(p.q + static_cast<size_t>(q0 + qi[qs]) * p.q_stride + h * D + 32 * ks + 8 * qd));
    }
  const int nblk = min((kv_end + bs - 1) / bs, kDmaTableCap);
  for (int i = tid; i < nblk; i += G::kThreads) tab_lds[i] = table[i];
  // q is consumed here so that no wait for it lands inside the tile loop
#pragma unroll
  for (int qs = 0; qs < kQS; ++qs)
#pragma unroll
    for (int ks = 0; ks < kSteps; ++ks) asm volatile("" : "+v"(qb[qs][ks]));
  __syncthreads();

  // Piece u of a tile for this lane: key row r0 + 32 u (each wave
  // instruction covers 1 KiB, the waves together 32 rows) and 16-byte chunk
  // c of the LDS image; the swizzles of r0 + 32 u equal those of r0.
  const int r0 = (wave * 1024 + lane * 16) / G::kRawRow;
  const int cx = ((wave * 1024 + lane * 16) % G::kRawRow) / 16;
  const int kx0 = (kInt8 ? cx : cx ^ G::kswz(r0)) << 4, vx0 = (kInt8 ? cx : cx ^ G::vswz(r0)) << 4;
  const unsigned char* kbase = static_cast<const unsigned char*>(p.kv.k);
  const unsigned char* vbase = static_cast<const unsigned char*>(p.kv.v);
  auto dma = [&](unsigned char* sb, int u, bool isv, const unsigned char* src) {
    __builtin_amdgcn_global_load_lds(
        src, (RLK_LDS void*)(sb + (isv ? G::kRawTile : 0) + (wave + G::kWaves * u) * 1024), 16, 0, 0);
  };
  // Block sizes that are powers of two: a whole tile inside the context takes
  // the block of each piece from its row (row >> log2 bs) plus the tile's
  // first block, and the byte offset inside the block from the row plus the
  // tile's offset into its block (non-zero for bs > 64).
  const bool pow2 = (bs & (bs - 1)) == 0;
  const int lbs = __builtin_ctz(bs);
  const uint32_t block_bytes = static_cast<uint32_t>(hkv) * bs * G::kRawRow;
  const uint32_t head_bytes = static_cast<uint32_t>(kvh) * bs * G::kRawRow;
  // keys past kv_end read the last key again: finite, and masked out of every row
  auto issue = [&](int tile, int stage) {
    const int k0 = tile * kBK;
    unsigned char* sb = pf_lds + stage * G::kStageBytes;
    if constexpr (kInt8) {
      // waves 0 and 1: the K and V scales of the tile's 64 keys, one per lane
      if (wave < 2) {
        const int pos = min(k0 + lane, kv_end - 1);
        const int blk = pos / bs, off = pos - blk * bs;
        const size_t cell = (static_cast<size_t>(tab_lds[blk]) * hkv + kvh) * bs + off;
        const unsigned char* sbase = reinterpret_cast<const unsigned char*>(wave == 0 ? p.kv.k_scale : p.kv.v_scale);
        const unsigned char* src = a.scale16 ? sbase + ((cell * 2) & ~size_t{3}) : sbase + cell * 4;
        __builtin_amdgcn_global_load_lds(src, (RLK_LDS void*)(sb + G::kScaleOff + wave * 4 * kBK), 4, 0, 0);
      }
    }
    // the lane constants pass through an empty asm so that the compiler
    // derives the addresses per tile instead of keeping them all live
    int r = r0, kx = kx0, vx = vx0;
    asm volatile("" : "+v"(r), "+v"(kx), "+v"(vx));
    if (pow2 && k0 + kBK <= kv_end) {
      const int blk0 = k0 >> lbs;
      const uint32_t koff = head_bytes + static_cast<uint32_t>(k0 & (bs - 1)) * G::kRawRow;
#pragma unroll
      for (int u = 0; u < G::kPieces; ++u) {
        const int ru = r + 32 * u;
        const uint64_t bb = static_cast<uint64_t>(static_cast<uint32_t>(tab_lds[blk0 + (ru >> lbs)])) * block_bytes;
        const uint32_t row_off = koff + static_cast<uint32_t>(ru & (bs - 1)) * G::kRawRow;
        dma(sb, u, false, kbase + bb + (row_off + kx));
        dma(sb, u, true, vbase + bb + (row_off + vx));
      }
      return;
    }
#pragma unroll
    for (int u = 0; u < G::kPieces; ++u) {
      const int pos = min(k0 + r + 32 * u, kv_end - 1);
      const int blk = pos / bs, off = pos - blk * bs;
      const size_t cell = (static_cast<size_t>(tab_lds[blk]) * hkv + kvh) * bs + off;
      dma(sb, u, false, kbase + cell * G::kRawRow + kx);
      dma(sb, u, true, vbase + cell * G::kRawRow + vx);
    }
  };
  // wait until the tile issued `later` tiles before the newest has landed
  auto wait_tiles = [&](int later) {
    if (later >= 2) {
      if (kInt8 && wave < 2) wait_vmem<2 * G::kOpsScales>();
      else wait_vmem<2 * G::kOps>();
    } else if (later == 1) {
      if (kInt8 && wave < 2) wait_vmem<G::kOpsScales>();
      else wait_vmem<G::kOps>();
    } else {
      wait_vmem<0>();
    }
  };
  // the fp16 operand image of tile t: the raw stage (FP16) or one of two
  // dequantised images (INT8)
  auto image = [&](int t) -> unsigned char* {
    if constexpr (kInt8) return pf_lds + G::kImageOff + (t & 1) * 2 * G::kTileBytes;
    else return pf_lds + (t % kDmaStages) * G::kStageBytes;
  };
  // INT8: dequantise raw stage t into image(t); each thread takes 16-byte
  // chunks of 8 codes, fp16 writes in the FP16 layout (swizzled)
  auto dequant = [&](int t) {
    if constexpr (kInt8) {
      const unsigned char* sb = pf_lds + (t % kDmaStages) * G::kStageBytes;
      unsigned char* img = image(t);
      const float* sc = reinterpret_cast<const float*>(sb + G::kScaleOff);
      constexpr int kChunks = kBK * D / 8;  // of K, and of V
      static_assert(kChunks % G::kThreads == 0, "whole chunks per thread");
      int me = tid;  // through an empty asm: addresses derived per tile, not kept live
      asm volatile("" : "+v"(me));
#pragma unroll
      for (int u = 0; u < 2 * kChunks / G::kThreads; ++u) {
        const bool isv = u >= kChunks / G::kThreads;
        const int j = me + G::kThreads * u - (isv ? kChunks : 0);
        const int r = j / (D / 8), c = j % (D / 8);
        const u32x2 codes = *reinterpret_cast<const u32x2*>(sb + (isv ? G::kRawTile : 0) + r * D + c * 8);
        float s = sc[(isv ? kBK : 0) + r];
        if (a.scale16) {
          // the dword holds the cells 2i and 2i + 1; the key's cell parity is
          // its position's (even block size)
          const uint32_t bits = __builtin_bit_cast(uint32_t, s);
          const int pos = min(t * kBK + r, kv_end - 1);
          s = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits >> (16 * (pos & 1)))));
        }
        const int sw = isv ? G::vswz(r) : G::kswz(r);
        *reinterpret_cast<f16x8*>(img + (isv ? G::kTileBytes : 0) + r * G::kRowBytes + ((c ^ sw) << 4)) =
            dequant8<true>(codes, s);
      }
    }
  };

  PfState<D, kQS> stt(p.scale);
  // transposing V reads: lane (qd, c16) reads key row 4 qd + tk (+ 32 j, + 16)
  // at dims 16 dt + 4 tm; byte offsets inside a V tile, for j = 0
  const int tk = c16 >> 2, tm = c16 & 3;
  // D = 128: dim tile dt + 4 sits at chunk pair (dt ^ sw) ^ 4, byte offset
  // ^ 128 of dt's (row offsets are multiples of 256), so 4 offsets are kept
  constexpr int kVrd = D == 128 ? 4 : D / 16;
  uint32_t vrd[kVrd];
#pragma unroll
  for (int dt = 0; dt < kVrd; ++dt) {
    const int row = 4 * qd + tk;  // row + 32 j and row + 16 share its swizzle
    vrd[dt] = row * G::kRowBytes + ((((2 * dt + (tm >> 1)) ^ G::vswz(row)) << 4) | ((tm & 1) << 3));
  }
  auto kfrag = [&](int t) {
    const unsigned char* kt = image(t);
    return [kt, c16, qd](int t, int ks) {
      const int row = 16 * t + c16;
      return *reinterpret_cast<const f16x8*>(kt + row * G::kRowBytes + (((4 * ks + qd) ^ G::kswz(c16)) << 4));
    };
  };
  auto vfrag = [&](int t) {
    const uint32_t vt_addr = static_cast<uint32_t>(
        reinterpret_cast<uintptr_t>((RLK_LDS const unsigned char*)(image(t) + G::kTileBytes)));
    // the offsets pass through an empty asm so that the compiler adds them
    // to this tile's base here instead of keeping every sum live
    uint32_t vo[kVrd];
#pragma unroll
    for (int i = 0; i < kVrd; ++i) {
      vo[i] = vrd[i];
      asm volatile("" : "+v"(vo[i]));
    }
    return [vt_addr, vo](auto jc, int dt) {
      // the transposing reads are issued as inline asm: the compiler's own
      // form of them waits for every load-to-LDS in flight
      constexpr int kOff = 32 * decltype(jc)::value * G::kRowBytes;
      const uint32_t addr = vt_addr + (dt < kVrd ? vo[dt] : vo[dt - kVrd] ^ 128u);
      u32x2 lo, hi;
      asm volatile("ds_read_b64_tr_b16 %0, %2 offset:%3\n\tds_read_b64_tr_b16 %1, %2 offset:%4"
                   : "=v"(lo), "=v"(hi)
                   : "v"(addr), "n"(kOff), "n"(kOff + 16 * G::kRowBytes));
      return __builtin_bit_cast(f16x8, u32x4{lo[0], lo[1], hi[0], hi[1]});
    };
  };
  auto vready = [](f16x8(&va)[4]) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(va[0]), "+v"(va[1]), "+v"(va[2]), "+v"(va[3]));
  };
  // the image's LDS writes are complete (a bare barrier does not wait)
  auto lds_written = []() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); };
  // a bare barrier: __syncthreads() would also drain the tiles in flight
  auto barrier = []() {
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };

  // Software pipeline over the tiles: the scores of tile t + 1 (MFMA) are
  // computed in the same straight-line code as the softmax of tile t (VALU),
  // so the matrix cores and the vector ALU of a wave overlap.
  const int ntiles = (kv_end + kBK - 1) / kBK;
  const int wtiles = (wave_kv_end + kBK - 1) / kBK;  // tiles this wave attends
  issue(0, 0);
  if (ntiles > 1) issue(1, 1);
  if (ntiles > 2) issue(2, 2);
  wait_tiles(min(ntiles, 3) - 1);
  barrier();
  if constexpr (kInt8) {
    dequant(0);
    lds_written();
    barrier();
  }
  f32x4 s_even[kQS][4], s_odd[kQS][4];
  if (wtiles > 0) score_tile<D, kQS>(s_even, qb, kfrag(0));

  auto body = [&](int t, f32x4(&sc)[kQS][4], f32x4(&sn)[kQS][4]) {
    // raw tile t + 1 in LDS for every wave; tile t - 1 consumed (its raw
    // stage takes tile t + 3, INT8: its image takes tile t + 1)
    wait_tiles(t + 2 < ntiles ? 1 : 0);
    barrier();
    if (t + 3 < ntiles) issue(t + 3, (t + 3) % kDmaStages);
    if constexpr (kInt8) {
      if (t + 1 < ntiles) dequant(t + 1);
      lds_written();
      barrier();
    }
    if (t >= wtiles) return;
    const int k0 = t * kBK;
    const bool masked = k0 + kBK - 1 > past + row0 || wave_rows < kWaveRows;
    f16x8 pb[kQS][2];
    float alpha[kQS];
    bool grew;
    if (t + 1 < wtiles) {
      const auto kf = kfrag(t + 1);
      grew = masked ? softmax_beside_scores<1>(stt, sc, pb, alpha, sn, qb, kf, k0, qi, q_len, past, qd)
                    : softmax_beside_scores<0>(stt, sc, pb, alpha, sn, qb, kf, k0, qi, q_len, past, qd);
    } else {
      grew = masked ? softmax_core<1>(stt, sc, pb, alpha, k0, qi, q_len, past, qd)
                    : softmax_core<0>(stt, sc, pb, alpha, k0, qi, q_len, past, qd);
    }
    if (grew) rescale_output(stt, alpha);
    value_tile<D, kQS>(stt, pb, vfrag(t), vready);
  };
  int t = 0;
  for (; t + 1 < ntiles; t += 2) {
    body(t, s_even, s_odd);
    body(t + 1, s_odd, s_even);
  }
  if (t < ntiles) body(t, s_even, s_odd);

  stt.store(p, q0, qi, q_len, h, qd);
}

// compute units of the current device (cached per device)
int device_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev] = n;
  }
  return cus[dev];
}

int prefill(const rlk_attention_params* params, const rlk_prefill_attention_work* work,
            int scale16, hipStream_t stream) {
  const char* what = "paged_attention_prefill";
  if (params == nullptr || work == nullptr) return fail(RLK_EINVAL, "%s: null argument", what);
  const rlk_attention_params& p = *params;
  const rlk_prefill_attention_work& w = *work;
  if (w.num_seqs <= 0 || w.max_q_tiles <= 0) return RLK_OK;
  if (p.kv.num_kv_heads <= 0 || p.num_heads <= 0 || p.num_heads % p.kv.num_kv_heads != 0)
    return fail(RLK_EINVAL, "%s: num_heads must be a multiple of num_kv_heads", what);
  if (p.kv.head_dim != 64 && p.kv.head_dim != 128)
    return fail(RLK_EUNSUPPORTED, "%s: unsupported head_dim %d", what, p.kv.head_dim);
  if (p.kv.block_size <= 0) return fail(RLK_EINVAL, "%s: bad block_size %d", what, p.kv.block_size);
  if (p.kv.dtype != RLK_KV_FP16 && p.kv.dtype != RLK_KV_INT8)
    return fail(RLK_EINVAL, "%s: unknown KV dtype %d", what, p.kv.dtype);
  if (w.num_seqs > 65535 || p.num_heads > 65535)
    return fail(RLK_EINVAL, "%s: %d sequences x %d heads exceed one launch grid; split the call",
                what, w.num_seqs, p.num_heads);
  const bool int8 = p.kv.dtype == RLK_KV_INT8;
  if (p.q == nullptr || p.out == nullptr || p.kv.k == nullptr || p.kv.v == nullptr ||
      p.block_tables == nullptr || w.seq_ids == nullptr || w.q_start == nullptr ||
      w.q_len == nullptr || w.ctx_len == nullptr ||
      (int8 && (p.kv.k_scale == nullptr || p.kv.v_scale == nullptr)))
    return fail(RLK_EINVAL, "%s: null pointer argument", what);
  if (reinterpret_cast<uintptr_t>(p.q) % 16 != 0 || p.q_stride % 8 != 0)
    return fail(RLK_EINVAL, "%s: q rows must be 16-byte aligned (q_stride %d)", what, p.q_stride);
  PrefillArgs a{p, w, scale16};
  // the work's tiles are the reference's 32-row tiles (kPrefillTileQ); ours hold kBQ rows
  const int rows = w.max_q_tiles * RLK_PREFILL_TILE_Q;
  auto go = [&](auto kernel, auto shape) {
    using S = decltype(shape);
    const dim3 grid((rows + S::kBQ - 1) / S::kBQ, p.num_heads, w.num_seqs);
    kernel<<<grid, S::kThreads, 0, stream>>>(a);
  };
  // The load-to-LDS kernel runs when the block table fits its LDS copy;
  // RLK_TUNE_PREFILL_DMA=0 forces the register-staged kernel
  // (the kernel keeps byte offsets inside a cache block in 32 bits)
  const bool dma_fits = p.max_blocks_per_seq <= kDmaTableCap &&
                        static_cast<uint64_t>(p.kv.num_kv_heads) * p.kv.block_size * p.kv.head_dim * 2 <
                            (uint64_t{1} << 32);
  // (INT8 with fp16 scales reads the dword that holds a scale and picks the
  // half by the key position's parity: even block sizes only)
  const bool dma_ok = dma_fits && (!int8 || !scale16 || p.kv.block_size % 2 == 0);
  if (dma_ok && tune_knob(kPrefillDma, 1) != 0) {
    auto dma = [&](auto kernel, auto geo) -> int {
      using G = decltype(geo);
      const size_t lds = G::lds_bytes(p.max_blocks_per_seq);
      const size_t want = G::lds_bytes(kDmaTableCap);
      const hipError_t e = grant_dynamic_lds(reinterpret_cast<const void*>(kernel), want);
      if (e != hipSuccess)
        return fail(RLK_EUNSUPPORTED, "%s: %zu bytes of LDS refused (%s)", what, want,
                    hipGetErrorString(e));
      const dim3 grid((rows + G::kBQ - 1) / G::kBQ, p.num_heads, w.num_seqs);
      kernel<<<grid, G::kThreads, lds, stream>>>(a);
      return launch_status(what);
    };
    if (p.kv.head_dim == 64)
      return int8 ? dma(prefill_dma_kernel<64, true, 2>, PfDma<64, true, 2>{})
                  : dma(prefill_dma_kernel<64, false, 2>, PfDma<64, false, 2>{});
    // D = 128: 16 query rows per wave when 32 would not give every CU two
    // workgroups (RLK_TUNE_PREFILL_QS=1 or 2 forces one form)
    const int grid2 = (rows + PfDma<128, false, 2>::kBQ - 1) / PfDma<128, false, 2>::kBQ * p.num_heads *
                      w.num_seqs;
    if (tune_knob(kPrefillQs, grid2 < 2 * device_cus() ? 1 : 2) == 1)
      return int8 ? dma(prefill_dma_kernel<128, true, 1>, PfDma<128, true, 1>{})
                  : dma(prefill_dma_kernel<128, false, 1>, PfDma<128, false, 1>{});
    return int8 ? dma(prefill_dma_kernel<128, true, 2>, PfDma<128, true, 2>{})
                : dma(prefill_dma_kernel<128, false, 2>, PfDma<128, false, 2>{});
  }
  if (p.kv.head_dim == 64) {
    if (int8) go(prefill_attention_kernel<64, true>, PfShape<64, true>{});
    else go(prefill_attention_kernel<64, false>, PfShape<64, false>{});
  } else {
    if (int8) go(prefill_attention_kernel<128, true>, PfShape<128, true>{});
    else go(prefill_attention_kernel<128, false>, PfShape<128, false>{});
  }
  return launch_status(what);
}

}  // namespace
}  // namespace rlk

using namespace rlk;

extern "C" int rlk_paged_attention_prefill(const rlk_attention_params* params,
                                           const rlk_prefill_attention_work* work,
                                           hipStream_t stream) {
  return prefill(params, work, 0, stream);
}

extern "C" int rlk_paged_attention_prefill_ex(const rlk_attention_params* params,
                                              const rlk_prefill_attention_work* work,
                                              const rlk_attention_options* options,
                                              hipStream_t stream) {
  const int scale_dtype = options != nullptr ? options->scale_dtype : RLK_SCALE_F32;
  if (scale_dtype != RLK_SCALE_F32 && scale_dtype != RLK_SCALE_F16)
    return fail(RLK_EINVAL, "paged_attention_prefill_ex: unknown scale dtype %d", scale_dtype);
  return prefill(params, work, scale_dtype == RLK_SCALE_F16, stream);
}
