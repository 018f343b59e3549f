// Weight-only INT4 GEMV for decode on gfx950 matrix cores, with an optional
// SwiGLU epilogue over interleaved (gate_i, up_i) weight rows.
//
// Reference behaviour: gemv_weight_only.cu:103-160 (y = s * sum(x q) + o *
// sum(x) per 32-aligned group of K), :46-63 (SwiGLU rounding points), launchers
// :222-241.
//
// Design.  At decode batch m <= 32 every weight byte is used 2m times, so a
// vector-ALU GEMV with fp32 FMAs is compute-bound on this chip from m ~ 4 on.
// The dot products run on MFMA (v_mfma_f32_16x16x32_f16) instead, with the
// activations as the A operand (16 rows of x) and the weights as B (16 weight
// rows, one per lane column):
//   * each lane holds 8 codes of its weight row per step (4 bytes), turned
//     into exact fp16 values 64 + q by OR-ing each nibble into the mantissa of
//     64.0 -- one VALU op per two codes plus shifts, no converts;
//   * once per scale window (a K range inside one quantisation group) the fp32
//     partial is folded in as acc += s * (x . (64 + q)) + (o - 64 s) * sum(x)
//     -- the reference's s * sum(x q) + o * sum(x) -- so the codes are never
//     rounded through a dequantised fp16 weight.  The output layout gives each
//     lane one weight row, so s and o are per-lane scalars.
// K order inside an MFMA is free as long as A and B agree: a lane takes 32
// consecutive K (16 code bytes, one 16-byte load per row and chunk) and the
// activations are permuted to the nibble order (0, 4, 1, 5, 2, 6, 3, 7) that
// the code unpacking produces.
//
// Kernels (the launch policy picks by m and shape; the kernels' own comments
// give the details):
//   * the pair kernel (m < 8): a workgroup stages x once in LDS, already
//     permuted, with sum(x) per chunk and row taken during the staging, and
//     each wave walks one 16-row tile over the full K with a ring of chunk
//     pairs in flight, loaded as full 128-byte lines (8 rows per load
//     instruction) and handed to the owning lanes by a DPP row rotation.
//     Activations are the expensive operand to fetch -- the load path pays
//     per cache line an instruction touches -- so x is staged once per CU;
//   * the K-slice kernel (m >= 8): wave w owns K slice w of every tile of its
//     workgroup, so it needs only its slice of x, in registers; codes take
//     two magics (codes_f16_2m) and the offset terms enter per tile as fp32
//     MFMAs; partials meet in LDS in a fixed order;
//   * the slab kernel for the remaining shapes (odd chunk counts, group sizes
//     whose /128 is not a power of two, 32-K chunks).
// The pair and slab kernels walk K in x passes when x does not fit the LDS
// budget (x re-staged per pass, accumulators kept).
// The INT8 weight-only GEMV (gemv_w8a16) runs the K-slice decomposition too
// (gemv_w8_kslice_kernel), or the pair kernel's INT8 form.
#include <algorithm>
#include <type_traits>
#include <utility>

#include "device.hpp"
#include "redline_amd/rlk.h"
#include "status.hpp"

namespace rlk {
namespace {

struct W4Args {
  const uint16_t* x;  // activations of this launch, [m, k]
  const uint8_t* w;
  const uint16_t* scales;
  const uint16_t* offsets;
  const uint16_t* bias;
  void* y;            // [m, y_ld]
  int m;              // activation rows (1 .. 16 MT)
  int n, k, group_size, groups, nchunks;
  int cpp;            // K chunks per x pass (a multiple of K-split ways x ring depth);
                      // K-slice kernel: 16-row tiles per workgroup
  int npass;
  int xstride;        // halves per staged x row
  int slab_off;       // bytes from the end of x to the first chunk-pair slab;
                      // K-slice kernel: bytes from the LDS base to the partial sums
  int y_ld;
  int gq_shift;       // pair kernel: log2(group_size / 128)
  int gpp;            // pair kernel: quantisation groups per x pass
};

constexpr int kModeF16 = 0, kModeF32 = 1, kModeSwiglu = 2;
constexpr int kSlabRow = 144;                // bytes per slab row: 128 code bytes + 16 pad
constexpr int kSlabBytes = 16 * kSlabRow;    // one wave's chunk-pair slab

// Codes of one lane for one chunk: 32 K (16 bytes) for 128-K chunks, 8 K
// (4 bytes) for 32-K chunks.  Weights are read exactly once: non-temporal.
template <int KC>
__device__ __forceinline__ u32x4 load_codes(const uint8_t* p) {
  if constexpr (KC == 128) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  } else {
    u32x4 v = {__builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p)), 0u, 0u, 0u};
    return v;
  }
}

// A value the compiler must keep in a VGPR without knowing it (the empty asm
// emits no instruction).  With the code magic opaque, (x & mask) | magic is
// selected as one v_and_or_b32 (mask in an SGPR); with both operands known
// constants the compiler splits it into AND + OR, because gfx9 VOP3
// encodings take no literal.  Writing the op itself as inline asm would hide
// it from the compiler's hazard recognizer, which must pad a VALU write of an
// MFMA source operand.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}

__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t mask, uint32_t magic) {
  return (x & mask) | magic;
}

// The 8 codes of a word (nibble e = code of K offset e) as fp16 values
// 64 + q, in the order (q0, q4, q1, q5, q2, q6, q3, q7): a nibble placed in
// mantissa bits 4..7 of 64.0 (0x5400) reads 64 + q exactly.  The bias of 64
// is removed through the offset term (o - 64 s), computed once per group in
// fp32; it keeps the MFMA sums within a small factor of the unbiased ones.
__device__ __forceinline__ f16x8 codes_f16(uint32_t word, uint32_t magic) {
  constexpr uint32_t kMask = 0x00F000F0u;
  const u32x4 r = {and_or(word << 4, kMask, magic), and_or(word, kMask, magic),
                   and_or(word >> 4, kMask, magic), and_or(word >> 8, kMask, magic)};
  return __builtin_bit_cast(f16x8, r);
}
constexpr float kCodeBias = 64.0f;

// The K-slice kernel's form: 5 VALU per 8 codes instead of 7.  Nibbles in
// mantissa bits 0..3 of 1024.0 read 1024 + q, in bits 4..7 of 64.0 read
// 64 + q, so the word needs one shift: (q0, q4) and (q2, q6) take magic
// m1024, (q1, q5) and (q3, q7) m64 -- the same element order as codes_f16.
// The biases leave through sum(x * kBias2) per chunk.  The larger bias costs
// fp32 sum bits (the kernel's relative error grows from ~1.5e-6 to ~2e-5 at
// k = 4096; the fp32-output bound is 1e-4).
__device__ __forceinline__ f16x8 codes_f16_2m(uint32_t word, uint32_t m1024, uint32_t m64) {
  const uint32_t w8 = word >> 8;
  const u32x4 r = {and_or(word, 0x000F000Fu, m1024), and_or(word, 0x00F000F0u, m64),
                   and_or(w8, 0x000F000Fu, m1024), and_or(w8, 0x00F000F0u, m64)};
  return __builtin_bit_cast(f16x8, r);
}
// The bias of each element of codes_f16_2m's output.
constexpr f16x8 kBias2 = {1024, 1024, 64, 64, 1024, 1024, 64, 64};

// 8 consecutive activations permuted to the codes' order.
__device__ __forceinline__ f16x8 x_perm(u32x4 v) {
  const f16x8 h = __builtin_bit_cast(f16x8, v);
  return __builtin_shufflevector(h, h, 0, 4, 1, 5, 2, 6, 3, 7);
}

// v / d for 0 <= v < 2^21 through a float reciprocal: (v + 1/2) / d lies at
// least 1/(2d) away from an integer and the float error is below 2^-22 * v/d.
__device__ __forceinline__ int quot(int v, float inv_d) {
  return static_cast<int>((static_cast<float>(v) + 0.5f) * inv_d);
}

__device__ __forceinline__ float swap_adjacent_lanes(float v) {
  // quad_perm (1, 0, 3, 2): each lane reads its odd/even neighbour
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF,
                                                            0xF, false));
}

// Output of one 16x16 tile: lane (qd, r16) holds rows m = m0 + 4 qd + e of
// weight row `row`.
template <int MODE>
__device__ __forceinline__ void store_tile(const W4Args& a, f32x4 v, int m0, int row, int r16) {
  if constexpr (MODE == kModeSwiglu) {
    // (gate, up) = rows (2i, 2i + 1) sit in lanes (r16, r16 + 1)
    f32x4 up;
#pragma unroll
    for (int e = 0; e < 4; ++e) up[e] = swap_adjacent_lanes(v[e]);
    if ((r16 & 1) != 0 || row >= a.n) return;
    uint16_t* y = static_cast<uint16_t*>(a.y) + row / 2;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (m0 + e >= a.m) break;
      const float g = round_f16(v[e]);
      const float u = round_f16(up[e]);
      y[static_cast<size_t>(m0 + e) * a.y_ld] =
          __builtin_bit_cast(uint16_t, static_cast<_Float16>(silu_f16(g) * u));
    }
  } else {
    if (row >= a.n) return;
    const float b =
        a.bias != nullptr ? static_cast<float>(__builtin_bit_cast(_Float16, a.bias[row])) : 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (m0 + e >= a.m) break;
      const size_t at = static_cast<size_t>(m0 + e) * a.y_ld + row;
      if constexpr (MODE == kModeF32) {
        static_cast<float*>(a.y)[at] = v[e] + b;
      } else {
        static_cast<uint16_t*>(a.y)[at] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(v[e] + b));
      }
    }
  }
}

// A workgroup owns `wr` 16-row weight tiles (wr row waves, a runtime value)
// times S K-split ways: wave w takes row slot w % wr and K part w / wr.
// P: chunks in flight per wave; KC: K per chunk (128 or 32); MT: 16-row
// activation tiles (m <= 16 MT).
//
// PR = 2 (128-K chunks, no K split, an even chunk count): codes are fetched
// as chunk pairs with 8 rows x 128 bytes per load instruction (full cache
// lines; the MFMA layout itself allows only 16 rows x 64 bytes) and moved to
// the MFMA layout through a private LDS slab of the wave.
//
// At most 8 waves per workgroup (about one workgroup per CU, so two waves per
// SIMD): a wave may use up to 256 VGPRs, which pays for a deep ring of loads
// in flight.
constexpr int kMaxWaves = 8;
// Word 3 of a buffer resource for raw byte-addressed loads (32-bit data
// format, no swizzle), and the cache-policy operand of the buffer-load
// builtins that marks a load non-temporal.
constexpr int kBufferFlags = 0x00020000;
constexpr int kNtLoad = 2;
// Largest weight the pair kernel addresses through 32-bit buffer offsets.
constexpr uint64_t kMaxBufferBytes = 0x7FFFFFFFu;

template <int S, int P, int KC, int MT, int MODE, int PR = 1>
__global__ __launch_bounds__(64 * kMaxWaves) void gemv_w4_kernel(W4Args a) {
  static_assert(PR == 1 || (PR == 2 && KC == 128 && S == 1), "chunk pairs: 128-K chunks, no split");
  constexpr int kSteps = KC / 32, kLaneK = KC / 4;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int threads = blockDim.x, wr = threads / (64 * S);
  const int rows_wg = 16 * wr;
  uint32_t* so_lds = reinterpret_cast<uint32_t*>(lds);  // [groups][rows_wg]: s | o << 16
  uint16_t* x_lds = reinterpret_cast<uint16_t*>(lds + static_cast<size_t>(a.groups) * rows_wg * 4);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int slot = wave % wr, part = wave / wr;
  const int r16 = lane & 15, qd = lane >> 4;
  const int row = blockIdx.x * wr * 16 + slot * 16 + r16;  // this lane's weight row
  const int rowc = min(row, a.n - 1);                       // rows past n re-read the last one
  const int last = a.nchunks - 1;

  // The weight codes of this lane's row travel in a ring of P chunks; part
  // `part` takes chunks part, part + S, part + 2S, ...  A ring slot holds PR
  // chunks; slot p of a round starts at chunk cb + (part + S p) PR.
  u32x4 wbuf[P][PR];
  const uint8_t* wp[PR];
  if constexpr (PR == 1) {
    wp[0] = a.w + static_cast<size_t>(rowc) * (a.k / 2) + qd * (kLaneK / 2);
  } else {  // load instruction h covers rows 8h .. 8h+7 of the tile, 8 lanes x 16 bytes each
#pragma unroll
    for (int h = 0; h < 2; ++h)
      wp[h] = a.w + static_cast<size_t>(min(row - r16 + 8 * h + lane / 8, a.n - 1)) * (a.k / 2) +
              (lane % 8) * 16;
  }
  const int last_slot = PR == 1 ? last : a.nchunks - PR;  // first chunk of the last slot
  auto fetch = [&](int p, int c) {
#pragma unroll
    for (int h = 0; h < PR; ++h)
      wbuf[p][h] = load_codes<KC>(wp[h] + static_cast<size_t>(c) * (KC / 2));
  };

  // Staging of scales/offsets (to LDS as [group][row]: per-lane loads of them
  // would touch 16 rows' lines per instruction, as costly as a weight load)
  // and of x, in batches of kBatch loads per thread (indices clamped so that
  // every load is consumed on every path).  The first batch of each is
  // requested BEFORE the ring's first chunks and stored after them: wait
  // counts retire in issue order, so the stores then wait for the staging
  // loads only, and the ring keeps flowing through the staging and the
  // barrier.  (Requested after the ring, the staging data would make every
  // wave wait for its whole ring before its first chunk.)
  constexpr int kBatch = 8;
  const int staged = rows_wg * a.groups;
  const float inv_groups = 1.0f / static_cast<float>(a.groups);
  const int row_wg0 = blockIdx.x * rows_wg;
  auto so_load = [&](int i0, uint32_t (&v)[kBatch]) {
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int i = min(i0 + u * threads, staged - 1);
      const int r = quot(i, inv_groups), g = i - r * a.groups;
      const size_t src = static_cast<size_t>(min(row_wg0 + r, a.n - 1)) * a.groups + g;
      v[u] = a.scales[src] | (static_cast<uint32_t>(a.offsets[src]) << 16);
    }
  };
  auto so_store = [&](int i0, const uint32_t (&v)[kBatch]) {
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {  // past the end: the last entry again, same value
      const int i = min(i0 + u * threads, staged - 1);
      const int r = quot(i, inv_groups), g = i - r * a.groups;
      so_lds[g * rows_wg + r] = v[u];
    }
  };
  struct XPass {
    int c0, vpr, total;
    float inv_vpr;
  };
  auto x_pass = [&](int c0, int c1) {
    const int vpr = (c1 - c0) * (KC / 8);  // 8-half vectors per row
    return XPass{c0, vpr, a.m * vpr, 1.0f / static_cast<float>(vpr)};
  };
  auto x_load = [&](const XPass& xp, int v0, u32x4 (&val)[kBatch]) {
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int v = min(v0 + u * threads, xp.total - 1);
      const int r = quot(v, xp.inv_vpr), e = v - r * xp.vpr;
      val[u] = load16(a.x + static_cast<size_t>(r) * a.k + static_cast<size_t>(xp.c0) * KC + e * 8);
    }
  };
  auto x_store = [&](const XPass& xp, int v0, const u32x4 (&val)[kBatch]) {
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {  // unconditional, as above
      const int v = min(v0 + u * threads, xp.total - 1);
      const int r = quot(v, xp.inv_vpr), e = v - r * xp.vpr;
      *reinterpret_cast<f16x8*>(x_lds + r * a.xstride + e * 8) = x_perm(val[u]);
    }
  };
  // a pass of x, from vector v_first of this thread on
  auto stage_x = [&](const XPass& xp, int v_first) {
    for (int v0 = v_first; v0 < xp.total; v0 += threads * kBatch) {
      u32x4 val[kBatch];
      x_load(xp, v0, val);
      x_store(xp, v0, val);
    }
  };
  {
    const XPass xp = x_pass(0, min(a.cpp, a.nchunks));
    uint32_t sov[kBatch];
    u32x4 xv[kBatch];
    so_load(tid, sov);
    x_load(xp, tid, xv);
#pragma unroll
    for (int p = 0; p < P; ++p) fetch(p, min((part + S * p) * PR, last_slot));
    so_store(tid, sov);
    x_store(xp, tid, xv);
    for (int i0 = tid + threads * kBatch; i0 < staged; i0 += threads * kBatch) {
      so_load(i0, sov);
      so_store(i0, sov);
    }
    stage_x(xp, tid + threads * kBatch);
  }

  // A-fragment rows of this lane (activation rows past m repeat the last one)
  const uint16_t* xl[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
    xl[mt] = x_lds + min(16 * mt + r16, a.m - 1) * a.xstride + qd * kLaneK;

  f32x4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  constexpr f16x8 kOnes = {1, 1, 1, 1, 1, 1, 1, 1};
  const uint32_t magic = opaque(0x54005400u);  // 64.0 in both halves

  // The wave's private slab for chunk-pair transposes (after x and the
  // split-K reduction space): 16 rows of 128 code bytes, rows padded to 144
  // bytes so that both the row-major writes and the MFMA-layout reads are
  // free of bank conflicts.
  uint8_t* slab = reinterpret_cast<uint8_t*>(x_lds + static_cast<size_t>(a.m) * a.xstride) +
                  a.slab_off + wave * kSlabBytes;

  // Rounds of P slots per part.  A pass holds cpp chunks, a multiple of
  // S*P*PR, so pass boundaries fall on round boundaries for every part alike.
  // Full rounds are straight-line code (every slot valid); only the last,
  // partial round of the last pass tests its slots.  Branches inside a round
  // would make the compiler's wait-count tracking merge conservatively and
  // wait for the whole ring instead of one slot.
  constexpr int kRound = S * P * PR;
  auto round = [&](int cb, int c0, auto full_tag) {
    constexpr bool kFull = decltype(full_tag)::value;
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int cs = cb + (part + S * p) * PR;
      if (kFull || cs < a.nchunks) {  // wave-uniform
        u32x4 words[PR];
        if constexpr (PR == 1) {
          words[0] = wbuf[p][0];
        } else {  // row-major pair -> MFMA layout (lane (qd, r16): row r16, 16 bytes at qd)
#pragma unroll
          for (int h = 0; h < 2; ++h)
            *reinterpret_cast<u32x4*>(slab + (8 * h + lane / 8) * kSlabRow + (lane % 8) * 16) =
                wbuf[p][h];
#pragma unroll
          for (int h = 0; h < 2; ++h)
            words[h] = *reinterpret_cast<const u32x4*>(slab + r16 * kSlabRow + h * 64 + qd * 16);
        }
#pragma unroll
        for (int h = 0; h < PR; ++h) {
          const int c = cs + h;
          f16x8 xa[MT][kSteps];
          f32x4 xs[MT];
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            xs[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < kSteps; ++j) {
              xa[mt][j] = *reinterpret_cast<const f16x8*>(xl[mt] + (c - c0) * KC + 8 * j);
              xs[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[mt][j], kOnes, xs[mt], 0, 0, 0);
            }
          }
          const uint32_t so = so_lds[(c * KC / a.group_size) * rows_wg + slot * 16 + r16];
          const float sc = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(so)));
          const float of = fmaf(-kCodeBias, sc,
                                static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(so >> 16))));
          f16x8 q[kSteps];
#pragma unroll
          for (int j = 0; j < kSteps; ++j) q[j] = codes_f16(words[h][j], magic);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < kSteps; ++j)
              d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[mt][j], q[j], d, 0, 0, 0);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[mt][e] = fmaf(of, xs[mt][e], fmaf(sc, d[e], acc[mt][e]));
          }
        }
      }
      // refill the slot with this part's chunks one round ahead
      fetch(p, min(cs + kRound, last_slot));
    }
  };
  for (int c0 = 0; c0 < a.nchunks; c0 += a.cpp) {  // x passes (workgroup-uniform)
    const int c1 = min(c0 + a.cpp, a.nchunks);
    if (c0 > 0) {
      __syncthreads();  // every wave is done with the previous pass's x
      stage_x(x_pass(c0, c1), tid);
    }
    __syncthreads();
    const int full_end = c0 + (c1 - c0) / kRound * kRound;
    for (int cb = c0; cb < full_end; cb += kRound) round(cb, c0, std::true_type{});
    if (full_end < c1) round(full_end, c0, std::false_type{});
  }

  if constexpr (S > 1) {
    // K parts 1..S-1 hand their partial sums to part 0 through LDS (after the
    // x region); part 0 adds them in part order, so the result is deterministic.
    f32x4* red = reinterpret_cast<f32x4*>(x_lds + static_cast<size_t>(a.m) * a.xstride);
    if (part > 0) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        red[(((part - 1) * wr + slot) * MT + mt) * kWave + lane] = acc[mt];
    }
    __syncthreads();
    if (part > 0) return;
#pragma unroll
    for (int q = 1; q < S; ++q)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[mt] += red[(((q - 1) * wr + slot) * MT + mt) * kWave + lane];
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) store_tile<MODE>(a, acc[mt], 16 * mt + 4 * qd, row, r16);
}

// The pair kernel: the default for 128-K chunks, an even chunk count and a
// power-of-two group_size / 128.  A wave owns one 16-row tile over the full K
// and walks it in chunk pairs (256 K = 128 bytes of each row).  Each pair is
// fetched by two load instructions of 8 rows x 128 bytes (full lines): in
// instruction 0 the lanes with (lane & 8) == 0 load piece qd of their own
// row r16 and the others piece 4 + qd of row r16 - 8; instruction 1 covers
// rows 8..15 the same way.  So every lane loads 16 bytes it keeps (chunk 0 of
// the pair in the MFMA layout: row r16, K qd*32 .. qd*32 + 31) and 16 bytes
// that its partner lane r16 ^ 8 keeps (chunk 1), handed over by one DPP
// row_ror:8 per dword -- no LDS round trip.
//
// The ring is read through buffer loads (the lane's row offset in a VGPR, the
// pair's offset in the scalar offset), and the last round's refills go
// through a buffer resource with no records, which reads nothing.
//
// Measured against the slab kernel above (same MFMA math): a ring of P = 4
// pairs per wave (8 KB in flight) beats deeper rings; the last round fetches
// nothing (re-fetching the last pair in every slot cost ~2 us at the
// Llama-3.1-8B gate_up shape); x is staged in one batch of loads; and each
// wave stages the scales and offsets of its own 16 rows into its own LDS rows
// with 16-byte loads, so that only x needs the workgroup barrier.
//
// Order of the prologue: x and scale loads, then the ring's first P pairs,
// then the LDS stores of x and scales.  Wait counts retire in issue order, so
// the stores wait for the staging loads only.
//
// kW8: the same walk over an INT8 weight [n, k] with one fp16 scale per row
// (gemv_w8a16): a pair is then 128 K, a chunk 64 K, the codes become exact
// fp16 values by byte permutes (int8x8_to_f16), the MFMAs accumulate straight
// into the output registers, and the row scale (and bias) apply once at the
// end.  K need only be a multiple of 16: the staged x is zero past k, and
// code loads past the end of a row are clamped to its last 16 bytes.
template <int P, int MT, int MODE, int NB, bool kMulti, bool kW8 = false>
__global__ __launch_bounds__(64 * kMaxWaves) void gemv_w4_pairs_kernel(W4Args a) {
  constexpr int kKP = kW8 ? 128 : 256;  // K per chunk pair
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int threads = blockDim.x, nw = threads / 64;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, qd = lane >> 4;
  const bool low = (lane & 8) == 0;
  const int npairs = a.nchunks / 2, lastp = npairs - 1;
  const int sstride = a.gpp + 1;  // dwords per staged row (odd: conflict-free column reads)
  uint32_t* so_lds = reinterpret_cast<uint32_t*>(lds) + wave * 16 * sstride;  // this wave's rows
  uint16_t* x_lds = reinterpret_cast<uint16_t*>(lds + static_cast<size_t>(nw) * 16 * sstride * 4);
  const int row0 = (blockIdx.x * nw + wave) * 16;  // first row of this wave's tile
  const int row = row0 + r16;                       // this lane's output row
  const int kb = kW8 ? a.k : a.k / 2;  // bytes per weight row
  const int pc0 = (low ? qd : 4 + qd) * 16, pc1 = (low ? 4 + qd : qd) * 16;
  // The codes are read through buffer loads: the lane's row offset in a
  // VGPR, the pair's offset (uniform) in the scalar offset, so a refill costs
  // no VALU.  The weight is < 4 GiB (launch_pairs).  A load through `none`
  // (no records) returns zeros without a memory access.
  const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(a.w), 0, static_cast<int>(static_cast<uint32_t>(a.n) * static_cast<uint32_t>(kb)),
      kBufferFlags);
  const __amdgpu_buffer_rsrc_t none = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(a.w), 0, 0, kBufferFlags);
  const uint32_t rb0 = static_cast<uint32_t>(min(row0 + (low ? r16 : r16 - 8), a.n - 1)) * kb;
  const uint32_t rb1 = static_cast<uint32_t>(min(row0 + (low ? r16 + 8 : r16), a.n - 1)) * kb;
  u32x4 ring[P][2];
  auto fetch_from = [&](int s, int q, __amdgpu_buffer_rsrc_t res) {
    if constexpr (kW8) {  // pieces past the row end are clamped to its last 16 bytes (x is zero there)
      const int o0 = min(q * 128 + pc0, kb - 16), o1 = min(q * 128 + pc1, kb - 16);
      ring[s][0] = __builtin_amdgcn_raw_buffer_load_b128(res, static_cast<int>(rb0) + o0, 0, kNtLoad);
      ring[s][1] = __builtin_amdgcn_raw_buffer_load_b128(res, static_cast<int>(rb1) + o1, 0, kNtLoad);
    } else {
      ring[s][0] = __builtin_amdgcn_raw_buffer_load_b128(res, static_cast<int>(rb0) + pc0, q * 128, kNtLoad);
      ring[s][1] = __builtin_amdgcn_raw_buffer_load_b128(res, static_cast<int>(rb1) + pc1, q * 128, kNtLoad);
    }
  };
  auto fetch = [&](int s, int q) { fetch_from(s, q, wres); };

  // x of pairs [qa, qa + cpp) -> LDS (INT4: permuted to the codes' order);
  // vectors past the end re-load the last one (same value, no branch).
  const int kpass = a.cpp * kKP;
  auto xcvt = [](u32x4 v) {
    if constexpr (kW8) return __builtin_bit_cast(f16x8, v);
    else return x_perm(v);
  };
  auto x_addr = [&](int v, int qa, int xvecs) {
    v = min(v, xvecs - 1);
    const int per = min(kpass, a.k - qa * kKP) / 8;  // vectors per row in this pass
    const int r = quot(v, 1.0f / static_cast<float>(per)), e = v - r * per;
    return std::pair<const uint16_t*, uint16_t*>(
        a.x + static_cast<size_t>(r) * a.k + static_cast<size_t>(qa) * kKP + e * 8,
        x_lds + r * a.xstride + e * 8);
  };
  // INT4: sum(x) over each 128-K chunk of the pass and each activation row,
  // [chunk][16 MT rows] in fp32 after x, taken while x is staged.  Vector v
  // of the pass holds K [8e, 8e + 8) of row r (v = r * per + e), and the 16
  // vectors of one (row, chunk) sit in 16 consecutive lanes of one aligned
  // group (v = tid + multiples of the block size, per a multiple of 16), so
  // one 16-lane DPP sum gives the chunk's sum.  Every wave reads these sums
  // instead of computing them with MFMAs against a ones operand.
  constexpr int kMP = 16 * MT;
  float* xsum_lds = reinterpret_cast<float*>(x_lds + static_cast<size_t>(a.m) * a.xstride);
  auto x_put = [&](int v, int qa, int xvecs, u32x4 raw) {
    const auto pr = x_addr(v, qa, xvecs);
    const f16x8 h = xcvt(raw);
    *reinterpret_cast<f16x8*>(pr.second) = h;
    if constexpr (!kW8) {
      const f16x2 one = {static_cast<_Float16>(1), static_cast<_Float16>(1)};
      float sum = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        sum = __builtin_amdgcn_fdot2(f16x2{h[2 * j], h[2 * j + 1]}, one, sum, false);
      sum = group_sum<16>(sum);
      if ((lane & 15) == 0 && v < xvecs) {
        const int per = min(kpass, a.k - qa * kKP) / 8;
        const int r = quot(v, 1.0f / static_cast<float>(per)), e = v - r * per;
        xsum_lds[(e >> 4) * kMP + r] = sum;
      }
    }
  };
  auto stage_x_rest = [&](int qa, int v_from) {  // in batches of 8 loads per thread
    const int xvecs = a.m * (min(kpass, a.k - qa * kKP) / 8);
    for (int v0 = v_from; v0 < xvecs; v0 += 8 * threads) {
      u32x4 val[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) val[u] = load16(x_addr(v0 + u * threads, qa, xvecs).first);
#pragma unroll
      for (int u = 0; u < 8; ++u) x_put(v0 + u * threads, qa, xvecs, val[u]);
    }
  };
  // INT8: zeros from k to the end of the last pair (LDS stores only)
  auto zero_x_tail = [&](int qa, int qe) {
    if constexpr (kW8) {
      const int real = (a.k - qa * kKP) / 8, padded = (qe - qa) * (kKP / 8);
      if (real >= padded) return;
      for (int i = tid; i < a.m * (padded - real); i += threads) {
        const int r = i / (padded - real), e = real + i % (padded - real);
        *reinterpret_cast<u32x4*>(x_lds + r * a.xstride + e * 8) = u32x4{0u, 0u, 0u, 0u};
      }
    }
  };
  // scales and offsets of this wave's rows for groups [g0, g0 + gn): lane
  // (qd, r16) takes row r16, 8 groups per 16-byte vector when aligned
  const bool svec = !kW8 && (a.groups % 8) == 0 && (a.gpp % 8) == 0;
  const size_t srow = static_cast<size_t>(min(row, a.n - 1)) * a.groups;
  auto so_put = [&](int gl, u32x4 s4, u32x4 o4) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      so_lds[r16 * sstride + gl + 2 * t] = (s4[t] & 0xFFFFu) | (o4[t] << 16);
      so_lds[r16 * sstride + gl + 2 * t + 1] = (s4[t] >> 16) | (o4[t] & 0xFFFF0000u);
    }
  };
  // (vector path: vectors first_vec, first_vec + 4, ...; scalar path: groups qd, qd + 4, ...)
  auto stage_so = [&](int g0, int gn, int first_vec) {
    if constexpr (kW8) return;
    if (svec) {
      for (int gv = first_vec; gv < gn / 8; gv += 4)
        so_put(gv * 8, load16(a.scales + srow + g0 + gv * 8), load16(a.offsets + srow + g0 + gv * 8));
    } else {
      for (int g = qd; g < gn; g += 4)
        so_lds[r16 * sstride + g] = a.scales[srow + g0 + g] |
                                    (static_cast<uint32_t>(a.offsets[srow + g0 + g]) << 16);
    }
  };

  uint16_t row_scale = 0;  // INT8: this lane's row scale, requested before the ring
  {  // prologue of pass 0
    const int xvecs = a.m * (min(kpass, a.k) / 8);
    u32x4 xv[NB];
#pragma unroll
    for (int u = 0; u < NB; ++u) xv[u] = load16(x_addr(tid + u * threads, 0, xvecs).first);
    if constexpr (kW8) row_scale = a.scales[min(row, a.n - 1)];
    const int gn = min(a.gpp, a.groups);
    const int gv0 = min(qd, gn / 8 - 1);  // first vector of this lane (clamped; vector path)
    u32x4 s4 = {0u, 0u, 0u, 0u}, o4 = {0u, 0u, 0u, 0u};
    if (svec) {
      s4 = load16(a.scales + srow + gv0 * 8);
      o4 = load16(a.offsets + srow + gv0 * 8);
    }
#pragma unroll
    for (int p = 0; p < P; ++p) fetch(p, min(p, lastp));
#pragma unroll
    for (int u = 0; u < NB; ++u) x_put(tid + u * threads, 0, xvecs, xv[u]);
    zero_x_tail(0, min(a.cpp, npairs));
    if (svec) {
      if (qd < gn / 8) so_put(gv0 * 8, s4, o4);
      stage_so(0, gn, qd + 4);
    } else {
      stage_so(0, gn, qd);
    }
    stage_x_rest(0, tid + NB * threads);
  }

  const uint16_t* xl[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
    xl[mt] = x_lds + min(16 * mt + r16, a.m - 1) * a.xstride + qd * (kW8 ? 16 : 32);
  f32x4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  const uint32_t magic = opaque(0x54005400u);

  // one 128-K chunk: c = chunk index within the pass
  // (passes hold whole groups, so the group of chunk c is c >> gq_shift)
  auto chunk = [&](int c, u32x4 words) {
    if constexpr (kW8) {  // 64 K: two MFMA steps of 8 codes per lane, into acc directly
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const f16x8 q = int8x8_to_f16(u32x2{words[2 * j], words[2 * j + 1]});
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
              *reinterpret_cast<const f16x8*>(xl[mt] + c * 64 + 8 * j), q, acc[mt], 0, 0, 0);
      }
      return;
    }
    f32x4 xs[MT], d[MT];
    f16x8 xa[MT][4];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      xs[mt] = *reinterpret_cast<const f32x4*>(xsum_lds + c * kMP + 16 * mt + 4 * qd);
      d[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 4; ++j) xa[mt][j] = *reinterpret_cast<const f16x8*>(xl[mt] + c * 128 + 8 * j);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f16x8 q = codes_f16(words[j], magic);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) d[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[mt][j], q, d[mt], 0, 0, 0);
    }
    const uint32_t so = so_lds[r16 * sstride + (c >> a.gq_shift)];
    const float sc = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(so)));
    const float of = fmaf(-kCodeBias, sc,
                          static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(so >> 16))));
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[mt][e] = fmaf(of, xs[mt][e], fmaf(sc, d[mt][e], acc[mt][e]));
  };
  // pair q (slot s) of the pass starting at pair qa
  auto consume = [&](int q, int s, int qa) {
    u32x4 keep, recv;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      keep[t] = low ? ring[s][0][t] : ring[s][1][t];
      recv[t] = static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(
          static_cast<int>(low ? ring[s][1][t] : ring[s][0][t]), 0x128, 0xF, 0xF, false));  // row_ror:8
    }
    chunk(2 * (q - qa), keep);
    chunk(2 * (q - qa) + 1, recv);
  };

  // One x pass over all pairs, a whole number of rounds (the single-pass
  // kernel): every round in one loop, the closing round's refills reading
  // nothing (`none`).  As straight-line code after the loop, the closing
  // round made the compiler copy the ring on the way in, and the copy waited
  // for every pair in flight; so did a second, general form of the rounds in
  // the same kernel.
  auto run_all = [&]() {
    for (int qb = 0; qb < npairs; qb += P) {
#pragma unroll
      for (int s = 0; s < P; ++s) {
        consume(qb + s, s, 0);
        fetch_from(s, qb + s + P, qb + s + P < npairs ? wres : none);
        __builtin_amdgcn_sched_barrier(0x78F);  // only vector-memory instructions stay put
      }
    }
  };
  // The pairs [qa, qe) of one x pass (the multi-pass kernel).  Full rounds
  // (every refill a valid pair) are straight-line code, so the compiler waits
  // per ring slot; a closing round of exactly P pairs is straight-line too.
  // Any other shape of the last rounds tests each slot.
  auto run_pass = [&](int qa, int qe) {
    int qb = qa;
    for (; qb + P <= qe && qb + 2 * P <= npairs; qb += P) {
#pragma unroll
      for (int s = 0; s < P; ++s) {
        consume(qb + s, s, qa);
        fetch(s, qb + s + P);
        // keep the refill here: left to the scheduler, all refills of a
        // round sank to its end and the ring drained once per round
        __builtin_amdgcn_sched_barrier(0x78F);  // only vector-memory instructions stay put
      }
    }
    if (qe == npairs && qb + P == qe) {
#pragma unroll
      for (int s = 0; s < P; ++s) consume(qb + s, s, qa);
      return;
    }
    for (; qb < qe; qb += P) {
#pragma unroll
      for (int s = 0; s < P; ++s) {
        if (qb + s < qe) {
          consume(qb + s, s, qa);
          if (qb + s + P < npairs) fetch(s, qb + s + P);
        }
      }
    }
  };
  __syncthreads();
  if constexpr (!kMulti) {
    run_all();
  } else {
    run_pass(0, min(a.cpp, npairs));
    for (int qa = a.cpp; qa < npairs; qa += a.cpp) {  // further x passes (workgroup-uniform)
      __syncthreads();  // every wave is done with the previous pass's x and scales
      stage_x_rest(qa, tid);
      zero_x_tail(qa, min(qa + a.cpp, npairs));
      const int g0 = (qa * 2) >> a.gq_shift;
      stage_so(g0, min(a.gpp, a.groups - g0), qd);
      __syncthreads();
      run_pass(qa, min(qa + a.cpp, npairs));
    }
  }
  if constexpr (kW8) {
    const float s = static_cast<float>(__builtin_bit_cast(_Float16, row_scale));
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] *= s;  // acc * s + bias, as gemv_weight_only.cu:36
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) store_tile<MODE>(a, acc[mt], 16 * mt + 4 * qd, row, r16);
}

// The K-slice kernel: the default for INT4 weights whose K is 8 or fewer
// slices of CPW 128-K chunks (the Llama-3.1-8B gate_up: 8 slices of 512 K)
// and whose rows are whole 16-row tiles.  A workgroup owns T consecutive
// 16-row tiles; wave w owns K slice w (chunks w CPW .. w CPW + CPW - 1) of
// every one of them.  So each wave needs only its own slice of x, which it
// loads once into registers in the MFMA A-operand layout (whole cache lines,
// transposed through the wave's own LDS rows; no per-chunk LDS reads of x,
// no workgroup-wide staging pass), and computes that slice's per-chunk
// sum(x) and sum(x * code bias) once, for all of its tiles.  The wave then
// walks its tiles, fetching each tile's slice as chunk pairs of full cache
// lines (the pair kernel's loads and DPP hand-over) through a ring of U
// tiles' pairs.  Codes become fp16 with two magics (codes_f16_2m, 5 VALU per
// 8 codes); per chunk only acc += s * (x . (bias + q)) runs on the vector
// ALU, and the offset and bias terms of all the slice's chunks enter each
// tile as two fp32 MFMAs with K = the chunks.  Each tile leaves one partial
// 16x16 result in LDS; after one barrier, wave w adds the nw partials of
// tile w (w + nw, ...) in slice order -- a fixed order, so the result is
// deterministic -- and stores it through the epilogue.  Scales and
// offsets of the workgroup's rows are staged once into LDS (coalesced:
// [n, groups] is contiguous over the workgroup's rows).
// Waves per workgroup of the K-slice kernel: 16 when a slice's x fits in
// half the registers (two 128-K chunks of one activation tile), else 8.
template <int CPW, int MT>
constexpr int kslice_max_waves() { return CPW * MT <= 2 ? 16 : kMaxWaves; }

template <int CPW, int U, int MT, int MODE>
__global__ __launch_bounds__((64 * kslice_max_waves<CPW, MT>())) void gemv_w4_kslice_kernel(W4Args a) {
  static_assert(CPW == 2 || CPW == 4, "a slice's chunks are the K of one fp32 MFMA (at most 4)");
  constexpr int kPPT = CPW / 2;  // chunk pairs per tile and wave
  constexpr int P = kPPT * U;    // ring depth in pairs: U tiles
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int threads = blockDim.x, nw = threads / 64;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, qd = lane >> 4;
  const bool low = (lane & 8) == 0;
  const int T = a.cpp;  // tiles per workgroup, a multiple of U
  const int ntiles = a.n / 16;
  const int tile0 = blockIdx.x * T;
  const int sstride = a.groups + 1;  // odd: the 16 rows' reads of one group fall in 16 banks
  uint32_t* so_lds = reinterpret_cast<uint32_t*>(lds);   // [16 T rows][groups + 1]: s | o << 16
  f32x4* red = reinterpret_cast<f32x4*>(lds + a.slab_off);  // [T][nw][MT][64 lanes]
  const int kb = a.k / 2;
  const int c0 = wave * CPW;  // first chunk of this wave's slice
  const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(a.w), 0, static_cast<int>(static_cast<uint32_t>(a.n) * static_cast<uint32_t>(kb)),
      kBufferFlags);
  const __amdgpu_buffer_rsrc_t none = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(a.w), 0, 0, kBufferFlags);
  // pair loads as in the pair kernel: instruction 0 covers rows 0..7 of the
  // tile (full 128-byte lines), instruction 1 rows 8..15
  const int pc0 = (low ? qd : 4 + qd) * 16, pc1 = (low ? 4 + qd : qd) * 16;
  const int vo0 = (low ? r16 : r16 - 8) * kb + pc0;
  const int vo1 = (low ? r16 + 8 : r16) * kb + pc1;
  const int nq = T * kPPT;  // (tile, pair) steps of this wave
  u32x4 ring[P][2];
  // step q: local tile q / kPPT, pair q % kPPT of the slice; tiles past the
  // last one (and steps past the end) read nothing
  auto fetch = [&](int s, int q) {
    const int t = tile0 + q / kPPT;
    const __amdgpu_buffer_rsrc_t res = (q < nq && t < ntiles) ? wres : none;
    const int soff = t * 16 * kb + (c0 / 2 + q % kPPT) * 128;
    ring[s][0] = __builtin_amdgcn_raw_buffer_load_b128(res, vo0, soff, kNtLoad);
    ring[s][1] = __builtin_amdgcn_raw_buffer_load_b128(res, vo1, soff, kNtLoad);
  };

  // x of this wave's slice in the A-operand layout: lane (qd, r16) holds
  // row min(16 mt + r16, m - 1), K (c0 + c) 128 + 32 qd + 8 j .. + 7,
  // permuted to the codes' nibble order.  Read straight in that layout, a
  // load instruction would touch 16 rows x 2 cache lines for 1 KB; instead
  // each (chunk, tile) block of 16 rows x 256 bytes is fetched as 4 loads of
  // 4 whole rows (full lines), written to the wave's own LDS rows and read
  // back in the MFMA layout.  The staging rows lie in the partial-sum region,
  // which no wave writes before the barrier below.
  f16x8 xa[CPW][MT][4];
  {
    constexpr int kXRow = 272;  // bytes per staged row: 256 + 16 (conflict-free column reads)
    uint8_t* xst = lds + a.slab_off + wave * 16 * kXRow;
    const int lr = lane / 16, lc = (lane % 16) * 16;  // load: row 4 i + lr, bytes lc
#pragma unroll
    for (int c = 0; c < CPW; ++c)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        u32x4 v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
          v[i] = load16(reinterpret_cast<const uint8_t*>(
                            a.x + static_cast<size_t>(min(16 * mt + 4 * i + lr, a.m - 1)) * a.k +
                            (c0 + c) * 128) + lc);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          *reinterpret_cast<u32x4*>(xst + (4 * i + lr) * kXRow + lc) = v[i];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          xa[c][mt][j] = x_perm(*reinterpret_cast<const u32x4*>(xst + r16 * kXRow + qd * 64 + 16 * j));
      }
  }
  // scales and offsets of the workgroup's rows, requested before the ring
  constexpr int kSoBatch = 8;
  const int staged = 16 * T * a.groups;
  const float inv_groups = 1.0f / static_cast<float>(a.groups);
  const size_t so_base = static_cast<size_t>(tile0) * 16 * a.groups;
  const size_t so_last = static_cast<size_t>(a.n) * a.groups - 1;
  uint32_t sov[kSoBatch];
  auto so_load = [&](int i0) {
#pragma unroll
    for (int u = 0; u < kSoBatch; ++u) {
      const size_t src = min(so_base + min(i0 + u * threads, staged - 1), so_last);
      sov[u] = a.scales[src] | (static_cast<uint32_t>(a.offsets[src]) << 16);
    }
  };
  auto so_store = [&](int i0) {
#pragma unroll
    for (int u = 0; u < kSoBatch; ++u) {  // past the end: the last entry again, same value
      const int i = min(i0 + u * threads, staged - 1);
      const int r = quot(i, inv_groups), g = i - r * a.groups;
      so_lds[r * sstride + g] = sov[u];
    }
  };
  so_load(tid);
#pragma unroll
  for (int p = 0; p < P; ++p) fetch(p, p);
  so_store(tid);
  for (int i0 = tid + threads * kSoBatch; i0 < staged; i0 += threads * kSoBatch) {
    so_load(i0);
    so_store(i0);
  }
  // Per chunk c of the slice and activation row m: sum(x) and sum(x * bias)
  // (kBias2), in the A layout of v_mfma_f32_16x16x4f32 (lane (qd, r16): row
  // m = r16, chunk qd).  x is the B operand here; A row 4 c holds ones and
  // row 4 c + 1 the biases, so D row 4 c + e, column m, is chunk c's sum e.
  constexpr f16x8 kOnes = {1, 1, 1, 1, 1, 1, 1, 1};
  constexpr f16x8 kZero = {0, 0, 0, 0, 0, 0, 0, 0};
  const f16x8 arow = (r16 & 3) == 0 ? kOnes : ((r16 & 3) == 1 ? kBias2 : kZero);
  float sx[MT], sb[MT];  // this lane's sum(x), sum(x * bias): row 16 mt + r16, chunk qd
  {
    f32x4 sums[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) sums[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
      const f16x8 ac = (r16 >> 2) == c ? arow : kZero;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          sums[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ac, xa[c][mt][j], sums[mt], 0, 0, 0);
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      sx[mt] = sums[mt][0];
      sb[mt] = sums[mt][1];
    }
  }
  const uint32_t m1024 = opaque(0x64006400u), m64 = opaque(0x54005400u);
  __syncthreads();  // scales and offsets staged

  for (int qb = 0; qb < nq; qb += P) {  // U tiles per round (wave-uniform)
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = qb / kPPT + u;  // local tile
      const uint32_t* so_row = so_lds + (t * 16 + r16) * sstride;
      // The tile starts from its slice's offset terms, the sum over its
      // chunks c of o_c sum(x)_c - s_c sum(x * bias)_c, as two fp32
      // products with K = the chunks: lane (qd, r16) brings row r16's o and
      // -s of chunk qd.
      f32x4 acc[MT];
      {
        const uint32_t so = qd < CPW ? so_row[(c0 + qd) >> a.gq_shift] : 0u;
        const float o = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(so >> 16)));
        const float ns = -static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(so)));
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          acc[mt] = __builtin_amdgcn_mfma_f32_16x16x4f32(sx[mt], o, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
          acc[mt] = __builtin_amdgcn_mfma_f32_16x16x4f32(sb[mt], ns, acc[mt], 0, 0, 0);
        }
      }
#pragma unroll
      for (int p = 0; p < kPPT; ++p) {
        const int s = u * kPPT + p;
        u32x4 words[2];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          words[0][e] = low ? ring[s][0][e] : ring[s][1][e];
          words[1][e] = static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(
              static_cast<int>(low ? ring[s][1][e] : ring[s][0][e]), 0x128, 0xF, 0xF, false));  // row_ror:8
        }
        fetch(s, qb + s + P);
        // Nothing crosses: left free, the scheduler hoisted the products of
        // later pairs above the refills and the ring drained once per round.
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int c = 2 * p + h;
          const uint32_t so = so_row[(c0 + c) >> a.gq_shift];
          const float sc = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(so)));
          f32x4 d[MT];
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) d[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const f16x8 q = codes_f16_2m(words[h][j], m1024, m64);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
              d[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[c][mt][j], q, d[mt], 0, 0, 0);
          }
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[mt][e] = fmaf(sc, d[mt][e], acc[mt][e]);
        }
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) red[((t * nw + wave) * MT + mt) * kWave + lane] = acc[mt];
    }
  }
  __syncthreads();  // every slice's partial of every tile is in LDS
  for (int t = wave; t < T; t += nw) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      f32x4 sum = red[((t * nw) * MT + mt) * kWave + lane];
      for (int w = 1; w < nw; ++w) sum += red[((t * nw + w) * MT + mt) * kWave + lane];
      store_tile<MODE>(a, sum, 16 * mt + 4 * qd, (tile0 + t) * 16 + r16, r16);
    }
  }
}

// The INT8 weights' K-slice kernel (gemv_w8a16 from m = 8 on): the INT4
// K-slice kernel's decomposition over an int8 [n, k] with one scale per row.
// Wave w owns K slice w (CPW lines of 128 K = 128 bytes of each row) of the
// workgroup's T tiles; a line of the tile's 16 rows comes as the pair
// kernel's two full-line loads and DPP hand-over, so a lane holds 16 codes of
// its row at bytes 16 qd (MFMA steps 0, 1) and 64 + 16 qd (steps 2, 3):
// step s covers K 64 (s / 2) + 16 qd + 8 (s % 2) .. + 7, the A operand x in
// that (natural) order.  Codes enter the MFMAs biased (1152 + code, 6 VALU
// per 8 codes, int8x8_to_f16_biased); each tile's sum starts from -1152
// sum(x) of the slice, so the products leave x . code.  The row scale and
// the bias apply once, to the reduced sum (gemv_weight_only.cu:36).
template <int CPW, int U, int MT, int MODE>
__global__ __launch_bounds__(64 * kMaxWaves) void gemv_w8_kslice_kernel(W4Args a) {
  constexpr int P = CPW * U;  // ring depth in lines: U tiles
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int threads = blockDim.x, nw = threads / 64;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, qd = lane >> 4;
  const bool low = (lane & 8) == 0;
  const int T = a.cpp;  // tiles per workgroup, a multiple of U
  const int ntiles = a.n / 16;
  const int tile0 = blockIdx.x * T;
  f32x4* red = reinterpret_cast<f32x4*>(lds);  // [T][nw][MT][64 lanes]
  const int kb = a.k;
  const int l0 = wave * CPW;  // first line of this wave's slice
  const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(a.w), 0, static_cast<int>(static_cast<uint32_t>(a.n) * static_cast<uint32_t>(kb)),
      kBufferFlags);
  const __amdgpu_buffer_rsrc_t none = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(a.w), 0, 0, kBufferFlags);
  const int pc0 = (low ? qd : 4 + qd) * 16, pc1 = (low ? 4 + qd : qd) * 16;
  const int vo0 = (low ? r16 : r16 - 8) * kb + pc0;
  const int vo1 = (low ? r16 + 8 : r16) * kb + pc1;
  const int nq = T * CPW;  // (tile, line) steps of this wave
  u32x4 ring[P][2];
  auto fetch = [&](int s, int q) {
    const int t = tile0 + q / CPW;
    const __amdgpu_buffer_rsrc_t res = (q < nq && t < ntiles) ? wres : none;
    const int soff = t * 16 * kb + (l0 + q % CPW) * 128;
    ring[s][0] = __builtin_amdgcn_raw_buffer_load_b128(res, vo0, soff, kNtLoad);
    ring[s][1] = __builtin_amdgcn_raw_buffer_load_b128(res, vo1, soff, kNtLoad);
  };

  // x of the slice in the A layout above, staged as in the INT4 kernel
  // (16 rows x 256 bytes per line and activation tile, whole-line loads,
  // read back transposed from the wave's own LDS rows)
  f16x8 xa[CPW][MT][4];
  {
    constexpr int kXRow = 272;
    uint8_t* xst = lds + wave * 16 * kXRow;
    const int lr = lane / 16, lc = (lane % 16) * 16;
#pragma unroll
    for (int c = 0; c < CPW; ++c)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        u32x4 v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
          v[i] = load16(reinterpret_cast<const uint8_t*>(
                            a.x + static_cast<size_t>(min(16 * mt + 4 * i + lr, a.m - 1)) * a.k +
                            (l0 + c) * 128) + lc);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          *reinterpret_cast<u32x4*>(xst + (4 * i + lr) * kXRow + lc) = v[i];
#pragma unroll
        for (int st = 0; st < 4; ++st)
          xa[c][mt][st] = __builtin_bit_cast(
              f16x8, *reinterpret_cast<const u32x4*>(xst + r16 * kXRow + 128 * (st >> 1) + 32 * qd + 16 * (st & 1)));
      }
  }
#pragma unroll
  for (int p = 0; p < P; ++p) fetch(p, p);
  // -1152 sum(x) of the slice per activation row (all 16 columns equal)
  const f16x8 kM1152 = {-1152, -1152, -1152, -1152, -1152, -1152, -1152, -1152};
  f32x4 base[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    base[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < CPW; ++c)
#pragma unroll
      for (int st = 0; st < 4; ++st)
        base[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[c][mt][st], kM1152, base[mt], 0, 0, 0);
  }
  __syncthreads();  // every wave is done with its staging rows (they hold partial sums next)

  for (int qb = 0; qb < nq; qb += P) {  // U tiles per round (wave-uniform)
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = qb / CPW + u;  // local tile
      f32x4 acc[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[mt] = base[mt];
#pragma unroll
      for (int c = 0; c < CPW; ++c) {
        const int s = u * CPW + c;
        u32x4 words[2];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          words[0][e] = low ? ring[s][0][e] : ring[s][1][e];
          words[1][e] = static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(
              static_cast<int>(low ? ring[s][1][e] : ring[s][0][e]), 0x128, 0xF, 0xF, false));  // row_ror:8
        }
        fetch(s, qb + s + P);
        __builtin_amdgcn_sched_barrier(0);  // the refill stays where it is issued
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          const u32x4 w = words[st >> 1];
          const f16x8 q = int8x8_to_f16_biased((st & 1) ? u32x2{w.z, w.w} : u32x2{w.x, w.y});
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[c][mt][st], q, acc[mt], 0, 0, 0);
        }
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) red[((t * nw + wave) * MT + mt) * kWave + lane] = acc[mt];
    }
  }
  __syncthreads();  // every slice's partial of every tile is in LDS
  for (int t = wave; t < T; t += nw) {
    const int row = (tile0 + t) * 16 + r16;
    if (tile0 + t >= ntiles) break;
    const float sc = static_cast<float>(__builtin_bit_cast(_Float16, a.scales[row]));
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      f32x4 sum = red[((t * nw) * MT + mt) * kWave + lane];
      for (int w = 1; w < nw; ++w) sum += red[((t * nw + w) * MT + mt) * kWave + lane];
      store_tile<MODE>(a, sum * sc, 16 * mt + 4 * qd, row, r16);
    }
  }
}

// LDS a workgroup may take: the device allows 160 KiB per workgroup.
constexpr size_t kLdsBudget = 160 * 1024;
constexpr int kNoFit = 1;  // launch(): the policy's smallest x pass exceeds the LDS budget

template <int S, int P, int KC, int MT, int MODE, int PR = 1>
int launch(W4Args a, int wr_max, hipStream_t stream) {
  if (PR == 2 && a.nchunks % 2 != 0) return kNoFit;
  // Row waves per workgroup: enough that the grid is about one workgroup per
  // compute unit, so x is staged about once per CU.
  const int tiles = (a.n + 15) / 16;
  const int cus = compute_units();
  const int wr = std::max(1, std::min(std::min(wr_max, kMaxWaves / S), (tiles + cus - 1) / cus));
  const size_t red_bytes = static_cast<size_t>(S - 1) * wr * MT * kWave * sizeof(f32x4);
  const size_t so_bytes = static_cast<size_t>(a.groups) * 16 * wr * 4;
  const size_t slab_bytes = PR == 2 ? static_cast<size_t>(wr) * S * kSlabBytes : 0;
  const size_t fixed = red_bytes + so_bytes + slab_bytes;
  const size_t unit = static_cast<size_t>(S) * P * PR;  // chunks per round
  const size_t min_x = static_cast<size_t>(a.m) * (unit * KC + 8) * 2;
  if (fixed + min_x > kLdsBudget) return kNoFit;
  // chunks per x pass: as many as fit, balanced over the passes, a multiple of a round
  const size_t fit =
      ((kLdsBudget - fixed) / (2 * static_cast<size_t>(a.m)) - 8) / KC / unit * unit;
  const int npass = static_cast<int>((a.nchunks + fit - 1) / fit);
  const int per = (a.nchunks + npass - 1) / npass;
  a.cpp = static_cast<int>((per + unit - 1) / unit * unit);
  a.npass = (a.nchunks + a.cpp - 1) / a.cpp;
  a.xstride = a.cpp * KC + 8;
  a.slab_off = static_cast<int>(red_bytes);
  const size_t lds = fixed + static_cast<size_t>(a.m) * a.xstride * 2;
  auto kernel = gemv_w4_kernel<S, P, KC, MT, MODE, PR>;
  if (lds > 64 * 1024) {
    // dynamic LDS above 64 KiB must be granted per kernel and device; the
    // grant is remembered so that steady-state launches make no extra call
    const hipError_t e = grant_dynamic_lds(reinterpret_cast<const void*>(kernel), kLdsBudget);
    if (e != hipSuccess)
      return fail(RLK_EUNSUPPORTED, "gemv_w4a16: %zu bytes of LDS refused (%s)", lds,
                  hipGetErrorString(e));
  }
  const int blocks = (tiles + wr - 1) / wr;
  kernel<<<blocks, 64 * wr * S, lds, stream>>>(a);
  return RLK_OK;
}

// The pair kernel's launch: x passes of cpp pairs (a multiple of P that holds
// whole quantisation groups), as many as the LDS budget allows.
template <int P, int MT, int MODE, bool kW8 = false>
int launch_pairs(W4Args a, hipStream_t stream) {
  constexpr int kKP = kW8 ? 128 : 256;
  const int gq = kW8 ? 1 : a.group_size / 128;
  if (a.nchunks % 2 != 0 || (gq & (gq - 1)) != 0) return kNoFit;
  if (static_cast<uint64_t>(a.n) * static_cast<uint64_t>(kW8 ? a.k : a.k / 2) > kMaxBufferBytes) return kNoFit;
  a.gq_shift = __builtin_ctz(gq);
  const int npairs = a.nchunks / 2;
  const int unit = std::max(P, gq / 2);  // both powers of two
  const int tiles = (a.n + 15) / 16;
  const int cus = compute_units();
  const int nw = std::max(1, std::min(kMaxWaves, (tiles + cus - 1) / cus));
  auto lds_for = [&](int cpp) {  // scales and offsets, x, and (INT4) the chunk sums of x
    const size_t gpp = kW8 ? 0 : static_cast<size_t>(cpp) * 2 / gq;
    return static_cast<size_t>(nw) * 16 * (gpp + 1) * 4 +
           static_cast<size_t>(a.m) * (static_cast<size_t>(cpp) * kKP + 8) * 2 +
           (kW8 ? 0 : static_cast<size_t>(cpp) * 2 * 16 * MT * 4);
  };
  int cpp = (npairs + unit - 1) / unit * unit;
  while (cpp > unit && lds_for(cpp) > kLdsBudget) cpp -= unit;
  if (lds_for(cpp) > kLdsBudget) return kNoFit;
  const int npass = (npairs + cpp - 1) / cpp;
  cpp = ((npairs + npass - 1) / npass + unit - 1) / unit * unit;
  a.cpp = cpp;
  a.npass = npass;
  a.gpp = kW8 ? 0 : cpp * 2 / gq;
  a.xstride = cpp * kKP + 8;
  const size_t lds = lds_for(cpp);
  const int threads = 64 * nw;
  const int xper = (a.m * (std::min(cpp * kKP, a.k) / 8) + threads - 1) / threads;
  auto go = [&](auto kernel) -> int {
    if (lds > 64 * 1024) {
      const hipError_t e = grant_dynamic_lds(reinterpret_cast<const void*>(kernel), kLdsBudget);
      if (e != hipSuccess)
        return fail(RLK_EUNSUPPORTED, "gemv_w4a16: %zu bytes of LDS refused (%s)", lds,
                    hipGetErrorString(e));
    }
    kernel<<<(tiles + nw - 1) / nw, threads, lds, stream>>>(a);
    return RLK_OK;
  };
  // the single-pass kernel takes a whole number of rounds; the rest is general
  if (npass > 1 || npairs % P != 0) return go(gemv_w4_pairs_kernel<P, MT, MODE, 8, true, kW8>);
  if constexpr (P == 4 || P == 2) {  // the defaults: x staged by as many loads per thread as needed
    if (xper <= 2) return go(gemv_w4_pairs_kernel<P, MT, MODE, 2, false, kW8>);
    if (xper <= 4) return go(gemv_w4_pairs_kernel<P, MT, MODE, 4, false, kW8>);
    if (xper <= 8) return go(gemv_w4_pairs_kernel<P, MT, MODE, 8, false, kW8>);
    if (xper <= 12) return go(gemv_w4_pairs_kernel<P, MT, MODE, 12, false, kW8>);
    if (xper <= 16) return go(gemv_w4_pairs_kernel<P, MT, MODE, 16, false, kW8>);
    if (xper <= 20) return go(gemv_w4_pairs_kernel<P, MT, MODE, 20, false, kW8>);
  }
  return go(gemv_w4_pairs_kernel<P, MT, MODE, 24, false, kW8>);  // the rest in a loop
}

// The K-slice kernel's launch: nw = nchunks / CPW waves (at most 8 or 16), T tiles
// per workgroup -- about one workgroup per compute unit, fewer when the
// partials of T tiles would not fit the LDS budget.
template <int CPW, int U, int MT, int MODE>
int launch_kslice(W4Args a, hipStream_t stream) {
  const int gq = a.group_size / 128;
  if (a.group_size % 128 != 0 || (gq & (gq - 1)) != 0 || a.n % 16 != 0 ||
      a.nchunks % CPW != 0 || a.nchunks / CPW > kslice_max_waves<CPW, MT>())
    return kNoFit;
  if (static_cast<uint64_t>(a.n) * static_cast<uint64_t>(a.k / 2) > kMaxBufferBytes) return kNoFit;
  a.gq_shift = __builtin_ctz(gq);
  const int nw = a.nchunks / CPW;
  const int ntiles = a.n / 16;
  const int cus = compute_units();
  auto lds_for = [&](int t) {  // scales and offsets, then the partial sums (which
    // double as the waves' x staging rows, 16 x 272 bytes each)
    const size_t so = (static_cast<size_t>(16) * t * (a.groups + 1) * 4 + 15) / 16 * 16;
    return so + std::max(static_cast<size_t>(t) * nw * MT * kWave * sizeof(f32x4),
                         static_cast<size_t>(nw) * 16 * 272);
  };
  int T = (ntiles + cus - 1) / cus;
  T = (T + U - 1) / U * U;
  while (T > U && lds_for(T) > kLdsBudget) T -= U;
  if (lds_for(T) > kLdsBudget) return kNoFit;

  a.cpp = T;
  a.slab_off = static_cast<int>((static_cast<size_t>(16) * T * (a.groups + 1) * 4 + 15) / 16 * 16);
  const size_t lds = lds_for(T);
  auto kernel = gemv_w4_kslice_kernel<CPW, U, MT, MODE>;
  if (lds > 64 * 1024) {
    const hipError_t e = grant_dynamic_lds(reinterpret_cast<const void*>(kernel), kLdsBudget);
    if (e != hipSuccess)
      return fail(RLK_EUNSUPPORTED, "gemv_w4a16: %zu bytes of LDS refused (%s)", lds,
                  hipGetErrorString(e));
  }
  kernel<<<(ntiles + T - 1) / T, 64 * nw, lds, stream>>>(a);
  return RLK_OK;
}

// Launch policies, selectable for tuning sweeps through RLK_TUNE_W4_CFG.
// Entry 0, the default, is the K-slice kernel (4 chunks per slice, two
// tiles' pairs in flight) from m = 8 on, and the pair kernel below m = 8 or
// where the K-slice kernel does not fit (4 pairs in flight up to m = 8, 2
// above); 9, 10 and 11 are the pair kernel with 2, 8 and 4 pairs at every m;
// 12-15 the K-slice kernel with (chunks per slice, tiles in flight) = (4, 1),
// (4, 2), (2, 2), (2, 4); 8 is the slab kernel with 8
// chunk pairs in flight; 1-7 are slab-kernel variants (K-split ways, slots in
// flight per wave, most row waves per workgroup, chunks per slot).  Shapes the
// pair kernel does not take (an odd chunk count, group_size / 128 not a power
// of two) use the slab kernel; 32-K chunks always use its single-chunk form.
template <int KC, int MT, int MODE>
int launch_cfg(const W4Args& a, int cfg, hipStream_t s) {
  int st = kNoFit;
  if constexpr (KC == 128) {
    switch (cfg) {
      case 8: st = launch<1, 8, KC, MT, MODE, 2>(a, 8, s); break;
      case 9: st = launch_pairs<2, MT, MODE>(a, s); break;
      case 10: st = launch_pairs<8, MT, MODE>(a, s); break;
      case 11: st = launch_pairs<4, MT, MODE>(a, s); break;
      case 12: st = launch_kslice<4, 1, MT, MODE>(a, s); break;
      case 13: st = launch_kslice<4, 2, MT, MODE>(a, s); break;
      case 14: st = launch_kslice<2, 2, MT, MODE>(a, s); break;
      case 15: st = launch_kslice<2, 4, MT, MODE>(a, s); break;
      case 1: st = launch<1, 8, KC, MT, MODE>(a, 8, s); break;
      case 2: st = launch<1, 4, KC, MT, MODE, 2>(a, 8, s); break;
      case 3: st = launch<1, 6, KC, MT, MODE, 2>(a, 8, s); break;
      case 4: st = launch<1, 16, KC, MT, MODE>(a, 8, s); break;
      case 5: st = launch<1, 12, KC, MT, MODE>(a, 8, s); break;
      case 6: st = launch<1, 8, KC, MT, MODE, 2>(a, 4, s); break;
      case 7: st = launch<2, 8, KC, MT, MODE>(a, 4, s); break;
      default:
        // measured at the Llama-3.1-8B gate_up shape: the pair kernel with 4
        // pairs in flight below m = 8 (m = 4: 14.5-14.8 against 15.1-15.9 us);
        // the K-slice kernel with two tiles' pairs in flight from m = 8 on,
        // where staging x per workgroup and reading it back from LDS per chunk
        // cost the most (m = 8: 15.2-15.3 against 15.4-15.6 us, m = 16:
        // 15.5-15.7 against 17.3-17.5, m = 32: 20.2 against 25.7)
        if (a.m >= 8) st = launch_kslice<4, 2, MT, MODE>(a, s);
        if (st == kNoFit)
          st = a.m <= 8 ? launch_pairs<4, MT, MODE>(a, s) : launch_pairs<2, MT, MODE>(a, s);
        break;
    }
    if (st == kNoFit) st = launch<1, 8, KC, MT, MODE, 2>(a, 8, s);
  }
  (void)cfg;
  // single-chunk slots, then shallower rings when x passes do not fit
  if (st == kNoFit) st = launch<1, 8, KC, MT, MODE>(a, 8, s);
  if (st == kNoFit) st = launch<1, 4, KC, MT, MODE>(a, 8, s);
  if (st == kNoFit) st = launch<1, 2, KC, MT, MODE>(a, 8, s);
  if (st == kNoFit)
    return fail(RLK_EUNSUPPORTED, "gemv_w4a16: k=%d does not fit the LDS budget", a.k);
  return st;
}

template <int MODE>
int dispatch(const W4Args& a, hipStream_t s) {
  const bool wide = a.group_size % 128 == 0;
  const int cfg = tune_knob(kW4Cfg, 0);
  if (a.m <= 16)
    return wide ? launch_cfg<128, 1, MODE>(a, cfg, s) : launch_cfg<32, 1, MODE>(a, cfg, s);
  return wide ? launch_cfg<128, 2, MODE>(a, cfg, s) : launch_cfg<32, 2, MODE>(a, cfg, s);
}

int gemv_w4(const char* what, const uint16_t* x, int m, const uint8_t* w, const uint16_t* scales,
            const uint16_t* offsets, int group_size, const uint16_t* bias, int n, int k, void* y,
            int mode, hipStream_t stream) {
  if (m <= 0) return RLK_OK;
  if (x == nullptr || w == nullptr || scales == nullptr || offsets == nullptr || y == nullptr)
    return fail(RLK_EINVAL, "%s: null pointer argument", what);
  if (m > RLK_GEMV_W4_MAX_M)
    return fail(RLK_EUNSUPPORTED, "%s: unsupported m=%d (at most %d)", what, m, RLK_GEMV_W4_MAX_M);
  if (n <= 0 || k <= 0 || group_size <= 0 || k % 32 != 0 || group_size % 32 != 0 ||
      k % group_size != 0)
    return fail(RLK_EINVAL, "%s needs K and group_size multiples of 32 (k=%d, group_size=%d)",
                what, k, group_size);
  if (k > (1 << 18))
    return fail(RLK_EUNSUPPORTED, "%s: k=%d exceeds %d", what, k, 1 << 18);
  if (mode == kModeSwiglu && n % 2 != 0)
    return fail(RLK_EINVAL, "%s: bad shape (n=%d must be even: interleaved gate/up rows)", what, n);
  if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || reinterpret_cast<uintptr_t>(w) % 16 != 0)
    return fail(RLK_EINVAL, "%s: x and w must be 16-byte aligned", what);
  W4Args a;
  a.x = x;
  a.w = w;
  a.scales = scales;
  a.offsets = offsets;
  a.bias = mode == kModeSwiglu ? nullptr : bias;
  a.y = y;
  a.m = m;
  a.n = n;
  a.k = k;
  a.group_size = group_size;
  a.groups = k / group_size;
  a.nchunks = k / (group_size % 128 == 0 ? 128 : 32);
  a.y_ld = mode == kModeSwiglu ? n / 2 : n;
  int st;
  switch (mode) {
    case kModeF32: st = dispatch<kModeF32>(a, stream); break;
    case kModeSwiglu: st = dispatch<kModeSwiglu>(a, stream); break;
    default: st = dispatch<kModeF16>(a, stream); break;
  }
  return st != RLK_OK ? st : launch_status(what);
}

// The INT8 K-slice kernel's launch: nw = k / 128 / CPW waves (at most 8), T
// tiles per workgroup -- about one workgroup per compute unit, fewer when
// their partials would not fit the LDS budget.
template <int CPW, int U, int MT, int MODE>
int launch_kslice_w8(W4Args a, hipStream_t stream) {
  if (a.n % 16 != 0 || a.k % (128 * CPW) != 0 || a.k / (128 * CPW) > kMaxWaves) return kNoFit;
  const int nw = a.k / (128 * CPW);
  const int ntiles = a.n / 16;
  const int cus = compute_units();
  auto lds_for = [&](int t) {  // the partial sums, which double as the x staging rows
    return std::max(static_cast<size_t>(t) * nw * MT * kWave * sizeof(f32x4),
                    static_cast<size_t>(nw) * 16 * 272);
  };
  int T = (ntiles + cus - 1) / cus;
  T = (T + U - 1) / U * U;
  while (T > U && lds_for(T) > kLdsBudget) T -= U;
  if (lds_for(T) > kLdsBudget) return kNoFit;
  a.cpp = T;
  const size_t lds = lds_for(T);
  auto kernel = gemv_w8_kslice_kernel<CPW, U, MT, MODE>;
  if (lds > 64 * 1024) {
    const hipError_t e = grant_dynamic_lds(reinterpret_cast<const void*>(kernel), kLdsBudget);
    if (e != hipSuccess)
      return fail(RLK_EUNSUPPORTED, "gemv_w8a16: %zu bytes of LDS refused (%s)", lds,
                  hipGetErrorString(e));
  }
  kernel<<<(ntiles + T - 1) / T, 64 * nw, lds, stream>>>(a);
  return RLK_OK;
}

// INT8 weight-only GEMV (gemv_weight_only.cu:64-93): the K-slice kernel with
// one tile's lines in flight where it fits (rows in whole tiles, K a multiple
// of 512 up to 4096: at the Llama-3.1-8B gate_up shape 23.2 / 23.4 / 23.6 /
// 26.4 us at m = 1 / 8 / 16 / 32 against 25.0 / 25.7 / 26.5 / 30.7 for the
// pair kernel, same run), else the pair kernel's INT8 form with P = 4 pairs
// in flight (equal to or faster than 2 and 8).  RLK_TUNE_W8_CFG = 1, 2, 3
// selects the pair kernel with P = 2, 4, 8, and 4, 5, 6 the K-slice kernel
// with (lines per slice, tiles in flight) = (4, 1), (4, 2), (2, 2).
template <int MT, int MODE>
int dispatch_w8(const W4Args& a, hipStream_t s) {
  int st = kNoFit;
  switch (tune_knob(kW8Cfg, 0)) {
    case 1: return launch_pairs<2, MT, MODE, true>(a, s);
    case 2: return launch_pairs<4, MT, MODE, true>(a, s);
    case 3: return launch_pairs<8, MT, MODE, true>(a, s);
    case 4: st = launch_kslice_w8<4, 1, MT, MODE>(a, s); break;
    case 5: st = launch_kslice_w8<4, 2, MT, MODE>(a, s); break;
    case 6: st = launch_kslice_w8<2, 2, MT, MODE>(a, s); break;
    default: st = launch_kslice_w8<4, 1, MT, MODE>(a, s); break;
  }
  if (st == kNoFit) st = launch_pairs<4, MT, MODE, true>(a, s);
  return st;
}

int gemv_w8(const uint16_t* x, int m, const int8_t* w, const uint16_t* scales, const uint16_t* bias,
            int n, int k, void* y, int y_fp32, hipStream_t stream) {
  const char* what = "gemv_w8a16";
  if (m <= 0) return RLK_OK;
  if (x == nullptr || w == nullptr || scales == nullptr || y == nullptr)
    return fail(RLK_EINVAL, "%s: null pointer argument", what);
  if (m > RLK_GEMV_W8_MAX_M)
    return fail(RLK_EUNSUPPORTED, "%s: unsupported m=%d (at most %d)", what, m, RLK_GEMV_W8_MAX_M);
  if (n <= 0 || k <= 0 || k % 16 != 0)
    return fail(RLK_EINVAL, "%s needs K %% 16 == 0, got %d (n=%d)", what, k, n);
  if (k > (1 << 20))
    return fail(RLK_EUNSUPPORTED, "%s: k=%d exceeds %d", what, k, 1 << 20);
  if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || reinterpret_cast<uintptr_t>(w) % 16 != 0)
    return fail(RLK_EINVAL, "%s: x and w must be 16-byte aligned", what);
  if (static_cast<uint64_t>(n) * static_cast<uint64_t>(k) > kMaxBufferBytes)
    return fail(RLK_EUNSUPPORTED, "%s: a weight of n*k = %llu bytes exceeds 2 GiB; split n", what,
                static_cast<unsigned long long>(n) * static_cast<unsigned long long>(k));
  W4Args a{};
  a.x = x;
  a.w = reinterpret_cast<const uint8_t*>(w);
  a.scales = scales;
  a.offsets = nullptr;
  a.bias = bias;
  a.y = y;
  a.m = m;
  a.n = n;
  a.k = k;
  a.group_size = 128;  // unused by the INT8 form
  a.groups = 0;
  a.nchunks = 2 * ((k + 127) / 128);  // 64-K chunks, a whole number of pairs
  a.y_ld = n;
  int st;
  if (y_fp32)
    st = m <= 16 ? dispatch_w8<1, kModeF32>(a, stream) : dispatch_w8<2, kModeF32>(a, stream);
  else
    st = m <= 16 ? dispatch_w8<1, kModeF16>(a, stream) : dispatch_w8<2, kModeF16>(a, stream);
  if (st == kNoFit) return fail(RLK_EUNSUPPORTED, "%s: m=%d does not fit the LDS budget", what, m);
  return st != RLK_OK ? st : launch_status(what);
}

}  // namespace
}  // namespace rlk

using namespace rlk;

extern "C" int rlk_gemv_w4a16(const uint16_t* x, int m, const uint8_t* w, const uint16_t* scales,
                              const uint16_t* offsets, int group_size, const uint16_t* bias, int n,
                              int k, void* y, int y_fp32, hipStream_t stream) {
  return gemv_w4("gemv_w4a16", x, m, w, scales, offsets, group_size, bias, n, k, y,
                 y_fp32 ? kModeF32 : kModeF16, stream);
}

extern "C" int rlk_gemv_w4a16_swiglu(const uint16_t* x, int m, const uint8_t* w,
                                     const uint16_t* scales, const uint16_t* offsets,
                                     int group_size, int n, int k, uint16_t* y,
                                     hipStream_t stream) {
  return gemv_w4("gemv_w4a16_swiglu", x, m, w, scales, offsets, group_size, nullptr, n, k, y,
                 kModeSwiglu, stream);
}

extern "C" int rlk_gemv_w8a16(const uint16_t* x, int m, const int8_t* w, const uint16_t* scales,
                              const uint16_t* bias, int n, int k, void* y, int y_fp32,
                              hipStream_t stream) {
  return gemv_w8(x, m, w, scales, bias, n, k, y, y_fp32, stream);
}
