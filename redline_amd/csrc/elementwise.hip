// Row-streaming kernels for gfx950: embedding gather / row gather, fused
// residual-add + RMSNorm, SwiGLU (split and interleaved), input-id resolve.
//
// All of them are HBM-bound (a few flops per byte).  What sets their speed on
// MI355X is how many 16-byte accesses are in flight and how the memory system
// treats them, so every kernel is templated on
//   BS  lanes per workgroup (64 = one wave64: the most workgroups, which
//       spreads a launch evenly over the 256 CUs / 8 XCDs),
//   NT  non-temporal (streaming) loads/stores, which measured faster than
//       cached accesses at every launch size from decode b32 to 16k rows,
// and the launch policy (`pick_flat`, the norm/rope launchers) chooses them.
// Numerics follow the reference kernels' fp16 rounding points
// (src/cuda/kernels/elementwise.cu:29-82,123-131 in Neil456/Redline).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "device.hpp"
#include "redline_amd/rlk.h"
#include "status.hpp"

namespace rlk {
namespace {

struct FlatPolicy {
  int bs;   // lanes per workgroup: 64, 128 or 256
  bool nt;  // non-temporal accesses
};

// Launch policy of the flat streaming kernels (measured on MI355X with cold,
// rotating buffers at decode b32 and 4k-16k-row prefill shapes): non-temporal
// accesses were faster at every size, by 8-20%; the best block width depends
// weakly on the launch size.  The RLK_TUNE_<NAME>_BS / _NT knobs (status.hpp)
// override it for tuning runs.
FlatPolicy pick_flat(int bs, Knob bs_knob, Knob nt_knob) {
  FlatPolicy p;
  p.bs = tune_knob(bs_knob, bs);
  p.nt = tune_knob(nt_knob, 1) != 0;
  return p;
}

// The flat kernels index the [rows, vecs] space of 16-byte vectors: lane l of
// block b handles vector b * BS + l, so every wave access is 1 KiB
// contiguous (except at row ends) and no lane idles when a row is not a
// multiple of the block width.

// ------------------------------------------------------------------ gathers

// dst[r, :] = src[idx ? idx[r] : r, :] for rows of `vecs` 16-byte vectors.
template <int BS, bool NT>
__global__ __launch_bounds__(BS) void gather_rows_kernel(const int32_t* __restrict__ idx,
                                                         const u32x4* __restrict__ src,
                                                         uint32_t vecs, uint32_t total,
                                                         u32x4* __restrict__ dst) {
  const uint32_t g = blockIdx.x * BS + threadIdx.x;
  if (g >= total) return;
  const uint32_t row = g / vecs;
  const uint32_t col = g - row * vecs;
  const uint64_t srow = idx != nullptr ? static_cast<uint32_t>(idx[row]) : row;
  st16<NT>(dst + g, ld16<NT>(src + srow * vecs + col));
}

template <int BS>
void launch_gather_bs(bool nt, uint64_t total, const int32_t* idx, const u32x4* s,
                      uint32_t vecs, u32x4* d, hipStream_t stream) {
  const uint32_t t32 = static_cast<uint32_t>(total);
  const uint64_t blocks = (total + BS - 1) / BS;
  if (nt) {
    gather_rows_kernel<BS, true><<<blocks, BS, 0, stream>>>(idx, s, vecs, t32, d);
  } else {
    gather_rows_kernel<BS, false><<<blocks, BS, 0, stream>>>(idx, s, vecs, t32, d);
  }
}

int launch_gather(const int32_t* idx, const void* src, int n, int vecs, void* dst,
                  hipStream_t stream, const char* what) {
  const uint64_t total = static_cast<uint64_t>(n) * vecs;
  if (total > 0x7fffffffull)
    return fail(RLK_EINVAL, "%s: %d rows x %d vectors exceed one launch; split the call", what, n,
                vecs);
  const FlatPolicy p = pick_flat(total >= (1u << 20) ? 256 : 128, kGatherBs, kGatherNt);
  const auto* s = static_cast<const u32x4*>(src);
  auto* d = static_cast<u32x4*>(dst);
  switch (p.bs) {
    case 128: launch_gather_bs<128>(p.nt, total, idx, s, vecs, d, stream); break;
    case 256: launch_gather_bs<256>(p.nt, total, idx, s, vecs, d, stream); break;
    default: launch_gather_bs<64>(p.nt, total, idx, s, vecs, d, stream); break;
  }
  return launch_status(what);
}

// ----------------------------------------------------------- add + RMSNorm

// One workgroup of TPR lanes owns one row, held in registers (NV vectors of 8
// halves per lane): the residual is read once, the sum of squares is a wave64
// butterfly plus one LDS exchange when TPR > 64, and the output pass needs no
// re-read.  Rounding points follow elementwise.cu:45,52,61: the residual sum
// is rounded to fp16, the sum of squares is fp32, x * inv is rounded to fp16
// before the fp16 weight multiply.
// Where the row comes from: the residual in place (kNoDelta), the residual
// plus delta written back (kDelta), or an embedding-table row table[ids[row]]
// written to the residual (kGather: embedding_lookup followed by
// fused_add_rmsnorm with delta == nullptr, in one pass).
enum NormSrc { kNoDelta = 0, kDelta = 1, kGather = 2 };

template <int TPR, int NV, int kSrc, bool NT>
__global__ __launch_bounds__(TPR) void add_rmsnorm_kernel(
    u32x4* __restrict__ residual, const u32x4* __restrict__ delta,
    const u32x4* __restrict__ weight, int vecs, float hidden, float eps,
    u32x4* __restrict__ out, const int32_t* __restrict__ ids) {
  constexpr int kWaves = TPR / kWave;
  __shared__ float partial[kWaves];
  const int lt = threadIdx.x;
  const int64_t row = blockIdx.x;
  u32x4* res = residual + row * vecs;
  // kGather: `delta` is the embedding table
  const u32x4* src =
      kSrc == kGather ? delta + static_cast<int64_t>(static_cast<uint32_t>(ids[row])) * vecs : res;

  u32x4 rv[NV], dv[NV], wv[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int i = lt + k * TPR;
    const bool ok = i < vecs;
    rv[k] = ok ? ld16<NT>(src + i) : u32x4{0, 0, 0, 0};
    if constexpr (kSrc == kDelta) dv[k] = ok ? ld16<NT>(delta + row * vecs + i) : u32x4{0, 0, 0, 0};
    wv[k] = ok ? weight[i] : u32x4{0, 0, 0, 0};  // shared by all rows: cached load, issued early
  }
  f32x8 x[NV];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    x[k] = unpack8(rv[k]);
    const int i = lt + k * TPR;
    if constexpr (kSrc == kDelta) {
      x[k] = round_f16(x[k] + unpack8(dv[k]));
      if (i < vecs) st16<NT>(res + i, pack8(x[k]));
    } else if constexpr (kSrc == kGather) {
      if (i < vecs) st16<NT>(res + i, rv[k]);  // the gathered row, bit for bit
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) ss += x[k][j] * x[k][j];
  }
  ss = wave_sum(ss);
  if constexpr (kWaves > 1) {
    if (lt % kWave == 0) partial[lt / kWave] = ss;
    __syncthreads();
    ss = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) ss += partial[w];
  }
  const float inv = 1.0f / __builtin_sqrtf(ss / hidden + eps);
  u32x4* o = out + row * vecs;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int i = lt + k * TPR;
    if (i < vecs) st16<NT>(o + i, pack8(round_f16(x[k] * inv) * unpack8(wv[k])));
  }
}

// Rows wider than the register-resident variants cover: one block per row,
// two passes (the second re-reads the residual from cache).
template <int kSrc>
__global__ __launch_bounds__(256) void add_rmsnorm_wide_kernel(
    u32x4* __restrict__ residual, const u32x4* __restrict__ delta,
    const u32x4* __restrict__ weight, int vecs, float hidden, float eps,
    u32x4* __restrict__ out, const int32_t* __restrict__ ids) {
  __shared__ float partial[256 / kWave];
  const int64_t row = blockIdx.x;
  u32x4* res = residual + row * vecs;
  const u32x4* src =
      kSrc == kGather ? delta + static_cast<int64_t>(static_cast<uint32_t>(ids[row])) * vecs : res;
  float ss = 0.f;
  for (int i = threadIdx.x; i < vecs; i += 256) {
    const u32x4 r = src[i];
    f32x8 x = unpack8(r);
    if constexpr (kSrc == kDelta) {
      x = round_f16(x + unpack8(delta[row * vecs + i]));
      res[i] = pack8(x);
    } else if constexpr (kSrc == kGather) {
      res[i] = r;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) ss += x[j] * x[j];
  }
  ss = wave_sum(ss);
  if (threadIdx.x % kWave == 0) partial[threadIdx.x / kWave] = ss;
  __syncthreads();
  ss = 0.f;
#pragma unroll
  for (int w = 0; w < 256 / kWave; ++w) ss += partial[w];
  const float inv = 1.0f / __builtin_sqrtf(ss / hidden + eps);
  u32x4* o = out + row * vecs;
  for (int i = threadIdx.x; i < vecs; i += 256)
    o[i] = pack8(round_f16(unpack8(res[i]) * inv) * unpack8(weight[i]));
}

struct NormArgs {
  u32x4* res;
  const u32x4* del;  // delta, or the embedding table (ids != nullptr)
  const u32x4* w;
  int rows, vecs;
  float hidden, eps;
  u32x4* out;
  const int32_t* ids;  // non-null: gather the rows from the table
};

int norm_src(const NormArgs& a) {
  return a.ids != nullptr ? kGather : (a.del != nullptr ? kDelta : kNoDelta);
}

template <int TPR, int NV, bool NT>
void launch_norm_tn(const NormArgs& a, hipStream_t stream) {
#define RLK_NORM_LAUNCH(S)                                                                       \
  add_rmsnorm_kernel<TPR, NV, S, NT>                                                             \
      <<<a.rows, TPR, 0, stream>>>(a.res, a.del, a.w, a.vecs, a.hidden, a.eps, a.out, a.ids)
  switch (norm_src(a)) {
    case kDelta: RLK_NORM_LAUNCH(kDelta); break;
    case kGather: RLK_NORM_LAUNCH(kGather); break;
    default: RLK_NORM_LAUNCH(kNoDelta); break;
  }
#undef RLK_NORM_LAUNCH
}

// Register-resident variants: NV vectors (8 halves each) per lane.
template <int TPR, bool NT>
bool launch_norm_t(int nv, const NormArgs& a, hipStream_t stream) {
#define RLK_NORM_CASE(N)                     \
  case N:                                    \
    launch_norm_tn<TPR, N, NT>(a, stream);   \
    return true;
  switch (nv) {
    RLK_NORM_CASE(1)
    RLK_NORM_CASE(2)
    RLK_NORM_CASE(3)
    RLK_NORM_CASE(4)
    RLK_NORM_CASE(5)
    RLK_NORM_CASE(6)
    RLK_NORM_CASE(7)
    RLK_NORM_CASE(8)
    RLK_NORM_CASE(12)
    RLK_NORM_CASE(16)
    default: return false;
  }
#undef RLK_NORM_CASE
}

int round_up_nv(int nv) {
  if (nv <= 8) return nv;
  if (nv <= 12) return 12;
  return nv <= 16 ? 16 : -1;
}

template <bool NT>
bool launch_norm_nt(int tpr, const NormArgs& a, hipStream_t stream) {
  const int nv = round_up_nv((a.vecs + tpr - 1) / tpr);
  if (nv < 0) return false;
  switch (tpr) {
    case 64: return launch_norm_t<64, NT>(nv, a, stream);
    case 128: return launch_norm_t<128, NT>(nv, a, stream);
    case 512: return launch_norm_t<512, NT>(nv, a, stream);
    default: return launch_norm_t<256, NT>(nv, a, stream);
  }
}

// Lanes per row: enough for one 16-byte vector per lane up to 512 lanes
// (eight waves); wider rows keep several vectors per lane in registers, and
// rows past 512 x 16 vectors take the two-pass kernel.  Non-temporal accesses
// measured faster at every batch size.
void launch_norm(const NormArgs& a, hipStream_t stream) {
  int tpr = 64;
  while (tpr < 512 && tpr < a.vecs) tpr *= 2;
  tpr = tune_knob(kNormTpr, tpr);
  const bool nt = tune_knob(kNormNt, 1) != 0;
  bool launched = nt ? launch_norm_nt<true>(tpr, a, stream) : launch_norm_nt<false>(tpr, a, stream);
  if (!launched) launched = launch_norm_nt<false>(512, a, stream);
  if (launched) return;
#define RLK_NORM_WIDE(S)                                                                   \
  add_rmsnorm_wide_kernel<S><<<a.rows, 256, 0, stream>>>(a.res, a.del, a.w, a.vecs, a.hidden, \
                                                         a.eps, a.out, a.ids)
  switch (norm_src(a)) {
    case kDelta: RLK_NORM_WIDE(kDelta); break;
    case kGather: RLK_NORM_WIDE(kGather); break;
    default: RLK_NORM_WIDE(kNoDelta); break;
  }
#undef RLK_NORM_WIDE
}

// ------------------------------------------------------------------ SwiGLU

// Split layout: gate in [r, 0:I], up in [r, I:2I]; flat over the [rows, vecs]
// output vectors (vecs = I / 8).
template <int BS, bool NT>
__global__ __launch_bounds__(BS) void silu_and_mul_kernel(const u32x4* __restrict__ gate_up,
                                                          uint32_t vecs, uint32_t total,
                                                          u32x4* __restrict__ out) {
  const uint32_t g = blockIdx.x * BS + threadIdx.x;
  if (g >= total) return;
  const uint32_t row = g / vecs;
  const uint64_t at = static_cast<uint64_t>(g) + static_cast<uint64_t>(row) * vecs;
  const u32x4 gv = ld16<NT>(gate_up + at);
  const u32x4 uv = ld16<NT>(gate_up + at + vecs);
  const f32x8 gf = unpack8(gv);
  f32x8 s;
#pragma unroll
  for (int j = 0; j < 8; ++j) s[j] = silu_f16(gf[j]);
  st16<NT>(out + g, pack8(s * unpack8(uv)));
}

// Interleaved layout (gate_i, up_i): output vector g (8 outputs) reads input
// vectors 2g and 2g + 1.  Needs inter % 8 == 0.
template <int BS, bool NT>
__global__ __launch_bounds__(BS) void silu_and_mul_interleaved_kernel(
    const u32x4* __restrict__ gate_up, uint32_t total, u32x4* __restrict__ out) {
  const uint32_t g = blockIdx.x * BS + threadIdx.x;
  if (g >= total) return;
  const f32x8 lo = unpack8(ld16<NT>(gate_up + 2 * static_cast<uint64_t>(g)));
  const f32x8 hi = unpack8(ld16<NT>(gate_up + 2 * static_cast<uint64_t>(g) + 1));
  f32x8 y;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    y[j] = silu_f16(lo[2 * j]) * lo[2 * j + 1];
    y[4 + j] = silu_f16(hi[2 * j]) * hi[2 * j + 1];
  }
  st16<NT>(out + g, pack8(y));
}

// Any inter: one output per lane from a 4-byte (gate, up) pair.
__global__ __launch_bounds__(256) void silu_and_mul_interleaved_scalar_kernel(
    const f16x2* __restrict__ gate_up, int64_t total, _Float16* __restrict__ out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= total) return;
  const f16x2 p = gate_up[i];  // pairs are row-major [rows, inter]: same flat index
  out[i] = static_cast<_Float16>(silu_f16(static_cast<float>(p[0])) * static_cast<float>(p[1]));
}

template <int BS, bool NT>
void launch_swiglu_bs(bool interleaved, uint64_t blocks, const u32x4* gu, uint32_t vecs,
                      uint32_t total, u32x4* o, hipStream_t stream) {
  if (interleaved) {
    silu_and_mul_interleaved_kernel<BS, NT><<<blocks, BS, 0, stream>>>(gu, total, o);
  } else {
    silu_and_mul_kernel<BS, NT><<<blocks, BS, 0, stream>>>(gu, vecs, total, o);
  }
}

void launch_swiglu(bool interleaved, const u32x4* gu, uint32_t vecs, uint32_t total, u32x4* o,
                   hipStream_t stream) {
  const FlatPolicy p = pick_flat(64, kSwigluBs, kSwigluNt);
  const uint64_t blocks = (total + p.bs - 1) / p.bs;
#define RLK_SWIGLU_BS(B)                                                               \
  p.nt ? launch_swiglu_bs<B, true>(interleaved, blocks, gu, vecs, total, o, stream)    \
       : launch_swiglu_bs<B, false>(interleaved, blocks, gu, vecs, total, o, stream)
  switch (p.bs) {
    case 128: RLK_SWIGLU_BS(128); break;
    case 256: RLK_SWIGLU_BS(256); break;
    default: RLK_SWIGLU_BS(64); break;
  }
#undef RLK_SWIGLU_BS
}

__global__ __launch_bounds__(256) void resolve_input_ids_kernel(
    int32_t* __restrict__ ids, const int32_t* __restrict__ src,
    const int32_t* __restrict__ prev_sampled, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) {
    const int s = src[i];
    if (s >= 0) ids[i] = prev_sampled[s];
  }
}

}  // namespace
}  // namespace rlk

using namespace rlk;

extern "C" int rlk_embedding_lookup(const int32_t* ids, const uint16_t* table, int n, int hidden,
                                    uint16_t* out, hipStream_t stream) {
  if (n <= 0) return RLK_OK;
  if (hidden <= 0 || hidden % 8 != 0)
    return fail(RLK_EINVAL, "embedding_lookup: hidden size must be a multiple of 8 (got %d)", hidden);
  if (ids == nullptr || table == nullptr || out == nullptr)
    return fail(RLK_EINVAL, "embedding_lookup: null pointer argument");
  return launch_gather(ids, table, n, hidden / 8, out, stream, "embedding_lookup");
}

extern "C" int rlk_gather_rows(const uint16_t* src, const int32_t* idx, int n, int cols,
                               uint16_t* dst, hipStream_t stream) {
  if (n <= 0) return RLK_OK;
  if (cols <= 0 || cols % 8 != 0)
    return fail(RLK_EINVAL, "gather_rows: row width must be a multiple of 8 (got %d)", cols);
  if (src == nullptr || dst == nullptr) return fail(RLK_EINVAL, "gather_rows: null pointer argument");
  return launch_gather(idx, src, n, cols / 8, dst, stream, "gather_rows");
}

extern "C" int rlk_fused_add_rmsnorm(uint16_t* residual, const uint16_t* delta,
                                     const uint16_t* weight, int rows, int hidden, float eps,
                                     uint16_t* out, hipStream_t stream) {
  if (rows <= 0) return RLK_OK;
  if (hidden <= 0 || hidden % 8 != 0)
    return fail(RLK_EINVAL, "fused_add_rmsnorm: hidden size must be a multiple of 8 (got %d)",
                hidden);
  if (residual == nullptr || weight == nullptr || out == nullptr)
    return fail(RLK_EINVAL, "fused_add_rmsnorm: null pointer argument");
  NormArgs a;
  a.res = reinterpret_cast<u32x4*>(residual);
  a.del = reinterpret_cast<const u32x4*>(delta);
  a.w = reinterpret_cast<const u32x4*>(weight);
  a.rows = rows;
  a.vecs = hidden / 8;
  a.hidden = static_cast<float>(hidden);
  a.eps = eps;
  a.out = reinterpret_cast<u32x4*>(out);
  a.ids = nullptr;
  launch_norm(a, stream);
  return launch_status("fused_add_rmsnorm");
}

extern "C" int rlk_embedding_rmsnorm(const int32_t* ids, const uint16_t* table, int n, int hidden,
                                     const uint16_t* weight, float eps, uint16_t* residual,
                                     uint16_t* out, hipStream_t stream) {
  if (n <= 0) return RLK_OK;
  if (hidden <= 0 || hidden % 8 != 0)
    return fail(RLK_EINVAL, "embedding_rmsnorm: hidden size must be a multiple of 8 (got %d)",
                hidden);
  if (ids == nullptr || table == nullptr || weight == nullptr || residual == nullptr ||
      out == nullptr)
    return fail(RLK_EINVAL, "embedding_rmsnorm: null pointer argument");
  if (((reinterpret_cast<uintptr_t>(table) | reinterpret_cast<uintptr_t>(weight) |
        reinterpret_cast<uintptr_t>(residual) | reinterpret_cast<uintptr_t>(out)) & 15) != 0)
    return fail(RLK_EINVAL, "embedding_rmsnorm: table, weight, residual and out must be 16-byte aligned");
  NormArgs a;
  a.res = reinterpret_cast<u32x4*>(residual);
  a.del = reinterpret_cast<const u32x4*>(table);
  a.w = reinterpret_cast<const u32x4*>(weight);
  a.rows = n;
  a.vecs = hidden / 8;
  a.hidden = static_cast<float>(hidden);
  a.eps = eps;
  a.out = reinterpret_cast<u32x4*>(out);
  a.ids = ids;
  launch_norm(a, stream);
  return launch_status("embedding_rmsnorm");
}

extern "C" int rlk_silu_and_mul(const uint16_t* gate_up, int rows, int inter, uint16_t* out,
                                hipStream_t stream) {
  if (rows <= 0) return RLK_OK;
  if (inter <= 0 || inter % 8 != 0)
    return fail(RLK_EINVAL, "silu_and_mul: intermediate size must be a multiple of 8 (got %d)",
                inter);
  if (gate_up == nullptr || out == nullptr) return fail(RLK_EINVAL, "silu_and_mul: null pointer argument");
  const uint32_t vecs = inter / 8;
  const uint64_t total = static_cast<uint64_t>(rows) * vecs;
  if (total > 0x7fffffffull)
    return fail(RLK_EINVAL, "silu_and_mul: %d rows exceed one launch; split the call", rows);
  launch_swiglu(false, reinterpret_cast<const u32x4*>(gate_up), vecs,
                static_cast<uint32_t>(total), reinterpret_cast<u32x4*>(out), stream);
  return launch_status("silu_and_mul");
}

extern "C" int rlk_silu_and_mul_interleaved(const uint16_t* gate_up, int rows, int inter,
                                            uint16_t* out, hipStream_t stream) {
  if (rows <= 0) return RLK_OK;
  if (inter <= 0) return fail(RLK_EINVAL, "silu_and_mul_interleaved: bad intermediate size %d", inter);
  if (gate_up == nullptr || out == nullptr)
    return fail(RLK_EINVAL, "silu_and_mul_interleaved: null pointer argument");
  const uint64_t pairs = static_cast<uint64_t>(rows) * inter;
  if (pairs > 0x7fffffffull)
    return fail(RLK_EINVAL, "silu_and_mul_interleaved: %d rows exceed one launch; split the call",
                rows);
  if (inter % 8 == 0) {
    launch_swiglu(true, reinterpret_cast<const u32x4*>(gate_up), inter / 8,
                  static_cast<uint32_t>(pairs / 8), reinterpret_cast<u32x4*>(out), stream);
  } else {
    const uint64_t blocks = (pairs + 255) / 256;
    silu_and_mul_interleaved_scalar_kernel<<<blocks, 256, 0, stream>>>(
        reinterpret_cast<const f16x2*>(gate_up), static_cast<int64_t>(pairs),
        reinterpret_cast<_Float16*>(out));
  }
  return launch_status("silu_and_mul_interleaved");
}

extern "C" int rlk_resolve_input_ids(int32_t* input_ids, const int32_t* src,
                                     const int32_t* prev_sampled, int n, hipStream_t stream) {
  if (n <= 0) return RLK_OK;
  // prev_sampled is read only where src >= 0, so a batch without such rows may pass null
  if (input_ids == nullptr || src == nullptr)
    return fail(RLK_EINVAL, "resolve_input_ids: null pointer argument");
  resolve_input_ids_kernel<<<(n + 255) / 256, 256, 0, stream>>>(input_ids, src, prev_sampled, n);
  return launch_status("resolve_input_ids");
}
