// Row-streaming kernels for gfx950: embedding gather / row gather, fused
// residual-add + RMSNorm, SwiGLU (split and interleaved), input-id resolve.
//
// All of them are HBM-bound (a few flops per byte), so the design goal is to
// keep enough 128-bit loads in flight per CU: every lane issues its NV
// 16-byte loads before it consumes any of them, workgroups are 256 lanes (four
// wave64s), and the grid is sized so that small batches still spread over many
// CUs.  Numerics follow the reference kernels' fp16 rounding points
// (src/cuda/kernels/elementwise.cu:29-82,123-131 in Neil456/Redline).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "device.hpp"
#include "redline_amd/rlk.h"
#include "status.hpp"

namespace rlk {
namespace {

constexpr int kThreads = 256;

// ------------------------------------------------------------------ gathers

// dst[r, :] = src[idx ? idx[r] : r, :] for rows of `vecs` 16-byte vectors.
// Block b copies chunk (b % chunks) of row (b / chunks); a chunk is
// kThreads * NV vectors, each lane loading its NV vectors before storing.
template <int NV>
__global__ __launch_bounds__(kThreads) void gather_rows_kernel(const int32_t* __restrict__ idx,
                                                               const u32x4* __restrict__ src,
                                                               int vecs, int chunks,
                                                               u32x4* __restrict__ dst) {
  const int64_t row = blockIdx.x / chunks;
  const int chunk = blockIdx.x - static_cast<int>(row) * chunks;
  const int64_t src_row = idx != nullptr ? idx[row] : row;
  const u32x4* s = src + src_row * vecs;
  u32x4* d = dst + row * vecs;
  const int base = chunk * kThreads * NV + threadIdx.x;
  u32x4 v[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int i = base + k * kThreads;
    if (i < vecs) v[k] = s[i];
  }
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int i = base + k * kThreads;
    if (i < vecs) d[i] = v[k];
  }
}

// Vectors per lane for a row-chunked launch: the largest NV in {1, 2, 4} that
// still leaves at least `min_blocks` workgroups (small batches favour more,
// smaller blocks; large ones favour more bytes in flight per lane).
int pick_nv(int64_t rows, int vecs, int64_t min_blocks) {
  int nv = 4;
  while (nv > 1) {
    const int64_t chunks = (vecs + kThreads * nv - 1) / (kThreads * nv);
    if (rows * chunks >= min_blocks) break;
    nv >>= 1;
  }
  return nv;
}

int launch_gather(const int32_t* idx, const void* src, int n, int vecs, void* dst,
                  hipStream_t stream, const char* what) {
  const int nv = tune_knob("RLK_TUNE_GATHER_NV", pick_nv(n, vecs, 2048));
  const int chunks = (vecs + kThreads * nv - 1) / (kThreads * nv);
  const int64_t blocks = static_cast<int64_t>(n) * chunks;
  if (blocks > 0x7fffffff) return fail(RLK_EINVAL, "%s: too many rows (%d)", what, n);
  const auto* s = static_cast<const u32x4*>(src);
  auto* d = static_cast<u32x4*>(dst);
  switch (nv) {
    case 1: gather_rows_kernel<1><<<blocks, kThreads, 0, stream>>>(idx, s, vecs, chunks, d); break;
    case 2: gather_rows_kernel<2><<<blocks, kThreads, 0, stream>>>(idx, s, vecs, chunks, d); break;
    default: gather_rows_kernel<4><<<blocks, kThreads, 0, stream>>>(idx, s, vecs, chunks, d); break;
  }
  return launch_status(what);
}

// ----------------------------------------------------------- add + RMSNorm

// TPR lanes own one row; the row lives in registers (NV vectors per lane), so
// the residual is read once, the sum of squares is a wave64 butterfly (plus a
// tiny LDS exchange when TPR > 64), and the output pass needs no re-read.
// Rounding points follow elementwise.cu:45,52,61: the residual sum is rounded
// to fp16, the sum of squares is fp32, x * inv is rounded to fp16 before the
// fp16 weight multiply.
template <int TPR, int NV, bool kDelta>
__global__ __launch_bounds__(kThreads) void add_rmsnorm_kernel(
    u32x4* __restrict__ residual, const u32x4* __restrict__ delta,
    const u32x4* __restrict__ weight, int rows, int vecs, float hidden, float eps,
    u32x4* __restrict__ out) {
  constexpr int kRowsPerBlock = kThreads / TPR;
  constexpr int kWavesPerRow = TPR / kWave;
  __shared__ float partial[kThreads / kWave];
  const int lt = threadIdx.x % TPR;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + threadIdx.x / TPR;
  const bool active = row < rows;
  u32x4* res = residual + row * vecs;

  u32x4 rv[NV], dv[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int i = lt + k * TPR;
    const bool ok = active && i < vecs;
    rv[k] = ok ? res[i] : u32x4{0, 0, 0, 0};
    if constexpr (kDelta) dv[k] = ok ? delta[row * vecs + i] : u32x4{0, 0, 0, 0};
  }
  f32x8 x[NV];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    x[k] = unpack8(rv[k]);
    if constexpr (kDelta) {
      x[k] = round_f16(x[k] + unpack8(dv[k]));
      const int i = lt + k * TPR;
      if (active && i < vecs) res[i] = pack8(x[k]);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) ss += x[k][j] * x[k][j];
  }
  ss = wave_sum(ss);
  if constexpr (kWavesPerRow > 1) {
    const int wave = threadIdx.x / kWave;
    if (threadIdx.x % kWave == 0) partial[wave] = ss;
    __syncthreads();
    const int first = (threadIdx.x / TPR) * kWavesPerRow;
    ss = 0.f;
#pragma unroll
    for (int w = 0; w < kWavesPerRow; ++w) ss += partial[first + w];
  }
  const float inv = 1.0f / __builtin_sqrtf(ss / hidden + eps);
  if (!active) return;
  u32x4* o = out + row * vecs;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int i = lt + k * TPR;
    if (i < vecs) o[i] = pack8(round_f16(x[k] * inv) * unpack8(weight[i]));
  }
}

// Rows wider than the register-resident variants cover: one block per row,
// two passes (the second re-reads the residual from cache).
template <bool kDelta>
__global__ __launch_bounds__(kThreads) void add_rmsnorm_wide_kernel(
    u32x4* __restrict__ residual, const u32x4* __restrict__ delta,
    const u32x4* __restrict__ weight, int vecs, float hidden, float eps,
    u32x4* __restrict__ out) {
  __shared__ float partial[kThreads / kWave];
  const int64_t row = blockIdx.x;
  u32x4* res = residual + row * vecs;
  float ss = 0.f;
  for (int i = threadIdx.x; i < vecs; i += kThreads) {
    f32x8 x = unpack8(res[i]);
    if constexpr (kDelta) {
      x = round_f16(x + unpack8(delta[row * vecs + i]));
      res[i] = pack8(x);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) ss += x[j] * x[j];
  }
  ss = wave_sum(ss);
  if (threadIdx.x % kWave == 0) partial[threadIdx.x / kWave] = ss;
  __syncthreads();
  ss = 0.f;
#pragma unroll
  for (int w = 0; w < kThreads / kWave; ++w) ss += partial[w];
  const float inv = 1.0f / __builtin_sqrtf(ss / hidden + eps);
  u32x4* o = out + row * vecs;
  for (int i = threadIdx.x; i < vecs; i += kThreads)
    o[i] = pack8(round_f16(unpack8(res[i]) * inv) * unpack8(weight[i]));
}

template <int TPR, int NV>
void launch_norm_tn(u32x4* res, const u32x4* del, const u32x4* w, int rows, int vecs,
                    float hidden_f, float eps, u32x4* out, hipStream_t stream) {
  constexpr int rpb = kThreads / TPR;
  const int blocks = (rows + rpb - 1) / rpb;
  if (del != nullptr) {
    add_rmsnorm_kernel<TPR, NV, true>
        <<<blocks, kThreads, 0, stream>>>(res, del, w, rows, vecs, hidden_f, eps, out);
  } else {
    add_rmsnorm_kernel<TPR, NV, false>
        <<<blocks, kThreads, 0, stream>>>(res, del, w, rows, vecs, hidden_f, eps, out);
  }
}

// Register-resident variants: NV vectors (8 halves each) per lane.
template <int TPR>
bool launch_norm_t(int nv, u32x4* res, const u32x4* del, const u32x4* w, int rows, int vecs,
                   float hidden_f, float eps, u32x4* out, hipStream_t stream) {
#define RLK_NORM_CASE(N)                                                                    \
  case N:                                                                                   \
    launch_norm_tn<TPR, N>(res, del, w, rows, vecs, hidden_f, eps, out, stream);          \
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

// ------------------------------------------------------------------ SwiGLU

// silu(g) rounded to fp16 (elementwise.cu:77), then times up.  exp and the
// division use the hardware's fast exp2 / reciprocal: the result is rounded
// to fp16 right after, far coarser than their error.
__device__ __forceinline__ float silu_f16(float g) {
  return round_f16(__fdividef(g, 1.0f + __expf(-g)));
}

// Split layout: gate in [r, 0:I], up in [r, I:2I].  Block b handles chunk
// (b % chunks) of row (b / chunks), kThreads * NV output vectors per chunk.
template <int NV>
__global__ __launch_bounds__(kThreads) void silu_and_mul_kernel(const u32x4* __restrict__ gate_up,
                                                                int vecs, int chunks,
                                                                u32x4* __restrict__ out) {
  const int64_t row = blockIdx.x / chunks;
  const int chunk = blockIdx.x - static_cast<int>(row) * chunks;
  const u32x4* g = gate_up + row * 2 * vecs;
  const u32x4* u = g + vecs;
  u32x4* o = out + row * vecs;
  const int base = chunk * kThreads * NV + threadIdx.x;
  u32x4 gv[NV], uv[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int i = base + k * kThreads;
    if (i < vecs) {
      gv[k] = g[i];
      uv[k] = u[i];
    }
  }
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int i = base + k * kThreads;
    if (i < vecs) {
      const f32x8 gf = unpack8(gv[k]);
      f32x8 s;
#pragma unroll
      for (int j = 0; j < 8; ++j) s[j] = silu_f16(gf[j]);
      o[i] = pack8(s * unpack8(uv[k]));
    }
  }
}

// Interleaved layout (gate_i, up_i): each lane reads two 16-byte vectors (8
// pairs) and writes one 16-byte vector of 8 outputs.  Needs inter % 8 == 0.
template <int NV>
__global__ __launch_bounds__(kThreads) void silu_and_mul_interleaved_kernel(
    const u32x4* __restrict__ gate_up, int vecs, int chunks, u32x4* __restrict__ out) {
  const int64_t row = blockIdx.x / chunks;
  const int chunk = blockIdx.x - static_cast<int>(row) * chunks;
  const u32x4* gu = gate_up + row * 2 * vecs;
  u32x4* o = out + row * vecs;
  const int base = chunk * kThreads * NV + threadIdx.x;
  u32x4 a[NV], b[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int i = base + k * kThreads;
    if (i < vecs) {
      a[k] = gu[2 * i];
      b[k] = gu[2 * i + 1];
    }
  }
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int i = base + k * kThreads;
    if (i < vecs) {
      const f32x8 lo = unpack8(a[k]), hi = unpack8(b[k]);
      f32x8 y;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        y[j] = silu_f16(lo[2 * j]) * lo[2 * j + 1];
        y[4 + j] = silu_f16(hi[2 * j]) * hi[2 * j + 1];
      }
      o[i] = pack8(y);
    }
  }
}

// Any inter: one output per lane from a 4-byte (gate, up) pair.
__global__ __launch_bounds__(kThreads) void silu_and_mul_interleaved_scalar_kernel(
    const f16x2* __restrict__ gate_up, int64_t total, _Float16* __restrict__ out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= total) return;
  const f16x2 p = gate_up[i];  // row-major [rows, inter] pairs: same flat index
  out[i] = static_cast<_Float16>(silu_f16(static_cast<float>(p[0])) * static_cast<float>(p[1]));
}

__global__ __launch_bounds__(kThreads) void resolve_input_ids_kernel(
    int32_t* __restrict__ ids, const int32_t* __restrict__ src,
    const int32_t* __restrict__ prev_sampled, int n) {
  const int i = blockIdx.x * kThreads + threadIdx.x;
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
  return launch_gather(ids, table, n, hidden / 8, out, stream, "embedding_lookup");
}

extern "C" int rlk_gather_rows(const uint16_t* src, const int32_t* idx, int n, int cols,
                               uint16_t* dst, hipStream_t stream) {
  if (n <= 0) return RLK_OK;
  if (cols <= 0 || cols % 8 != 0)
    return fail(RLK_EINVAL, "gather_rows: row width must be a multiple of 8 (got %d)", cols);
  return launch_gather(idx, src, n, cols / 8, dst, stream, "gather_rows");
}

extern "C" int rlk_fused_add_rmsnorm(uint16_t* residual, const uint16_t* delta,
                                     const uint16_t* weight, int rows, int hidden, float eps,
                                     uint16_t* out, hipStream_t stream) {
  if (rows <= 0) return RLK_OK;
  if (hidden <= 0 || hidden % 8 != 0)
    return fail(RLK_EINVAL, "fused_add_rmsnorm: hidden size must be a multiple of 8 (got %d)",
                hidden);
  const int vecs = hidden / 8;
  auto* res = reinterpret_cast<u32x4*>(residual);
  const auto* del = reinterpret_cast<const u32x4*>(delta);
  const auto* w = reinterpret_cast<const u32x4*>(weight);
  auto* o = reinterpret_cast<u32x4*>(out);
  const float hidden_f = static_cast<float>(hidden);
  // Lanes per row: one wave64 per row once there are enough rows to fill the
  // chip; a whole 256-lane block per row for small (decode) batches so that a
  // row's loads spread over four SIMDs.
  int tpr = rows >= 2048 ? 64 : 256;
  tpr = tune_knob("RLK_TUNE_NORM_TPR", tpr);
  bool launched = false;
  int nv = round_up_nv((vecs + tpr - 1) / tpr);
  if (nv > 0) {
    switch (tpr) {
      case 64: launched = launch_norm_t<64>(nv, res, del, w, rows, vecs, hidden_f, eps, o, stream); break;
      case 128: launched = launch_norm_t<128>(nv, res, del, w, rows, vecs, hidden_f, eps, o, stream); break;
      default: launched = launch_norm_t<256>(nv, res, del, w, rows, vecs, hidden_f, eps, o, stream); break;
    }
  }
  if (!launched) {
    nv = round_up_nv((vecs + kThreads - 1) / kThreads);
    if (nv > 0) {
      launched = launch_norm_t<256>(nv, res, del, w, rows, vecs, hidden_f, eps, o, stream);
    }
  }
  if (!launched) {
    if (del != nullptr) {
      add_rmsnorm_wide_kernel<true><<<rows, kThreads, 0, stream>>>(res, del, w, vecs, hidden_f, eps, o);
    } else {
      add_rmsnorm_wide_kernel<false><<<rows, kThreads, 0, stream>>>(res, del, w, vecs, hidden_f, eps, o);
    }
  }
  return launch_status("fused_add_rmsnorm");
}

extern "C" int rlk_silu_and_mul(const uint16_t* gate_up, int rows, int inter, uint16_t* out,
                                hipStream_t stream) {
  if (rows <= 0) return RLK_OK;
  if (inter <= 0 || inter % 8 != 0)
    return fail(RLK_EINVAL, "silu_and_mul: intermediate size must be a multiple of 8 (got %d)",
                inter);
  const int vecs = inter / 8;
  const int nv = tune_knob("RLK_TUNE_SWIGLU_NV", pick_nv(rows, vecs, 2048));
  const int chunks = (vecs + kThreads * nv - 1) / (kThreads * nv);
  const int64_t blocks = static_cast<int64_t>(rows) * chunks;
  if (blocks > 0x7fffffff) return fail(RLK_EINVAL, "silu_and_mul: too many rows (%d)", rows);
  const auto* gu = reinterpret_cast<const u32x4*>(gate_up);
  auto* o = reinterpret_cast<u32x4*>(out);
  switch (nv) {
    case 1: silu_and_mul_kernel<1><<<blocks, kThreads, 0, stream>>>(gu, vecs, chunks, o); break;
    case 2: silu_and_mul_kernel<2><<<blocks, kThreads, 0, stream>>>(gu, vecs, chunks, o); break;
    default: silu_and_mul_kernel<4><<<blocks, kThreads, 0, stream>>>(gu, vecs, chunks, o); break;
  }
  return launch_status("silu_and_mul");
}

extern "C" int rlk_silu_and_mul_interleaved(const uint16_t* gate_up, int rows, int inter,
                                            uint16_t* out, hipStream_t stream) {
  if (rows <= 0) return RLK_OK;
  if (inter <= 0) return fail(RLK_EINVAL, "silu_and_mul_interleaved: bad intermediate size %d", inter);
  if (inter % 8 == 0) {
    const int vecs = inter / 8;
    const int nv = tune_knob("RLK_TUNE_SWIGLU_NV", pick_nv(rows, vecs, 2048));
    const int chunks = (vecs + kThreads * nv - 1) / (kThreads * nv);
    const int64_t blocks = static_cast<int64_t>(rows) * chunks;
    if (blocks > 0x7fffffff) return fail(RLK_EINVAL, "silu_and_mul_interleaved: too many rows");
    const auto* gu = reinterpret_cast<const u32x4*>(gate_up);
    auto* o = reinterpret_cast<u32x4*>(out);
    switch (nv) {
      case 1: silu_and_mul_interleaved_kernel<1><<<blocks, kThreads, 0, stream>>>(gu, vecs, chunks, o); break;
      case 2: silu_and_mul_interleaved_kernel<2><<<blocks, kThreads, 0, stream>>>(gu, vecs, chunks, o); break;
      default: silu_and_mul_interleaved_kernel<4><<<blocks, kThreads, 0, stream>>>(gu, vecs, chunks, o); break;
    }
  } else {
    const int64_t total = static_cast<int64_t>(rows) * inter;
    const int64_t blocks = (total + kThreads - 1) / kThreads;
    if (blocks > 0x7fffffff) return fail(RLK_EINVAL, "silu_and_mul_interleaved: too many rows");
    silu_and_mul_interleaved_scalar_kernel<<<blocks, kThreads, 0, stream>>>(
        reinterpret_cast<const f16x2*>(gate_up), total, reinterpret_cast<_Float16*>(out));
  }
  return launch_status("silu_and_mul_interleaved");
}

extern "C" int rlk_resolve_input_ids(int32_t* input_ids, const int32_t* src,
                                     const int32_t* prev_sampled, int n, hipStream_t stream) {
  if (n <= 0) return RLK_OK;
  resolve_input_ids_kernel<<<(n + kThreads - 1) / kThreads, kThreads, 0, stream>>>(
      input_ids, src, prev_sampled, n);
  return launch_status("resolve_input_ids");
}
