// C++ launch interface of the MI355X fused per-layer kernels.
//
// Same namespace, names, parameter order and KVLayerView field layout as the
// reference's redline::kernels (src/cuda/kernels/kernels.h:13-27, 64-88), spelled
// with hipStream_t and __half.  Each launcher forwards to the C ABI in rlk.h and
// turns a non-zero status into a thrown redline::Error, which is how the
// reference reports RL_CHECK failures (src/core/common.h:25-32) and failed
// launches (src/cuda/cuda_utils.h:19).  Launchers are asynchronous on `stream`,
// never allocate or synchronise, and are capturable into HIP graphs.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>

#include "redline_amd/rlk.h"

// Inside a Redline build (src/ on the include path) the engine's own
// redline::Error is used; standalone, an identical class is declared here.
#if __has_include("core/common.h")
#include "core/common.h"
#else
namespace redline {

class Error : public std::runtime_error {
 public:
  explicit Error(const std::string& msg) : std::runtime_error(msg) {}
};

}  // namespace redline
#endif

namespace redline {

enum class KVDType { kFP16 = RLK_KV_FP16, kINT8 = RLK_KV_INT8 };

// One layer of the paged KV cache.
//   k, v:             [num_blocks, num_kv_heads, block_size, head_dim]  (half or int8)
//   k_scale, v_scale: [num_blocks, num_kv_heads, block_size] float     (INT8 only)
struct KVLayerView {
  void* k = nullptr;
  void* v = nullptr;
  float* k_scale = nullptr;
  float* v_scale = nullptr;
  int block_size = 16;
  int num_kv_heads = 0;
  int head_dim = 0;
  KVDType dtype = KVDType::kFP16;
};

static_assert(sizeof(KVLayerView) == sizeof(rlk_kv_layer_view), "KVLayerView layout");
static_assert(offsetof(KVLayerView, block_size) == offsetof(rlk_kv_layer_view, block_size),
              "KVLayerView layout");
static_assert(offsetof(KVLayerView, dtype) == offsetof(rlk_kv_layer_view, dtype),
              "KVLayerView layout");

namespace kernels {

// Attention interface structs: field order of the reference's
// (src/cuda/kernels/kernels.h:91-117).
struct AttentionParams {
  const half* q = nullptr;  // query rows, stride q_stride elements per token
  int q_stride = 0;
  half* out = nullptr;      // [num_tokens, num_heads * head_dim]
  int num_heads = 0;
  float scale = 1.0f;
  KVLayerView kv;
  const int32_t* block_tables = nullptr;  // [num_seqs, max_blocks_per_seq]
  int max_blocks_per_seq = 0;
  const int32_t* positions = nullptr;     // [num_tokens]
};

struct DecodeAttentionWork {
  const int32_t* item_token = nullptr;  // [num_items]
  const int32_t* item_seq = nullptr;    // [num_items]
  int num_items = 0;
  int max_partitions = 1;   // grid size; partitions beyond the context exit early.
                            // Must be >= ceil(context / 256) for every item: keys
                            // past max_partitions * 256 are not read (no error)
  float* ws_out = nullptr;  // [num_items, num_heads, max_partitions, head_dim]
  float* ws_max = nullptr;  // [num_items, num_heads, max_partitions]
  float* ws_sum = nullptr;
};
constexpr int kDecodePartitionSize = RLK_DECODE_PARTITION_SIZE;

static_assert(sizeof(AttentionParams) == sizeof(rlk_attention_params), "AttentionParams layout");
static_assert(offsetof(AttentionParams, positions) == offsetof(rlk_attention_params, positions),
              "AttentionParams layout");
static_assert(sizeof(DecodeAttentionWork) == sizeof(rlk_decode_attention_work),
              "DecodeAttentionWork layout");

// Prefill attention: tiled causal attention for sequences processing several
// new tokens, attending to cached + new keys (kernels.h:118-132 of the reference).
struct PrefillAttentionWork {
  const int32_t* seq_ids = nullptr;  // [num_seqs] indices into the arrays below
  const int32_t* q_start = nullptr;  // [*] first token row of each sequence
  const int32_t* q_len = nullptr;    // [*] number of new tokens
  const int32_t* ctx_len = nullptr;  // [*] total context after this step
  int num_seqs = 0;
  int max_q_tiles = 0;
};
constexpr int kPrefillTileQ = RLK_PREFILL_TILE_Q;

static_assert(sizeof(PrefillAttentionWork) == sizeof(rlk_prefill_attention_work),
              "PrefillAttentionWork layout");
static_assert(offsetof(PrefillAttentionWork, max_q_tiles) ==
                  offsetof(rlk_prefill_attention_work, max_q_tiles),
              "PrefillAttentionWork layout");

namespace detail {

inline void check(int status) {
  if (status != RLK_OK) throw Error(rlk_last_error());
}
inline uint16_t* bits(half* p) { return reinterpret_cast<uint16_t*>(p); }
inline const uint16_t* bits(const half* p) { return reinterpret_cast<const uint16_t*>(p); }

}  // namespace detail

// input_ids[i] = src[i] >= 0 ? prev_sampled[src[i]] : input_ids[i]
inline void resolve_input_ids(int32_t* input_ids, const int32_t* src, const int32_t* prev_sampled,
                              int n, hipStream_t stream) {
  detail::check(rlk_resolve_input_ids(input_ids, src, prev_sampled, n, stream));
}

inline void embedding_lookup(const int32_t* ids, const half* table, int n, int hidden, half* out,
                             hipStream_t stream) {
  detail::check(rlk_embedding_lookup(ids, detail::bits(table), n, hidden, detail::bits(out), stream));
}

// residual += delta (skipped when delta == nullptr); out = rmsnorm(residual) * weight.
inline void fused_add_rmsnorm(half* residual, const half* delta, const half* weight, int rows,
                              int hidden, float eps, half* out, hipStream_t stream) {
  detail::check(rlk_fused_add_rmsnorm(detail::bits(residual), detail::bits(delta),
                                      detail::bits(weight), rows, hidden, eps, detail::bits(out),
                                      stream));
}

// Extension: residual = table[ids]; out = rmsnorm(residual) * weight in one
// launch (the reference's embedding_lookup + fused_add_rmsnorm(delta = nullptr)
// pair at the start of the forward pass, llama.cpp:79-80).
inline void embedding_rmsnorm(const int32_t* ids, const half* table, int n, int hidden,
                              const half* weight, float eps, half* residual, half* out,
                              hipStream_t stream) {
  detail::check(rlk_embedding_rmsnorm(ids, detail::bits(table), n, hidden, detail::bits(weight),
                                      eps, detail::bits(residual), detail::bits(out), stream));
}

// out[r, i] = silu(gate_up[r, i]) * gate_up[r, inter + i]
inline void silu_and_mul(const half* gate_up, int rows, int inter, half* out, hipStream_t stream) {
  detail::check(rlk_silu_and_mul(detail::bits(gate_up), rows, inter, detail::bits(out), stream));
}

// Same, for gate/up columns interleaved as (gate_0, up_0, gate_1, up_1, ...).
inline void silu_and_mul_interleaved(const half* gate_up, int rows, int inter, half* out,
                                     hipStream_t stream) {
  detail::check(
      rlk_silu_and_mul_interleaved(detail::bits(gate_up), rows, inter, detail::bits(out), stream));
}

// dst[i, :] = src[idx[i], :]
inline void gather_rows(const half* src, const int32_t* idx, int n, int cols, half* dst,
                        hipStream_t stream) {
  detail::check(rlk_gather_rows(detail::bits(src), idx, n, cols, detail::bits(dst), stream));
}

// RoPE on the q and k heads of qkv [num_tokens, (Hq + 2 Hkv) * D]; roped q is
// written back in place and k/v go to the paged cache at slot_mapping[t]
// (block * block_size + offset; negative = skip).
inline void rope_and_write_kv(half* qkv, const int32_t* positions, const int32_t* slot_mapping,
                              int num_tokens, int num_heads, const float* cos_table,
                              const float* sin_table, const KVLayerView& kv, hipStream_t stream) {
  detail::check(rlk_rope_and_write_kv(detail::bits(qkv), positions, slot_mapping, num_tokens,
                                      num_heads, cos_table, sin_table,
                                      reinterpret_cast<const rlk_kv_layer_view*>(&kv), stream));
}

// Paged decode attention (flash-decoding split-K over 256-key partitions).
inline void paged_attention_decode(const AttentionParams& p, const DecodeAttentionWork& w,
                                   hipStream_t stream) {
  detail::check(rlk_paged_attention_decode(reinterpret_cast<const rlk_attention_params*>(&p),
                                           reinterpret_cast<const rlk_decode_attention_work*>(&w),
                                           stream));
}

// Paged prefill attention (causal, tiled on the matrix cores).
inline void paged_attention_prefill(const AttentionParams& p, const PrefillAttentionWork& w,
                                    hipStream_t stream) {
  detail::check(rlk_paged_attention_prefill(reinterpret_cast<const rlk_attention_params*>(&p),
                                            reinterpret_cast<const rlk_prefill_attention_work*>(&w),
                                            stream));
}

// INT8 weight-only GEMV (kernels.h:157-163 of the reference): y = (x . W^T) *
// scales (+ bias), one fp16 scale per row.  The reference chunks batches into
// kGemvW8MaxM = 16 rows per launch; this library serves up to 32 in one launch.
constexpr int kGemvW8MaxM = RLK_GEMV_W8_MAX_M;

inline void gemv_w8a16(const half* x, int m, const int8_t* w, const half* scales, const half* bias,
                       int n, int k, void* y, bool y_fp32, hipStream_t stream) {
  detail::check(rlk_gemv_w8a16(detail::bits(x), m, w, detail::bits(scales), detail::bits(bias), n,
                               k, y, y_fp32 ? 1 : 0, stream));
}

// INT4 weight-only GEMV (kernels.h:156-171 of the reference).  The reference
// serves m <= kGemvW4MaxM = 16 per launch; this library serves up to
// kGemvW4MaxM here (32) in one launch.
constexpr int kGemvW4MaxM = RLK_GEMV_W4_MAX_M;

inline void gemv_w4a16(const half* x, int m, const uint8_t* w, const half* scales,
                       const half* offsets, int group_size, const half* bias, int n, int k, void* y,
                       bool y_fp32, hipStream_t stream) {
  detail::check(rlk_gemv_w4a16(detail::bits(x), m, w, detail::bits(scales), detail::bits(offsets),
                               group_size, detail::bits(bias), n, k, y, y_fp32 ? 1 : 0, stream));
}

// Same kernel for a [gate; up] weight whose rows are interleaved (gate_i, up_i):
// writes silu(gate) * up, fp16 [m, n / 2], from the GEMV epilogue.
inline void gemv_w4a16_swiglu(const half* x, int m, const uint8_t* w, const half* scales,
                              const half* offsets, int group_size, int n, int k, half* y,
                              hipStream_t stream) {
  detail::check(rlk_gemv_w4a16_swiglu(detail::bits(x), m, w, detail::bits(scales),
                                      detail::bits(offsets), group_size, n, k, detail::bits(y),
                                      stream));
}

}  // namespace kernels
}  // namespace redline
