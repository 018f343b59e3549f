/*
 * rlk.h — C ABI of the MI355X (gfx950) fused per-layer kernels.
 *
 * Every device entry point is asynchronous on the given HIP stream, never
 * allocates, frees or synchronises, and is therefore capturable into a HIP
 * graph.  Pointers are device pointers owned by the caller.  fp16 tensors are
 * passed as uint16_t* holding IEEE binary16 bit patterns.  Row data moves as
 * 16-byte vectors, as in the reference's kernels: tensors and row strides must
 * be 16-byte aligned (hipMalloc'd buffers are), and an output must not overlap
 * an input unless the entry point says it is updated in place (residual, qkv).
 *
 * Return value: RLK_OK (0) on success; a negative RLK_E* code for an argument
 * error detected on the host before anything is launched; a positive hipError_t
 * value when the launch itself failed.  rlk_last_error() gives the message of
 * the most recent failure on the calling thread.
 *
 * Reference interface replaced: redline::kernels in
 * src/cuda/kernels/kernels.h:64-88 (Neil456/Redline).  The C++ header
 * redline_amd/kernels.h wraps these entry points with the reference's exact
 * names, parameter order and exception behaviour.
 */
#ifndef REDLINE_AMD_RLK_H_
#define REDLINE_AMD_RLK_H_

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RLK_OK 0
#define RLK_EINVAL (-1)      /* invalid shape / argument (reference: RL_CHECK throw) */
#define RLK_EUNSUPPORTED (-2) /* unsupported configuration, e.g. head_dim */

/* KV cache element type; values match redline::KVDType (kernels.h:13). */
#define RLK_KV_FP16 0
#define RLK_KV_INT8 1

/*
 * One layer of the paged KV cache.  Field order, types and sizes are those of
 * redline::KVLayerView (src/cuda/kernels/kernels.h:18-27), so a pointer to the
 * reference struct can be passed unchanged.
 *   k, v              [num_blocks, num_kv_heads, block_size, head_dim]  fp16 or int8
 *   k_scale, v_scale  [num_blocks, num_kv_heads, block_size]  fp32 (INT8 only)
 */
typedef struct rlk_kv_layer_view {
  void* k;
  void* v;
  float* k_scale; /* fp16 cells instead with RLK_SCALE_F16 (rlk_rope_and_write_kv_ex) */
  float* v_scale;
  int block_size;
  int num_kv_heads;
  int head_dim;
  int dtype; /* RLK_KV_FP16 | RLK_KV_INT8 */
} rlk_kv_layer_view;

/* Message of the last failure on this thread ("" if none). */
const char* rlk_last_error(void);
/* Library version string. */
const char* rlk_version(void);

/* Tuning hook (no counterpart in the reference): sets (set != 0) or clears
 * the launch-policy override `name` (one of RLK_TUNE_GATHER_BS, _GATHER_NT,
 * _NORM_TPR, _NORM_NT, _SWIGLU_BS, _SWIGLU_NT, _ROPE_WPT, _ATTN_PERSIST,
 * _W4_CFG, _W8_CFG, _PREFILL_DMA, _PREFILL_QS, _ATTN_PV).  The environment variables of
 * the same names are read once, at the first launch of the process; later
 * changes go through this call only.  Unknown name: RLK_EINVAL.
 * The knobs are process-wide, not per stream or thread: a change applies to
 * every later launch from any thread, so change them only while no other
 * thread launches (tuning runs and tests). */
int rlk_set_tune_knob(const char* name, int value, int set);
/* Reads the override `name`: *is_set = 1 and *value = its value when set,
 * else *is_set = 0 and *value = 0.  Unknown name or null output: RLK_EINVAL. */
int rlk_get_tune_knob(const char* name, int* value, int* is_set);

/* ------------------------------------------------------------ elementwise */

/* out[t, :] = table[ids[t], :]   (table [V, hidden], out [n, hidden]).
 * Replaces kernels::embedding_lookup, elementwise.cu:106-112.
 * n <= 0: no-op.  hidden % 8 != 0: RLK_EINVAL.  ids are not bounds-checked. */
int rlk_embedding_lookup(const int32_t* ids, const uint16_t* table, int n, int hidden,
                         uint16_t* out, hipStream_t stream);

/* residual = fp16(residual + delta) in place (skipped when delta == NULL);
 * out = fp16(fp16(residual * rsqrt(mean(residual^2) + eps)) * weight).
 * Replaces kernels::fused_add_rmsnorm, elementwise.cu:114-121.
 * rows <= 0: no-op.  hidden % 8 != 0: RLK_EINVAL. */
int rlk_fused_add_rmsnorm(uint16_t* residual, const uint16_t* delta, const uint16_t* weight,
                          int rows, int hidden, float eps, uint16_t* out, hipStream_t stream);

/* Extension, no single counterpart in the reference: residual[t, :] =
 * table[ids[t], :] and out = RMSNorm(residual) * weight in one launch -- the
 * same results as the reference's back-to-back embedding_lookup(ids, table,
 * n, hidden, residual) and fused_add_rmsnorm(residual, NULL, weight, n,
 * hidden, eps, out) that start its forward pass (src/cuda/model/llama.cpp:79-80),
 * with one launch and one pass over the rows instead of two.
 * n <= 0: no-op.  hidden % 8 != 0: RLK_EINVAL.  ids are not bounds-checked.
 * table, weight, residual and out are read and written as 16-byte vectors:
 * each must be 16-byte aligned (else RLK_EINVAL), and residual and out must
 * not overlap each other or the table. */
int rlk_embedding_rmsnorm(const int32_t* ids, const uint16_t* table, int n, int hidden,
                          const uint16_t* weight, float eps, uint16_t* residual, uint16_t* out,
                          hipStream_t stream);

/* out[r, i] = fp16(fp16(silu(gate_up[r, i])) * gate_up[r, inter + i]).
 * Replaces kernels::silu_and_mul, elementwise.cu:140-145.
 * rows <= 0: no-op.  inter % 8 != 0: RLK_EINVAL. */
int rlk_silu_and_mul(const uint16_t* gate_up, int rows, int inter, uint16_t* out,
                     hipStream_t stream);

/* Same with gate/up interleaved: gate = gate_up[r, 2i], up = gate_up[r, 2i+1].
 * Replaces kernels::silu_and_mul_interleaved, elementwise.cu:133-138.
 * rows <= 0: no-op.  Any inter >= 1 is accepted (as in the reference). */
int rlk_silu_and_mul_interleaved(const uint16_t* gate_up, int rows, int inter, uint16_t* out,
                                 hipStream_t stream);

/* ---------------------------------------------- INT4 weight-only GEMV (decode)
 *
 * y[m, n] = x[m, k] . W[n, k]^T (+ bias[n]) with W group-quantised INT4:
 *   W[r][c] = q * scales[r][c / g] + offsets[r][c / g],
 *   q = code c of row r: byte c / 2 of the row, low nibble for even c.
 * w is [n, k/2] bytes; scales and offsets fp16 [n, k/g]; x fp16 [m, k].
 * m <= 0: no-op.  m > RLK_GEMV_W4_MAX_M: RLK_EUNSUPPORTED (the reference
 * serves m <= 16, kernels.h:161; this build serves m <= 32 in one launch).
 * k and group_size multiples of 32 with k % group_size == 0, else RLK_EINVAL;
 * x and w 16-byte aligned. */
#define RLK_GEMV_W4_MAX_M 32

/* INT8 weight-only GEMV (decode):
 * y[m, n] = (x[m, k] . W[n, k]^T) * scales[n] (+ bias[n]), W int8 row-major
 * with one fp16 scale per output row (the layout of quantize_int8_rows,
 * random_model.cpp:99-115); fp32 accumulation.  y fp16 [m, n], or fp32 when
 * y_fp32 != 0; bias fp16 [n] or NULL.  m <= 0: no-op.  m > RLK_GEMV_W8_MAX_M:
 * RLK_EUNSUPPORTED (the reference serves m <= 16).  k % 16 != 0: RLK_EINVAL;
 * x and w 16-byte aligned.  A weight over 2 GiB (n * k bytes): RLK_EUNSUPPORTED
 * (split n over calls).
 * Replaces kernels::gemv_w8a16, gemv_weight_only.cu:217-226 (kernels.h:162-163). */
#define RLK_GEMV_W8_MAX_M 32
int rlk_gemv_w8a16(const uint16_t* x, int m, const int8_t* w, const uint16_t* scales,
                   const uint16_t* bias, int n, int k, void* y, int y_fp32, hipStream_t stream);

/* y fp16 [m, n], or fp32 when y_fp32 != 0; bias fp16 [n] or NULL.
 * Replaces kernels::gemv_w4a16, gemv_weight_only.cu:228-239 (kernels.h:164-168). */
int rlk_gemv_w4a16(const uint16_t* x, int m, const uint8_t* w, const uint16_t* scales,
                   const uint16_t* offsets, int group_size, const uint16_t* bias, int n, int k,
                   void* y, int y_fp32, hipStream_t stream);

/* SwiGLU in the GEMV epilogue: rows (2i, 2i + 1) of w are (gate_i, up_i), the
 * loader's INT4 gate_up layout (weights.cpp:157-167); y fp16 [m, n/2] =
 * fp16(fp16(silu(fp16(gate))) * fp16(up)).  n must be even.
 * Replaces kernels::gemv_w4a16_swiglu, gemv_weight_only.cu:241-248 (kernels.h:169-171). */
int rlk_gemv_w4a16_swiglu(const uint16_t* x, int m, const uint8_t* w, const uint16_t* scales,
                          const uint16_t* offsets, int group_size, int n, int k, uint16_t* y,
                          hipStream_t stream);

/* dst[i, :] = src[idx[i], :].  Replaces kernels::gather_rows,
 * elementwise.cu:147-153.  n <= 0: no-op.  cols % 8 != 0: RLK_EINVAL. */
int rlk_gather_rows(const uint16_t* src, const int32_t* idx, int n, int cols, uint16_t* dst,
                    hipStream_t stream);

/* input_ids[i] = prev_sampled[src[i]] where src[i] >= 0.  Replaces
 * kernels::resolve_input_ids, elementwise.cu:99-104.  n <= 0: no-op. */
int rlk_resolve_input_ids(int32_t* input_ids, const int32_t* src, const int32_t* prev_sampled,
                          int n, hipStream_t stream);

/* ------------------------------------------------------------- rope / kv */

/* RoPE (rotate-half pairs (i, i + D/2)) on the q and k heads of
 * qkv [num_tokens, (num_heads + 2*kv->num_kv_heads) * D]; the roped q heads are
 * written back in place (the k section of qkv is left as it was); roped k and
 * unchanged v are written into the paged cache cell
 * ((slot / bs * Hkv + kvh) * bs + slot % bs) * D for slot = slot_mapping[t]
 * (slot < 0: no KV write).  INT8 cache: per-(token, head) scale amax/127
 * stored as fp32, codes rint(clamp(x / scale, -127, 127)).
 * cos_table / sin_table: fp32 [max_pos, D/2].
 * Replaces kernels::rope_and_write_kv, rope_kv.cu:107-123.
 * num_tokens <= 0: no-op.  head_dim not in {64, 128}: RLK_EUNSUPPORTED. */
int rlk_rope_and_write_kv(uint16_t* qkv, const int32_t* positions, const int32_t* slot_mapping,
                          int num_tokens, int num_heads, const float* cos_table,
                          const float* sin_table, const rlk_kv_layer_view* kv,
                          hipStream_t stream);

/* Extension with no counterpart in the reference interface: options of
 * rlk_rope_and_write_kv_ex.
 *   qkv_bias     fp16 [(Hq + 2*Hkv) * D] added to every head before the
 *                rotation (x = fp16(x + b)), the Qwen2 attention bias that the
 *                reference adds in its QKV GEMM epilogue
 *                (src/cuda/gemm/linear.cpp:108); NULL = no bias.  The k and v
 *                sections of qkv are left as they were (only the cache sees the
 *                biased k/v); the q section receives bias + RoPE.
 *   scale_dtype  RLK_SCALE_F32: fp32 per-cell scales (the reference layout,
 *                kv_cache.cpp:45-48).  RLK_SCALE_F16: scales stored as fp16 and
 *                codes quantised against the stored (fp16-rounded) scale; the
 *                k_scale / v_scale pointers then address uint16_t cells.
 *                Codes may differ by 1 from the fp32-scale codes. */
#define RLK_SCALE_F32 0
#define RLK_SCALE_F16 1

typedef struct rlk_rope_kv_options {
  const uint16_t* qkv_bias;
  int scale_dtype;
} rlk_rope_kv_options;

/* rlk_rope_and_write_kv with options (NULL options = the plain entry point). */
int rlk_rope_and_write_kv_ex(uint16_t* qkv, const int32_t* positions,
                             const int32_t* slot_mapping, int num_tokens, int num_heads,
                             const float* cos_table, const float* sin_table,
                             const rlk_kv_layer_view* kv, const rlk_rope_kv_options* options,
                             hipStream_t stream);

/* -------------------------------------------------------------- attention */

/* Keys per split-K partition of the decode attention (the reference's
 * kDecodePartitionSize, kernels.h:116); it fixes the workspace layout. */
#define RLK_DECODE_PARTITION_SIZE 256

/* Field order and types of redline::kernels::AttentionParams
 * (src/cuda/kernels/kernels.h:91-101). */
typedef struct rlk_attention_params {
  const uint16_t* q;     /* query rows, q_stride elements per token (fp16) */
  int q_stride;
  uint16_t* out;         /* [num_tokens, num_heads * head_dim] fp16 */
  int num_heads;
  float scale;           /* softmax scale, applied to q */
  rlk_kv_layer_view kv;
  const int32_t* block_tables; /* [num_seqs, max_blocks_per_seq] */
  int max_blocks_per_seq;
  const int32_t* positions;    /* [num_tokens] */
} rlk_attention_params;

/* Field order and types of redline::kernels::DecodeAttentionWork
 * (kernels.h:106-115). */
typedef struct rlk_decode_attention_work {
  const int32_t* item_token; /* [num_items] query token of each decode item */
  const int32_t* item_seq;   /* [num_items] its sequence (row of block_tables) */
  int num_items;
  int max_partitions;        /* grid size; partitions beyond a context exit early */
  float* ws_out;             /* [num_items, num_heads, max_partitions, head_dim] */
  float* ws_max;             /* [num_items, num_heads, max_partitions] */
  float* ws_sum;
} rlk_decode_attention_work;

/* Decode attention: item i's query token t attends to positions
 * [0, positions[t]] of its sequence through the paged cache (FP16, or INT8
 * with fp32 scales); all G = num_heads / num_kv_heads query heads of a kv head
 * share each K/V read; contexts longer than one partition are split and merged
 * through the caller's workspace.  Replaces kernels::paged_attention_decode,
 * src/cuda/kernels/attention.cu:70-210,362-398.
 * num_items <= 0: no-op.  head_dim not in {64, 128} or G > 8: RLK_EUNSUPPORTED.
 * max_partitions > 1 needs ws_out / ws_max / ws_sum (scratch: what they hold
 * after a call is unspecified).
 * Contract: max_partitions >= ceil((positions[t] + 1) / 256) for every item.
 * Keys past max_partitions * 256 are not read, and no error is reported (the
 * launcher cannot see device-side positions without synchronising). */
int rlk_paged_attention_decode(const rlk_attention_params* params,
                               const rlk_decode_attention_work* work, hipStream_t stream);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): rlk_paged_attention_decode with the split-K partials in a
 * library-owned device array of RLK_DECODE_SCRATCH_BYTES per GPU instead of
 * work->ws_out / ws_max / ws_sum, which are ignored.  The array is a static
 * device variable: it is reserved (32 MiB of HBM) on every GPU the library's
 * code object is loaded on, whether or not this entry point is ever called,
 * and is held until the process ends.  max_partitions == 1 uses no scratch.  Allocates nothing.  Needs num_items * num_heads * max_partitions *
 * (head_dim + 2) * 4 bytes (each of the three regions rounded up to 256);
 * more than RLK_DECODE_SCRATCH_BYTES: RLK_EINVAL.  Every call on a GPU shares
 * that GPU's array: calls that overlap on one GPU (different streams, or
 * threads) race and must be serialised by the caller. */
#define RLK_DECODE_SCRATCH_BYTES (32u << 20)
int rlk_paged_attention_decode_noalloc(const rlk_attention_params* params,
                                       const rlk_decode_attention_work* work, hipStream_t stream);

/* Extension, no counterpart in the reference (whose scales are fp32 only):
 * decode attention over an INT8 cache whose scales were stored as fp16 by
 * rlk_rope_and_write_kv_ex with RLK_SCALE_F16 (k_scale / v_scale then address
 * uint16_t cells).  options->scale_dtype: RLK_SCALE_F32 or RLK_SCALE_F16;
 * NULL options = rlk_paged_attention_decode. */
typedef struct rlk_attention_options {
  int scale_dtype;
} rlk_attention_options;

int rlk_paged_attention_decode_ex(const rlk_attention_params* params,
                                  const rlk_decode_attention_work* work,
                                  const rlk_attention_options* options, hipStream_t stream);

/* Field order and types of redline::kernels::PrefillAttentionWork
 * (kernels.h:122-129).  max_q_tiles counts the reference's 32-row query tiles
 * (kPrefillTileQ, kernels.h:130), as BatchBuilder writes it. */
#define RLK_PREFILL_TILE_Q 32
typedef struct rlk_prefill_attention_work {
  const int32_t* seq_ids; /* [num_seqs] indices into the arrays below */
  const int32_t* q_start; /* [*] first query row of each sequence */
  const int32_t* q_len;   /* [*] number of new tokens */
  const int32_t* ctx_len; /* [*] total context after this step */
  int num_seqs;
  int max_q_tiles;        /* ceil(max q_len / RLK_PREFILL_TILE_Q) */
} rlk_prefill_attention_work;

/* Prefill attention: causal attention of each sequence's new tokens (rows
 * q_start .. q_start + q_len - 1 of q and out) over positions [0, past + i],
 * past = ctx_len - q_len, through the paged cache (FP16, or INT8 with fp32
 * per-cell scales, dequantised to fp16 as the reference does).  num_seqs <= 0 or
 * max_q_tiles <= 0: no-op; head_dim not in {64, 128}: RLK_EUNSUPPORTED;
 * num_heads not a multiple of num_kv_heads, a null pointer, or q rows that are
 * not 16-byte aligned: RLK_EINVAL.
 * Replaces kernels::paged_attention_prefill, attention.cu:423-431 (kernels.h:131-132). */
int rlk_paged_attention_prefill(const rlk_attention_params* params,
                                const rlk_prefill_attention_work* work, hipStream_t stream);

/* Extension, no counterpart in the reference: prefill attention over an INT8
 * cache whose scales rlk_rope_and_write_kv_ex stored as fp16 (options as for
 * rlk_paged_attention_decode_ex). */
int rlk_paged_attention_prefill_ex(const rlk_attention_params* params,
                                   const rlk_prefill_attention_work* work,
                                   const rlk_attention_options* options, hipStream_t stream);

/* ------------------------------------------------------ host-side helpers */

/* IEEE fp16 <-> fp32 with round-to-nearest-even.
 * Replace redline::float_to_half_bits / half_bits_to_float, common.cpp:37-89. */
uint16_t rlk_float_to_half_bits(float f);
float rlk_half_bits_to_float(uint16_t h);

/* Rotary inverse frequencies [head_dim/2] in double, with optional scaling:
 * scaling_type 0 = none, 1 = linear, 2 = llama3.
 * Replaces redline::rope_inv_freq, model_config.cpp:126-153. */
int rlk_rope_inv_freq(double theta, int head_dim, int scaling_type, double factor,
                      double low_freq_factor, double high_freq_factor,
                      int original_max_position_embeddings, double* inv_freq);

/* fp32 cos/sin tables [max_pos, head_dim/2], angle = float(p) * float(inv[i]).
 * Replaces redline::rope_cos_sin_tables, model_config.cpp:155-169. */
int rlk_rope_cos_sin_tables(double theta, int head_dim, int scaling_type, double factor,
                            double low_freq_factor, double high_freq_factor,
                            int original_max_position_embeddings, int max_pos,
                            float* cos_table, float* sin_table);

/* ------------------------------------------------- batch metadata (host) */

/* Shape of a serialized batch; fields of redline::BatchShape, batch_builder.h:16-26. */
typedef struct rlk_batch_shape {
  int num_tokens;
  int num_seqs;
  int num_logit_rows;
  int num_decode_items;
  int num_prefill_seqs;
  int max_prefill_q_tiles;
  int max_context;
} rlk_batch_shape;

/* Word offsets inside the metadata buffer; fields of redline::MetaLayout,
 * batch_builder.h:29-38, in the same order. */
typedef struct rlk_meta_layout {
  size_t input_ids, input_src, positions, slot_mapping;
  size_t seq_q_start, seq_q_len, seq_ctx_len;
  size_t block_tables;
  size_t decode_token, decode_seq;
  size_t prefill_seq;
  size_t logit_token, param_row;
  size_t temperature, top_k, top_p, seed_lo, seed_hi;
  size_t total_words;
} rlk_meta_layout;

/* Logits selection of BatchBuilder::add (redline::LogitsMode). */
#define RLK_LOGITS_NONE 0
#define RLK_LOGITS_LAST 1
#define RLK_LOGITS_ALL 2

typedef struct rlk_batch_builder rlk_batch_builder;

/* Replaces MetaLayout::make, batch_builder.cpp:17-46. */
int rlk_meta_layout_make(const rlk_batch_shape* shape, int max_blocks_per_seq,
                         rlk_meta_layout* out);

/* Replaces the BatchBuilder constructor, batch_builder.cpp:48-55.  NULL on bad args. */
rlk_batch_builder* rlk_batch_builder_create(int max_tokens, int max_seqs, int max_logit_rows,
                                            int max_blocks_per_seq, int block_size,
                                            int decode_query_threshold);
void rlk_batch_builder_destroy(rlk_batch_builder* b);
void rlk_batch_builder_reset(rlk_batch_builder* b);
size_t rlk_batch_builder_max_meta_words(const rlk_batch_builder* b);
/* Replaces BatchBuilder::add, batch_builder.cpp:80-122.  tokens may be NULL
 * when every src_rows[i] >= 0; src_rows may be NULL.  *first_row receives the
 * first logits row added (or -1).  Errors (RLK_EINVAL) leave the builder
 * unchanged. */
int rlk_batch_builder_add(rlk_batch_builder* b, const int32_t* tokens, int start_pos, int n,
                          const int32_t* src_rows, const int32_t* blocks, int num_blocks,
                          float temperature, int top_k, float top_p, uint64_t seed,
                          int logits_mode, int* first_row);
/* Replaces BatchBuilder::pad_decode_to, batch_builder.cpp:124-129. */
int rlk_batch_builder_pad_decode_to(rlk_batch_builder* b, int num_seqs);
/* Replaces BatchBuilder::shape / write, batch_builder.cpp:131-188.  dst holds
 * at least rlk_batch_builder_max_meta_words() int32 words. */
int rlk_batch_builder_shape(const rlk_batch_builder* b, rlk_batch_shape* shape);
int rlk_batch_builder_write(const rlk_batch_builder* b, int32_t* dst, rlk_batch_shape* shape);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif /* REDLINE_AMD_RLK_H_ */
