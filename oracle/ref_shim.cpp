// extern "C" entry points onto the reference's own host core (compiled from
// /root/reference/src/core by oracle/Makefile's `ref` target).  TEST
// INFRASTRUCTURE ONLY: used by tests/golden/make_golden.py to write golden
// vectors and by tests/test_oracle.py to pin the oracle; never shipped.
#include <cstdint>
#include <cstring>
#include <exception>
#include <vector>

#include "core/batch_builder.h"
#include "core/common.h"
#include "core/model_config.h"
#include "cpu/random_model.h"
#include "cpu/reference_model.h"

using namespace redline;

namespace {
ModelConfig rope_cfg(double theta, int head_dim, int scaling, double factor, double lo, double hi,
                     int old_ctx) {
  ModelConfig c;
  c.head_dim = head_dim;
  c.rope_theta = theta;
  c.rope_scaling.type = scaling == 1 ? "linear" : (scaling == 2 ? "llama3" : "none");
  c.rope_scaling.factor = factor;
  c.rope_scaling.low_freq_factor = lo;
  c.rope_scaling.high_freq_factor = hi;
  c.rope_scaling.original_max_position_embeddings = old_ctx;
  return c;
}
}  // namespace

extern "C" {

uint16_t ref_float_to_half_bits(float f) { return float_to_half_bits(f); }
float ref_half_bits_to_float(uint16_t h) { return half_bits_to_float(h); }

void ref_float_to_half_many(const float* in, size_t n, uint16_t* out) {
  for (size_t i = 0; i < n; ++i) out[i] = float_to_half_bits(in[i]);
}

void ref_rope_inv_freq(double theta, int head_dim, int scaling, double factor, double lo, double hi,
                       int old_ctx, double* out) {
  const auto v = rope_inv_freq(rope_cfg(theta, head_dim, scaling, factor, lo, hi, old_ctx));
  std::memcpy(out, v.data(), v.size() * sizeof(double));
}

void ref_rope_cos_sin_tables(double theta, int head_dim, int scaling, double factor, double lo,
                             double hi, int old_ctx, int max_pos, float* cos_t, float* sin_t) {
  std::vector<float> c, s;
  rope_cos_sin_tables(rope_cfg(theta, head_dim, scaling, factor, lo, hi, old_ctx), max_pos, &c, &s);
  std::memcpy(cos_t, c.data(), c.size() * sizeof(float));
  std::memcpy(sin_t, s.data(), s.size() * sizeof(float));
}

void* ref_bb_create(int max_tokens, int max_seqs, int max_rows, int max_blocks, int bs, int thr) {
  return new BatchBuilder(max_tokens, max_seqs, max_rows, max_blocks, bs, thr);
}
void ref_bb_destroy(void* b) { delete static_cast<BatchBuilder*>(b); }
size_t ref_bb_max_meta_words(void* b) { return static_cast<BatchBuilder*>(b)->max_meta_words(); }

// Returns the first logits row (>= -1), or -2 when the reference threw.
int ref_bb_add(void* b, const int32_t* tokens, int start_pos, int n, const int32_t* src_rows,
               const int32_t* blocks, int num_blocks, float temperature, int top_k, float top_p,
               uint64_t seed, int mode) {
  SamplingParams sp;
  sp.temperature = temperature;
  sp.top_k = top_k;
  sp.top_p = top_p;
  sp.seed = seed;
  const LogitsMode m = mode == 0 ? LogitsMode::kNone : (mode == 1 ? LogitsMode::kLast : LogitsMode::kAll);
  try {
    return static_cast<BatchBuilder*>(b)->add(tokens, start_pos, n, src_rows,
                                              std::vector<int32_t>(blocks, blocks + num_blocks), sp, m);
  } catch (const std::exception&) {
    return -2;
  }
}

void ref_bb_pad_decode_to(void* b, int n) { static_cast<BatchBuilder*>(b)->pad_decode_to(n); }

void ref_bb_write(void* b, int32_t* dst, int* shape7) {
  const BatchShape s = static_cast<BatchBuilder*>(b)->write(dst);
  const int v[7] = {s.num_tokens, s.num_seqs, s.num_logit_rows, s.num_decode_items,
                    s.num_prefill_seqs, s.max_prefill_q_tiles, s.max_context};
  std::memcpy(shape7, v, sizeof(v));
}

void ref_meta_layout(const int* shape7, int max_blocks, size_t* out19) {
  BatchShape s;
  s.num_tokens = shape7[0];
  s.num_seqs = shape7[1];
  s.num_logit_rows = shape7[2];
  s.num_decode_items = shape7[3];
  s.num_prefill_seqs = shape7[4];
  s.max_prefill_q_tiles = shape7[5];
  s.max_context = shape7[6];
  const MetaLayout m = MetaLayout::make(s, max_blocks);
  const size_t v[19] = {m.input_ids,   m.input_src,   m.positions,    m.slot_mapping,
                        m.seq_q_start, m.seq_q_len,   m.seq_ctx_len,  m.block_tables,
                        m.decode_token, m.decode_seq, m.prefill_seq,  m.logit_token,
                        m.param_row,   m.temperature, m.top_k,        m.top_p,
                        m.seed_lo,     m.seed_hi,     m.total_words};
  std::memcpy(out19, v, sizeof(v));
}

// The reference's model config JSON (ModelConfig::to_json) for tiny_test_config
// with the given dimensions, FP16 weights (int4 = 0) or INT4 layer weights
// (int4 = 1, group size 64); returns its length, or -1 when it does not fit
// `cap` bytes or the reference rejects the config.
int ref_model_config_json(int vocab, int hidden, int inter, int layers, int heads, int kv_heads,
                          int head_dim, double theta, double eps, int int4, char* buf, int cap) {
  try {
    ModelConfig c = tiny_test_config(int4 ? QuantType::kINT4 : QuantType::kFP16);
    c.vocab_size = vocab;
    c.hidden_size = hidden;
    c.intermediate_size = inter;
    c.num_layers = layers;
    c.num_heads = heads;
    c.num_kv_heads = kv_heads;
    c.head_dim = head_dim;
    c.rope_theta = theta;
    c.rms_norm_eps = eps;
    c.validate();
    const std::string s = c.to_json().dump();
    if (static_cast<int>(s.size()) + 1 > cap) return -1;
    std::memcpy(buf, s.c_str(), s.size() + 1);
    return static_cast<int>(s.size());
  } catch (const std::exception&) {
    return -1;
  }
}

// Logits [n, vocab] of the reference's fp32 CPU model (CpuReferenceModel::
// forward, src/cpu/reference_model.cpp:157-238) on a model file; 0 on success.
int ref_model_forward(const char* path, const int32_t* tokens, int n, float* logits) {
  try {
    CpuReferenceModel m(path);
    const std::vector<float> out = m.forward(std::vector<int32_t>(tokens, tokens + n));
    std::memcpy(logits, out.data(), out.size() * sizeof(float));
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

// The reference's weight quantisers (src/cpu/random_model.cpp:99-140): w is
// fp32 [n, k]; outputs are sized by the caller.
void ref_quantize_int8_rows(const float* w, int n, int k, int8_t* q, uint16_t* scales) {
  std::vector<int8_t> qv;
  std::vector<uint16_t> sv;
  quantize_int8_rows(std::vector<float>(w, w + static_cast<size_t>(n) * k), n, k, &qv, &sv);
  std::memcpy(q, qv.data(), qv.size());
  std::memcpy(scales, sv.data(), sv.size() * 2);
}

void ref_quantize_int4_groups(const float* w, int n, int k, int group_size, uint8_t* packed,
                              uint16_t* scales, uint16_t* offsets) {
  std::vector<uint8_t> pv;
  std::vector<uint16_t> sv, ov;
  quantize_int4_groups(std::vector<float>(w, w + static_cast<size_t>(n) * k), n, k, group_size,
                       &pv, &sv, &ov);
  std::memcpy(packed, pv.data(), pv.size());
  std::memcpy(scales, sv.data(), sv.size() * 2);
  std::memcpy(offsets, ov.data(), ov.size() * 2);
}

}  // extern "C"
