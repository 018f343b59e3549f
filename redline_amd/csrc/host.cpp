// Host-side pieces of the path: fp16 bit conversion, RoPE inverse frequencies
// and cos/sin tables, and the per-step batch metadata (BatchBuilder) whose
// positions / slot_mapping arrays drive the kernels.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <new>
#include <vector>

#include "redline_amd/rlk.h"
#include "status.hpp"

using rlk::fail;

// ------------------------------------------------------------------ fp16 bits

// IEEE binary16 -> binary32 (exact).  Follows the contract of
// redline::half_bits_to_float (src/core/common.cpp:37-62).
extern "C" float rlk_half_bits_to_float(uint16_t h) {
  const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu;
  const uint32_t m = h & 0x3ffu;
  uint32_t out;
  if (e == 0x1f) {
    out = sign | 0x7f800000u | (m << 13);
  } else if (e != 0) {
    out = sign | ((e + 112u) << 23) | (m << 13);
  } else if (m == 0) {
    out = sign;
  } else {
    // Subnormal: m * 2^-24, exact in binary32.
    float f = std::ldexp(static_cast<float>(m), -24);
    std::memcpy(&out, &f, 4);
    out |= sign;
  }
  float f;
  std::memcpy(&f, &out, 4);
  return f;
}

// binary32 -> binary16 with round-to-nearest-even; overflow gives inf, NaN
// stays a quiet NaN.  Follows redline::float_to_half_bits (common.cpp:64-89).
extern "C" uint16_t rlk_float_to_half_bits(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint16_t sign = static_cast<uint16_t>((x >> 16) & 0x8000u);
  const uint32_t mag = x & 0x7fffffffu;
  if (mag > 0x7f800000u) return sign | 0x7e00u;  // NaN
  if (mag == 0x7f800000u) return sign | 0x7c00u;  // inf
  const int exp = static_cast<int>(mag >> 23) - 127;
  if (exp >= 16) return sign | 0x7c00u;
  // Place the value on the fp16 grid as an integer multiple of its ulp and
  // round the discarded bits half-to-even.
  uint32_t mant = (mag & 0x7fffffu) | (mag >= 0x00800000u ? 0x800000u : 0u);
  int shift;  // bits to drop from the 24-bit significand
  uint32_t biased;
  if (exp >= -14) {  // normal fp16
    shift = 13;
    biased = static_cast<uint32_t>(exp + 15);
  } else {  // subnormal fp16 (or underflow to zero)
    shift = 13 + (-14 - exp);
    biased = 0;
    if (shift > 24) return sign;
  }
  uint32_t q = mant >> shift;
  const uint32_t rem = mant & ((1u << shift) - 1u);
  const uint32_t halfway = 1u << (shift - 1);
  if (rem > halfway || (rem == halfway && (q & 1u))) ++q;
  // For normals q carries the implicit bit (0x400); adding the exponent field
  // lets a mantissa overflow roll into the next exponent (or into inf).
  const uint32_t bits = biased == 0 ? q : ((biased << 10) + (q - 0x400u));
  return static_cast<uint16_t>(sign | bits);
}

// ----------------------------------------------------------------- RoPE tables

// inv[i] = theta^(-2i/D) in double, then the optional scaling: linear divides
// every frequency by `factor`; llama3 leaves wavelengths shorter than
// old_ctx/high_freq_factor alone, divides those longer than
// old_ctx/low_freq_factor by `factor` and blends linearly in between
// (semantics of redline::rope_inv_freq, src/core/model_config.cpp:126-153).
extern "C" int rlk_rope_inv_freq(double theta, int head_dim, int scaling_type, double factor,
                                 double low_freq_factor, double high_freq_factor,
                                 int original_max_position_embeddings, double* inv_freq) {
  if (head_dim <= 0 || head_dim % 2 != 0)
    return fail(RLK_EINVAL, "rope_inv_freq: head_dim must be even (got %d)", head_dim);
  if (scaling_type < 0 || scaling_type > 2)
    return fail(RLK_EINVAL, "rope_inv_freq: unknown scaling type %d", scaling_type);
  const int n = head_dim / 2;
  const double old_ctx = original_max_position_embeddings;
  const double long_wave = old_ctx / low_freq_factor;   // beyond: fully scaled
  const double short_wave = old_ctx / high_freq_factor;  // below: untouched
  for (int i = 0; i < n; ++i) {
    double f = 1.0 / std::pow(theta, (2.0 * i) / head_dim);
    if (scaling_type == 1) {
      f /= factor;
    } else if (scaling_type == 2) {
      const double wavelen = 2.0 * M_PI / f;
      if (wavelen > long_wave) {
        f /= factor;
      } else if (wavelen >= short_wave) {
        const double t = (old_ctx / wavelen - low_freq_factor) / (high_freq_factor - low_freq_factor);
        f = (1.0 - t) * f / factor + t * f;
      }
    }
    inv_freq[i] = f;
  }
  return RLK_OK;
}

// cos/sin [max_pos, D/2]; the angle is formed in fp32 from the fp32-rounded
// frequency (model_config.cpp:155-169), and cos/sin are the C library's fp32
// functions.
extern "C" int rlk_rope_cos_sin_tables(double theta, int head_dim, int scaling_type,
                                       double factor, double low_freq_factor,
                                       double high_freq_factor,
                                       int original_max_position_embeddings, int max_pos,
                                       float* cos_table, float* sin_table) {
  if (max_pos < 0) return fail(RLK_EINVAL, "rope_cos_sin_tables: negative max_pos");
  if (head_dim <= 0 || head_dim % 2 != 0)
    return fail(RLK_EINVAL, "rope_cos_sin_tables: head_dim must be even (got %d)", head_dim);
  const int n = head_dim / 2;
  std::vector<double> inv(n);
  const int st = rlk_rope_inv_freq(theta, head_dim, scaling_type, factor, low_freq_factor,
                                   high_freq_factor, original_max_position_embeddings, inv.data());
  if (st != RLK_OK) return st;
  std::vector<float> inv32(n);
  for (int i = 0; i < n; ++i) inv32[i] = static_cast<float>(inv[i]);
  for (int p = 0; p < max_pos; ++p) {
    const float pf = static_cast<float>(p);
    float* c = cos_table + static_cast<size_t>(p) * n;
    float* s = sin_table + static_cast<size_t>(p) * n;
    for (int i = 0; i < n; ++i) {
      const float angle = pf * inv32[i];
      c[i] = cosf(angle);
      s[i] = sinf(angle);
    }
  }
  return RLK_OK;
}

// -------------------------------------------------------------- batch metadata

// Word offsets of the arrays in the one int32 metadata buffer, in the order of
// redline::MetaLayout::make (src/core/batch_builder.cpp:17-46); DeviceBatch
// binds the same offsets on the device side.
extern "C" int rlk_meta_layout_make(const rlk_batch_shape* s, int max_blocks_per_seq,
                                    rlk_meta_layout* m) {
  if (s == nullptr || m == nullptr || max_blocks_per_seq < 0)
    return fail(RLK_EINVAL, "meta_layout_make: bad arguments");
  const size_t T = static_cast<size_t>(s->num_tokens), S = static_cast<size_t>(s->num_seqs);
  const size_t R = static_cast<size_t>(s->num_logit_rows);
  const size_t sizes[] = {T, T, T, T, S, S, S, S * static_cast<size_t>(max_blocks_per_seq),
                          static_cast<size_t>(s->num_decode_items),
                          static_cast<size_t>(s->num_decode_items),
                          static_cast<size_t>(s->num_prefill_seqs), R, R, S, S, S, S, S};
  size_t* fields[] = {&m->input_ids,   &m->input_src,   &m->positions,   &m->slot_mapping,
                      &m->seq_q_start, &m->seq_q_len,   &m->seq_ctx_len, &m->block_tables,
                      &m->decode_token, &m->decode_seq, &m->prefill_seq, &m->logit_token,
                      &m->param_row,   &m->temperature, &m->top_k,       &m->top_p,
                      &m->seed_lo,     &m->seed_hi};
  size_t at = 0;
  for (size_t i = 0; i < sizeof(sizes) / sizeof(sizes[0]); ++i) {
    *fields[i] = at;
    at += sizes[i];
  }
  m->total_words = at;
  return RLK_OK;
}

namespace {
// Query-tile height of the reference's prefill attention (kBatchPrefillTileQ,
// src/core/batch_builder.h:41); it sets max_prefill_q_tiles.
constexpr int kPrefillTileQ = 32;
}  // namespace

// One step's worth of per-token and per-sequence metadata, built on the host.
// Semantics of redline::BatchBuilder (src/core/batch_builder.cpp:48-188):
// tokens of a sequence segment get positions start..start+n-1 and KV slots
// blocks[pos / bs] * bs + pos % bs; sequences adding at most
// `decode_query_threshold` tokens become decode work items, longer ones
// prefill sequences.
struct rlk_batch_builder {
  int max_tokens, max_seqs, max_logit_rows, max_blocks, block_size, decode_threshold;
  std::vector<int32_t> ids, src, pos, slot;              // per token
  std::vector<int32_t> q_start, q_len, ctx_len, tables;  // per sequence
  std::vector<int32_t> logit_token, param_row;           // per logits row
  std::vector<float> temperature, top_p;                 // per sequence
  std::vector<int32_t> top_k;
  std::vector<uint32_t> seed_lo, seed_hi;

  int num_tokens() const { return static_cast<int>(ids.size()); }
  int num_seqs() const { return static_cast<int>(q_start.size()); }
  int num_rows() const { return static_cast<int>(logit_token.size()); }

  rlk_batch_shape shape() const {
    rlk_batch_shape s{};
    s.num_tokens = num_tokens();
    s.num_seqs = num_seqs();
    s.num_logit_rows = num_rows();
    for (int i = 0; i < num_seqs(); ++i) {
      if (q_len[i] <= decode_threshold) {
        s.num_decode_items += q_len[i];
      } else {
        ++s.num_prefill_seqs;
        s.max_prefill_q_tiles =
            std::max(s.max_prefill_q_tiles, (q_len[i] + kPrefillTileQ - 1) / kPrefillTileQ);
      }
      s.max_context = std::max(s.max_context, ctx_len[i]);
    }
    return s;
  }
};

extern "C" rlk_batch_builder* rlk_batch_builder_create(int max_tokens, int max_seqs,
                                                       int max_logit_rows, int max_blocks_per_seq,
                                                       int block_size,
                                                       int decode_query_threshold) {
  if (max_tokens < 0 || max_seqs < 0 || max_logit_rows < 0 || max_blocks_per_seq < 0 ||
      block_size <= 0) {
    fail(RLK_EINVAL, "batch_builder_create: bad limits");
    return nullptr;
  }
  auto* b = new (std::nothrow) rlk_batch_builder();
  if (b == nullptr) return nullptr;
  b->max_tokens = max_tokens;
  b->max_seqs = max_seqs;
  b->max_logit_rows = max_logit_rows;
  b->max_blocks = max_blocks_per_seq;
  b->block_size = block_size;
  b->decode_threshold = decode_query_threshold;
  return b;
}

extern "C" void rlk_batch_builder_destroy(rlk_batch_builder* b) { delete b; }

extern "C" void rlk_batch_builder_reset(rlk_batch_builder* b) {
  if (b == nullptr) return;
  for (auto* v : {&b->ids, &b->src, &b->pos, &b->slot, &b->q_start, &b->q_len, &b->ctx_len,
                  &b->tables, &b->logit_token, &b->param_row, &b->top_k})
    v->clear();
  b->temperature.clear();
  b->top_p.clear();
  b->seed_lo.clear();
  b->seed_hi.clear();
}

extern "C" size_t rlk_batch_builder_max_meta_words(const rlk_batch_builder* b) {
  if (b == nullptr) return 0;
  // Worst case of every array at once: all tokens decode items, all
  // sequences prefill sequences.
  rlk_batch_shape s{};
  s.num_tokens = b->max_tokens;
  s.num_seqs = b->max_seqs;
  s.num_logit_rows = b->max_logit_rows;
  s.num_decode_items = b->max_tokens;
  s.num_prefill_seqs = b->max_seqs;
  rlk_meta_layout m;
  rlk_meta_layout_make(&s, b->max_blocks, &m);
  return m.total_words;
}

extern "C" int rlk_batch_builder_add(rlk_batch_builder* b, const int32_t* tokens, int start_pos,
                                     int n, const int32_t* src_rows, const int32_t* blocks,
                                     int num_blocks, float temperature, int top_k, float top_p,
                                     uint64_t seed, int logits_mode, int* first_row) {
  if (first_row != nullptr) *first_row = -1;
  if (b == nullptr) return fail(RLK_EINVAL, "batch_builder_add: null builder");
  if (n < 1) return fail(RLK_EINVAL, "empty sequence segment");
  if (start_pos < 0) return fail(RLK_EINVAL, "negative start position %d", start_pos);
  if (b->num_tokens() + n > b->max_tokens)
    return fail(RLK_EINVAL, "batch exceeds max tokens (%d)", b->max_tokens);
  if (b->num_seqs() + 1 > b->max_seqs)
    return fail(RLK_EINVAL, "batch exceeds max sequences (%d)", b->max_seqs);
  if (num_blocks < 0 || num_blocks > b->max_blocks) return fail(RLK_EINVAL, "block table too long");
  if (blocks == nullptr && num_blocks > 0) return fail(RLK_EINVAL, "null block table");
  if (static_cast<int64_t>(num_blocks) * b->block_size < static_cast<int64_t>(start_pos) + n)
    return fail(RLK_EINVAL, "sequence has too few KV blocks for position %d", start_pos + n - 1);
  for (int i = 0; i < n; ++i) {
    if (!(src_rows != nullptr && src_rows[i] >= 0) && tokens == nullptr)
      return fail(RLK_EINVAL, "token %d has no source", i);
  }
  const int rows = logits_mode == RLK_LOGITS_NONE ? 0 : (logits_mode == RLK_LOGITS_ALL ? n : 1);
  if (b->num_rows() + rows > b->max_logit_rows)
    return fail(RLK_EINVAL, "batch exceeds max logits rows (%d)", b->max_logit_rows);

  const int seq = b->num_seqs();
  const int t0 = b->num_tokens();
  b->q_start.push_back(t0);
  b->q_len.push_back(n);
  b->ctx_len.push_back(start_pos + n);
  b->tables.insert(b->tables.end(), blocks, blocks + num_blocks);
  b->tables.resize(static_cast<size_t>(seq + 1) * b->max_blocks, 0);
  const int bs = b->block_size;
  for (int i = 0; i < n; ++i) {
    const int p = start_pos + i;
    const bool dev = src_rows != nullptr && src_rows[i] >= 0;
    b->ids.push_back(dev ? 0 : tokens[i]);
    b->src.push_back(dev ? src_rows[i] : -1);
    b->pos.push_back(p);
    b->slot.push_back(blocks[p / bs] * bs + p % bs);
  }
  if (rows > 0) {
    if (first_row != nullptr) *first_row = b->num_rows();
    for (int i = 0; i < rows; ++i) {
      b->logit_token.push_back(logits_mode == RLK_LOGITS_ALL ? t0 + i : t0 + n - 1);
      b->param_row.push_back(seq);
    }
  }
  b->temperature.push_back(temperature);
  b->top_k.push_back(top_k);
  b->top_p.push_back(top_p);
  b->seed_lo.push_back(static_cast<uint32_t>(seed & 0xffffffffu));
  b->seed_hi.push_back(static_cast<uint32_t>(seed >> 32));
  return RLK_OK;
}

// Dummy one-token greedy sequences at position 0 of the scratch block 0, so a
// decode batch reaches a fixed graph bucket size (batch_builder.cpp:124-129).
extern "C" int rlk_batch_builder_pad_decode_to(rlk_batch_builder* b, int num_seqs) {
  if (b == nullptr) return fail(RLK_EINVAL, "batch_builder_pad_decode_to: null builder");
  const int32_t tok = 0, scratch_block = 0;
  while (b->num_seqs() < num_seqs) {
    const int st = rlk_batch_builder_add(b, &tok, 0, 1, nullptr, &scratch_block, 1, 0.0f, 0, 1.0f,
                                         0, RLK_LOGITS_LAST, nullptr);
    if (st != RLK_OK) return st;
  }
  return RLK_OK;
}

extern "C" int rlk_batch_builder_shape(const rlk_batch_builder* b, rlk_batch_shape* shape) {
  if (b == nullptr || shape == nullptr) return fail(RLK_EINVAL, "batch_builder_shape: null argument");
  *shape = b->shape();
  return RLK_OK;
}

extern "C" int rlk_batch_builder_write(const rlk_batch_builder* b, int32_t* dst,
                                       rlk_batch_shape* shape_out) {
  if (b == nullptr || dst == nullptr) return fail(RLK_EINVAL, "batch_builder_write: null argument");
  const rlk_batch_shape s = b->shape();
  rlk_meta_layout m;
  rlk_meta_layout_make(&s, b->max_blocks, &m);
  auto put = [dst](size_t at, const void* src, size_t words) {
    if (words != 0) std::memcpy(dst + at, src, words * 4);
  };
  put(m.input_ids, b->ids.data(), b->ids.size());
  put(m.input_src, b->src.data(), b->src.size());
  put(m.positions, b->pos.data(), b->pos.size());
  put(m.slot_mapping, b->slot.data(), b->slot.size());
  put(m.seq_q_start, b->q_start.data(), b->q_start.size());
  put(m.seq_q_len, b->q_len.data(), b->q_len.size());
  put(m.seq_ctx_len, b->ctx_len.data(), b->ctx_len.size());
  put(m.block_tables, b->tables.data(), b->tables.size());
  size_t nd = 0, np = 0;
  for (int q = 0; q < b->num_seqs(); ++q) {
    if (b->q_len[q] <= b->decode_threshold) {
      for (int i = 0; i < b->q_len[q]; ++i, ++nd) {
        dst[m.decode_token + nd] = b->q_start[q] + i;
        dst[m.decode_seq + nd] = q;
      }
    } else {
      dst[m.prefill_seq + np++] = q;
    }
  }
  put(m.logit_token, b->logit_token.data(), b->logit_token.size());
  put(m.param_row, b->param_row.data(), b->param_row.size());
  put(m.temperature, b->temperature.data(), b->temperature.size());
  put(m.top_k, b->top_k.data(), b->top_k.size());
  put(m.top_p, b->top_p.data(), b->top_p.size());
  put(m.seed_lo, b->seed_lo.data(), b->seed_lo.size());
  put(m.seed_hi, b->seed_hi.data(), b->seed_hi.size());
  if (shape_out != nullptr) *shape_out = s;
  return RLK_OK;
}
