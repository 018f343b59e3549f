/*
 * oracle.c — CPU restatement of Redline's fused per-layer kernels.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP kernels in
 * redline_amd/ are compared against (by tests/, __graft_entry__.smoke() and
 * the cpu_baseline leg of bench.py).  Nothing in the product links or calls it.
 *
 * Each function restates the reference's semantics, citing the file:line of
 * Neil456/Redline it follows.  fp16 values are IEEE binary16 bit patterns
 * (uint16_t).  Build with -ffp-contract=off and without -ffast-math: every
 * fp32 operation below is then rounded exactly as written.
 *
 * How each function is pinned (tests/test_oracle.py):
 *   orc_f2h / orc_h2f          exhaustive agreement with the compiled reference
 *                              host core (float_to_half_bits / half_bits_to_float)
 *                              plus the KATs of tests/cpp/test_core.cpp:97-112.
 *   orc_rope_cos_sin_tables    bit-exact against golden tables written by the
 *                              compiled reference (rope_cos_sin_tables) for
 *                              theta 1e4 / 5e5 / 1e6, D 64 / 128, llama3 scaling.
 *   orc_embedding_lookup       closed form (pure copy) on integer-valued rows.
 *   orc_fused_add_rmsnorm      float64 numpy restatement of reference_model.cpp:
 *                              145-155 within fp16 rounding, constant-row closed
 *                              form, delta == NULL reduction, residual bit-exact.
 *   orc_silu_and_mul(_interl.) scipy expit-based float64 silu within fp16
 *                              rounding, special values (0, large +/-), layout
 *                              equivalence of split vs interleaved.
 *   orc_rope_and_write_kv_ex   bias: equivalence with the plain function on
 *                              fp16(qkv + bias); fp16 scale: scale == fp16(amax/127)
 *                              and tie-masked float64 codes against the stored scale.
 *   orc_paged_attention_decode scipy softmax attention in float64 over the
 *                              gathered cache, q = 0 -> mean of V, a dominant key
 *                              -> its V, invariance under physical block moves,
 *                              INT8 == FP16 path on the dequantised cache.
 *   orc_paged_attention_prefill  numpy float64 causal softmax attention over the
 *                              gathered, fp16-dequantised cache; a one-token
 *                              chunk equals the decode oracle (FP16); the first
 *                              new token of an empty context returns its own V;
 *                              invariance under physical block moves.
 *   orc_gemv_w8a16             numpy float64 matmul of x and the int8 codes, then
 *                              scale and bias; a code KAT (-128, -1, 0, 1, 127:
 *                              two's complement bytes), zero weight -> bias, one-hot
 *                              x -> scaled column, scale linearity.
 *   orc_gemv_w4a16(_swiglu)    numpy float64 matmul against a weight matrix built
 *                              first and then packed (nibble order KAT from
 *                              tests/cuda/test_gemm.cu:40-45), q = 0 -> offset
 *                              * sum(x), one-hot x -> the dequantised column,
 *                              SwiGLU == orc_silu_and_mul_interleaved of the
 *                              fp16-rounded GEMV output.
 *   orc_rope_and_write_kv      pos 0 identity, V passthrough, rotation by angle
 *                              against float64 rotation matrix, norm
 *                              preservation, slot/cell address KATs from
 *                              tests/cpp/test_core.cpp:365-367, INT8 bounds of
 *                              tests/cuda/test_kernels.cu:318-321, amax 0 -> 1.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------ fp16 bits */

/* Exact binary16 -> binary32 through the value formula
 * (-1)^s * 2^(e-15) * (1 + m/1024), or m * 2^-24 for subnormals. */
float orc_h2f(uint16_t h) {
  const int s = h >> 15, e = (h >> 10) & 31, m = h & 1023;
  float v;
  if (e == 31) {
    v = m ? NAN : INFINITY;
  } else if (e == 0) {
    v = ldexpf((float)m, -24);
  } else {
    v = ldexpf((float)(1024 + m), e - 25);
  }
  return s ? -v : v;
}

/* binary32 -> binary16, round to nearest, ties to even, following the
 * reference's float_to_half_bits (src/core/common.cpp:64-89): the value is
 * scaled to an integer count of fp16 ulps in double and rounded with rint()
 * (the default rounding mode is nearest-even). */
uint16_t orc_f2h(float f) {
  uint16_t sign = signbit(f) ? 0x8000 : 0;
  if (isnan(f)) return sign | 0x7e00;
  double a = fabs((double)f);
  if (a >= 65520.0) return sign | 0x7c00; /* rounds past the largest finite half */
  if (a < ldexp(1.0, -14)) {              /* subnormal range: ulp 2^-24 */
    double q = rint(a * ldexp(1.0, 24));  /* exact scaling, then RNE */
    return sign | (uint16_t)q;           /* q == 1024 is the smallest normal */
  }
  int e;
  frexp(a, &e);                       /* a = mant * 2^e, mant in [0.5, 1) */
  int ulp_exp = e - 11;               /* 11 significant bits */
  double q = rint(ldexp(a, -ulp_exp)); /* in [1024, 2048] */
  int be = e - 1 + 15;
  if (q == 2048.0) {
    q = 1024.0;
    be += 1;
  }
  if (be >= 31) return sign | 0x7c00;
  return sign | (uint16_t)((be << 10) | ((int)q - 1024));
}

static inline float rnd16(float x) { return orc_h2f(orc_f2h(x)); }

/* ------------------------------------------------------------ RoPE tables */

/* inv[i] = 1 / theta^(2i/D) in double with linear / llama3 scaling
 * (model_config.cpp:126-153); angle = (float)p * (float)inv[i] in fp32;
 * cos/sin in fp32 via the C library (model_config.cpp:155-169). */
void orc_rope_cos_sin_tables(double theta, int D, int scaling, double factor, double lo_ff,
                             double hi_ff, int old_ctx_i, int max_pos, float* cos_t,
                             float* sin_t) {
  const int half = D / 2;
  const double old_ctx = (double)old_ctx_i;
  for (int i = 0; i < half; ++i) {
    double inv = 1.0 / pow(theta, (2.0 * i) / D);
    if (scaling == 1) {
      inv = inv / factor;
    } else if (scaling == 2) {
      const double wl = 2.0 * M_PI / inv;
      if (wl < old_ctx / hi_ff) {
        /* high frequency: unchanged */
      } else if (wl > old_ctx / lo_ff) {
        inv = inv / factor;
      } else {
        const double sm = (old_ctx / wl - lo_ff) / (hi_ff - lo_ff);
        inv = (1.0 - sm) * inv / factor + sm * inv;
      }
    }
    const float invf = (float)inv;
    for (int p = 0; p < max_pos; ++p) {
      const float ang = (float)p * invf;
      cos_t[(size_t)p * half + i] = cosf(ang);
      sin_t[(size_t)p * half + i] = sinf(ang);
    }
  }
}

/* ------------------------------------------------------------ elementwise */

/* out[t, :] = table[ids[t], :]  (elementwise.cu:19-24; reference_model.cpp:167). */
void orc_embedding_lookup(const int32_t* ids, const uint16_t* table, int n, int hidden,
                          uint16_t* out) {
  for (int t = 0; t < n; ++t)
    memcpy(out + (size_t)t * hidden, table + (size_t)ids[t] * hidden, (size_t)hidden * 2);
}

/* dst[i, :] = src[idx[i], :]  (elementwise.cu:84-89). */
void orc_gather_rows(const uint16_t* src, const int32_t* idx, int n, int cols, uint16_t* dst) {
  orc_embedding_lookup(idx, src, n, cols, dst);
}

/* ids[i] = prev[src[i]] where src[i] >= 0  (elementwise.cu:12-16). */
void orc_resolve_input_ids(int32_t* ids, const int32_t* src, const int32_t* prev, int n) {
  for (int i = 0; i < n; ++i)
    if (src[i] >= 0) ids[i] = prev[src[i]];
}

/* Fused residual add + RMSNorm with the kernel's fp16 rounding points
 * (elementwise.cu:29-64), in the form of the reference's own CPU restatement
 * (tests/cuda/test_kernels.cu:26-39): r = fp16(res + delta); ss summed in
 * double; inv = 1 / sqrtf((float)(ss / H) + eps); out = fp16(fp16(r * inv) * w). */
void orc_fused_add_rmsnorm(uint16_t* residual, const uint16_t* delta, const uint16_t* weight,
                           int rows, int hidden, float eps, uint16_t* out) {
  for (int r = 0; r < rows; ++r) {
    uint16_t* res = residual + (size_t)r * hidden;
    double ss = 0.0;
    for (int c = 0; c < hidden; ++c) {
      float x = orc_h2f(res[c]);
      if (delta) {
        x = rnd16(x + orc_h2f(delta[(size_t)r * hidden + c]));
        res[c] = orc_f2h(x);
      }
      ss += (double)x * x;
    }
    const float inv = 1.0f / sqrtf((float)(ss / hidden) + eps);
    for (int c = 0; c < hidden; ++c) {
      const float y = rnd16(orc_h2f(res[c]) * inv) * orc_h2f(weight[c]);
      out[(size_t)r * hidden + c] = orc_f2h(y);
    }
  }
}

/* silu(g) rounded to fp16, times up, rounded (elementwise.cu:66-82, 123-131;
 * unrounded form reference_model.cpp:224-230). */
static inline uint16_t swiglu1(float g, float u) {
  const float s = rnd16(g / (1.0f + expf(-g)));
  return orc_f2h(s * u);
}

void orc_silu_and_mul(const uint16_t* gate_up, int rows, int inter, uint16_t* out) {
  for (int r = 0; r < rows; ++r) {
    const uint16_t* g = gate_up + (size_t)r * 2 * inter;
    for (int i = 0; i < inter; ++i)
      out[(size_t)r * inter + i] = swiglu1(orc_h2f(g[i]), orc_h2f(g[inter + i]));
  }
}

void orc_silu_and_mul_interleaved(const uint16_t* gate_up, int rows, int inter, uint16_t* out) {
  for (int r = 0; r < rows; ++r) {
    const uint16_t* g = gate_up + (size_t)r * 2 * inter;
    for (int i = 0; i < inter; ++i)
      out[(size_t)r * inter + i] = swiglu1(orc_h2f(g[2 * i]), orc_h2f(g[2 * i + 1]));
  }
}

/* ------------------------------------------------------ INT8 weight-only GEMV */

/* y[m, n] = (x[m, k] . W[n, k]^T) * scale[n] (+ bias[n]), W int8 row-major with
 * one fp16 scale per row: the reference sums x * code in fp32 over K and applies
 * the per-channel scale and the bias once, to the sum (gemv_weight_only.cu:64-93,
 * store_outputs :19-44 with per_channel_scale; weight layout and scales from
 * quantize_int8_rows, random_model.cpp:99-115).  Every product and sum here is
 * float64, so y is the exact value the kernels approximate. */
void orc_gemv_w8a16(const uint16_t* x, int m, const int8_t* w, const uint16_t* scales,
                    const uint16_t* bias, int n, int k, double* y) {
  double* xs = (double*)malloc(sizeof(double) * (size_t)k);
  for (int i = 0; i < m; ++i) {
    for (int c = 0; c < k; ++c) xs[c] = orc_h2f(x[(size_t)i * k + c]);
    for (int r = 0; r < n; ++r) {
      const int8_t* row = w + (size_t)r * k;
      double acc = 0.0;
      for (int c = 0; c < k; ++c) acc += xs[c] * (double)row[c];
      y[(size_t)i * n + r] = acc * orc_h2f(scales[r]) + (bias ? orc_h2f(bias[r]) : 0.0);
    }
  }
  free(xs);
}

/* ------------------------------------------------------ INT4 weight-only GEMV */

/* y[m, n] = x[m, k] . W[n, k]^T (+ bias) with W dequantised group-wise:
 *   W[r][c] = q * scale[r][c / g] + offset[r][c / g],  q = nibble c of row r,
 * nibble c held in byte c / 2 of the row, low nibble for even c
 * (gemv_weight_only.cu:103-160, packing tests/cuda/test_gemm.cu:40-45,
 * python/redline/quantize.py:4,84-86).  The reference evaluates the group sum as
 * s * sum(x q) + o * sum(x) in fp32; here every product and sum is float64, so
 * y is the exact value the kernels approximate. */
void orc_gemv_w4a16(const uint16_t* x, int m, const uint8_t* w, const uint16_t* scales,
                    const uint16_t* offsets, int group_size, const uint16_t* bias, int n, int k,
                    double* y) {
  const int groups = k / group_size;
  double* xs = (double*)malloc(sizeof(double) * (size_t)k);
  for (int i = 0; i < m; ++i) {
    for (int c = 0; c < k; ++c) xs[c] = orc_h2f(x[(size_t)i * k + c]);
    for (int r = 0; r < n; ++r) {
      const uint8_t* row = w + (size_t)r * (k / 2);
      double acc = bias ? orc_h2f(bias[r]) : 0.0;
      for (int gi = 0; gi < groups; ++gi) {
        const double s = orc_h2f(scales[(size_t)r * groups + gi]);
        const double o = orc_h2f(offsets[(size_t)r * groups + gi]);
        for (int c = gi * group_size; c < (gi + 1) * group_size; ++c) {
          const int q = (c & 1) ? (row[c / 2] >> 4) : (row[c / 2] & 15);
          acc += xs[c] * (q * s + o);
        }
      }
      y[(size_t)i * n + r] = acc;
    }
  }
  free(xs);
}

/* The SwiGLU epilogue over interleaved (gate_i, up_i) rows 2i, 2i + 1, fp16
 * out [m, n / 2], with the rounding points of the unfused path: gate and up
 * rounded to fp16 as GEMM outputs, then silu rounded, then the product
 * (gemv_weight_only.cu:46-63, row interleave weights.cpp:157-167). */
void orc_gemv_w4a16_swiglu(const uint16_t* x, int m, const uint8_t* w, const uint16_t* scales,
                           const uint16_t* offsets, int group_size, int n, int k, uint16_t* y) {
  double* acc = (double*)malloc(sizeof(double) * (size_t)m * n);
  orc_gemv_w4a16(x, m, w, scales, offsets, group_size, NULL, n, k, acc);
  for (int i = 0; i < m; ++i)
    for (int j = 0; j < n / 2; ++j) {
      const float g = rnd16((float)acc[(size_t)i * n + 2 * j]);
      const float u = rnd16((float)acc[(size_t)i * n + 2 * j + 1]);
      y[(size_t)i * (n / 2) + j] = swiglu1(g, u);
    }
  free(acc);
}

/* ------------------------------------------------------------- rope / kv */

/* RoPE + paged KV write (rope_kv.cu:13-87):
 *   q and k heads: pairs (i, i + D/2) -> a = x0*c - x1*s, b = x1*c + x0*s, each
 *   rounded to fp16; q written back in place; the k section of qkv is NOT
 *   written back (only the cache receives roped k); v heads pass unchanged.
 *   slot = slot_mapping[t] < 0: no KV write.  Cell
 *   ((slot / bs * Hkv + kvh) * bs + slot % bs) * D  (rope_kv.cu:60-64).
 *   INT8: amax over the head's fp16-rounded values, scale = amax > 0 ?
 *   amax / 127 : 1, inv = 1 / scale, code = rint(clamp(x * inv, -127, 127))
 *   (rope_kv.cu:71-85), scales fp32 per cell. */
void orc_rope_and_write_kv_ex(uint16_t* qkv, const int32_t* positions, const int32_t* slots,
                              int T, int Hq, int Hkv, int D, const float* cos_t,
                              const float* sin_t, void* k_cache, void* v_cache, void* k_scale,
                              void* v_scale, int bs, int int8, const uint16_t* bias,
                              int scale16) {
  const int half = D / 2, heads = Hq + 2 * Hkv;
  float x[256];
  for (int t = 0; t < T; ++t) {
    const int pos = positions[t], slot = slots[t];
    uint16_t* row = qkv + (size_t)t * heads * D;
    for (int h = 0; h < heads; ++h) {
      uint16_t* v = row + (size_t)h * D;
      for (int i = 0; i < D; ++i) x[i] = orc_h2f(v[i]);
      if (bias) /* extension: QKV bias added before the rotation, fp16-rounded */
        for (int i = 0; i < D; ++i) x[i] = rnd16(x[i] + orc_h2f(bias[h * D + i]));
      if (h < Hq + Hkv) {
        for (int i = 0; i < half; ++i) {
          const float c = cos_t[(size_t)pos * half + i], s = sin_t[(size_t)pos * half + i];
          const float x0 = x[i], x1 = x[i + half];
          const float a = x0 * c - x1 * s;
          const float b = x1 * c + x0 * s;
          x[i] = rnd16(a);
          x[i + half] = rnd16(b);
        }
      }
      if (h < Hq) {
        for (int i = 0; i < D; ++i) v[i] = orc_f2h(x[i]);
        continue;
      }
      if (slot < 0) continue;
      const int is_v = h >= Hq + Hkv;
      const int kvh = is_v ? h - Hq - Hkv : h - Hq;
      const int blk = slot / bs, off = slot % bs;
      const size_t cell = ((size_t)blk * Hkv + kvh) * bs + off;
      if (!int8) {
        uint16_t* dst = (uint16_t*)(is_v ? v_cache : k_cache) + cell * D;
        for (int i = 0; i < D; ++i) dst[i] = orc_f2h(x[i]);
      } else {
        float amax = 0.0f;
        for (int i = 0; i < D; ++i) amax = fmaxf(amax, fabsf(x[i]));
        float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
        /* extension: fp16-stored scale, codes quantised against the stored
         * value (the reference's host quantiser convention,
         * src/cpu/random_model.cpp:107-108) */
        if (scale16) scale = rnd16(scale);
        const float inv = 1.0f / scale;
        int8_t* dst = (int8_t*)(is_v ? v_cache : k_cache) + cell * D;
        for (int i = 0; i < D; ++i) dst[i] = (int8_t)rintf(fminf(fmaxf(x[i] * inv, -127.0f), 127.0f));
        if (scale16)
          ((uint16_t*)(is_v ? v_scale : k_scale))[cell] = orc_f2h(scale);
        else
          ((float*)(is_v ? v_scale : k_scale))[cell] = scale;
      }
    }
  }
}

void orc_rope_and_write_kv(uint16_t* qkv, const int32_t* positions, const int32_t* slots, int T,
                           int Hq, int Hkv, int D, const float* cos_t, const float* sin_t,
                           void* k_cache, void* v_cache, float* k_scale, float* v_scale, int bs,
                           int int8) {
  orc_rope_and_write_kv_ex(qkv, positions, slots, T, Hq, Hkv, D, cos_t, sin_t, k_cache, v_cache,
                           k_scale, v_scale, bs, int8, NULL, 0);
}

/* Paged decode attention (attention.cu:70-210): item i's token t attends to
 * positions [0, positions[t]] of sequence item_seq[i] through the block table;
 * query head h uses kv head h / (num_heads / Hkv).  Evaluated in double:
 * s_j = (q * scale) . k_j (k dequantised as code * k_scale for INT8),
 * p = softmax(s), out = fp16(sum_j p_j v_j).  The kernel's split-K partition
 * merge is an exact identity of this formula and has no counterpart here. */
void orc_paged_attention_decode(const uint16_t* q, int q_stride, uint16_t* out, int num_heads,
                                float scale, const void* k_cache, const void* v_cache,
                                const float* k_scale, const float* v_scale, int bs, int Hkv,
                                int D, int int8, const int32_t* block_tables, int max_blocks,
                                const int32_t* positions, const int32_t* item_token,
                                const int32_t* item_seq, int num_items) {
  const int G = num_heads / Hkv;
  for (int it = 0; it < num_items; ++it) {
    const int t = item_token[it], seq = item_seq[it];
    const int ctx = positions[t] + 1;
    const int32_t* table = block_tables + (size_t)seq * max_blocks;
    double* s = (double*)malloc(sizeof(double) * (size_t)ctx);
    double acc[256];
    for (int h = 0; h < num_heads; ++h) {
      const int kvh = h / G;
      const uint16_t* qh = q + (size_t)t * q_stride + (size_t)h * D;
      double mx = -INFINITY;
      for (int j = 0; j < ctx; ++j) {
        const size_t cell = ((size_t)table[j / bs] * Hkv + kvh) * bs + j % bs;
        double dot = 0.0;
        for (int d = 0; d < D; ++d) {
          const double kv = int8 ? (double)((const int8_t*)k_cache)[cell * D + d] * k_scale[cell]
                                 : (double)orc_h2f(((const uint16_t*)k_cache)[cell * D + d]);
          dot += (double)orc_h2f(qh[d]) * (double)scale * kv;
        }
        s[j] = dot;
        if (dot > mx) mx = dot;
      }
      double den = 0.0;
      for (int d = 0; d < D; ++d) acc[d] = 0.0;
      for (int j = 0; j < ctx; ++j) {
        const double e = exp(s[j] - mx);
        den += e;
        const size_t cell = ((size_t)table[j / bs] * Hkv + kvh) * bs + j % bs;
        for (int d = 0; d < D; ++d) {
          const double vv = int8 ? (double)((const int8_t*)v_cache)[cell * D + d] * v_scale[cell]
                                 : (double)orc_h2f(((const uint16_t*)v_cache)[cell * D + d]);
          acc[d] += e * vv;
        }
      }
      for (int d = 0; d < D; ++d)
        out[(size_t)t * num_heads * D + (size_t)h * D + d] = orc_f2h((float)(acc[d] / den));
    }
    free(s);
  }
}

/* Paged prefill attention (attention.cu:210-360, launcher :399-408, entry
 * :423-431): sequence seq_ids[z] has q_len new tokens, query rows
 * q_start .. q_start + q_len - 1, and ctx_len keys after this step; new token i
 * sits at position past + i (past = ctx_len - q_len) and attends to positions
 * [0, past + i] through the block table.  INT8 K and V are dequantised the way
 * the reference's tile loader does it, fp16(float(code) * scale) (:266-274),
 * and FP16 ones are read as they are.  Evaluated in double:
 * s_j = (q . k_j) * scale, p = softmax(s), out = fp16(sum_j p_j v_j).  The
 * kernel's tiling and online softmax are exact identities of this formula. */
static double prefill_kv(const void* cache, const float* scl, size_t cell, int D, int d, int int8) {
  if (!int8) return (double)orc_h2f(((const uint16_t*)cache)[cell * D + d]);
  const float x = (float)((const int8_t*)cache)[cell * D + d] * scl[cell];
  return (double)orc_h2f(orc_f2h(x));
}

void orc_paged_attention_prefill(const uint16_t* q, int q_stride, uint16_t* out, int num_heads,
                                 float scale, const void* k_cache, const void* v_cache,
                                 const float* k_scale, const float* v_scale, int bs, int Hkv,
                                 int D, int int8, const int32_t* block_tables, int max_blocks,
                                 const int32_t* seq_ids, const int32_t* q_start,
                                 const int32_t* q_len, const int32_t* ctx_len, int num_seqs) {
  const int G = num_heads / Hkv;
  for (int z = 0; z < num_seqs; ++z) {
    const int seq = seq_ids[z], n = q_len[seq], q0 = q_start[seq], ctx = ctx_len[seq];
    const int past = ctx - n;
    const int32_t* table = block_tables + (size_t)seq * max_blocks;
    double* s = (double*)malloc(sizeof(double) * (size_t)(ctx > 0 ? ctx : 1));
    double acc[256];
    for (int i = 0; i < n; ++i) {
      const int keys = past + i + 1;
      for (int h = 0; h < num_heads; ++h) {
        const int kvh = h / G;
        const uint16_t* qh = q + (size_t)(q0 + i) * q_stride + (size_t)h * D;
        double mx = -INFINITY;
        for (int j = 0; j < keys; ++j) {
          const size_t cell = ((size_t)table[j / bs] * Hkv + kvh) * bs + j % bs;
          double dot = 0.0;
          for (int d = 0; d < D; ++d)
            dot += (double)orc_h2f(qh[d]) * prefill_kv(k_cache, k_scale, cell, D, d, int8);
          s[j] = dot * (double)scale;
          if (s[j] > mx) mx = s[j];
        }
        double den = 0.0;
        for (int d = 0; d < D; ++d) acc[d] = 0.0;
        for (int j = 0; j < keys; ++j) {
          const double e = exp(s[j] - mx);
          den += e;
          const size_t cell = ((size_t)table[j / bs] * Hkv + kvh) * bs + j % bs;
          for (int d = 0; d < D; ++d) acc[d] += e * prefill_kv(v_cache, v_scale, cell, D, d, int8);
        }
        for (int d = 0; d < D; ++d)
          out[(size_t)(q0 + i) * num_heads * D + (size_t)h * D + d] = orc_f2h((float)(acc[d] / den));
      }
    }
    free(s);
  }
}

/* One layer's hot path on one batch, as a single call, in the reference's
 * forward-pass order (src/cuda/model/llama.cpp:79-80,122,131,139): embedding
 * gather into emb, RMSNorm of emb (no delta), RoPE + KV write, residual add +
 * RMSNorm (FFN input), SwiGLU. */
void orc_layer_step(const int32_t* ids, const uint16_t* table, int T, int H, uint16_t* emb,
                    uint16_t* residual, const uint16_t* delta, const uint16_t* w_norm, float eps,
                    uint16_t* normed, uint16_t* qkv, const int32_t* positions,
                    const int32_t* slots, int Hq, int Hkv, int D, const float* cos_t,
                    const float* sin_t, void* k_cache, void* v_cache, float* k_scale,
                    float* v_scale, int bs, int int8, const uint16_t* gate_up, int I,
                    uint16_t* act) {
  orc_embedding_lookup(ids, table, T, H, emb);
  orc_fused_add_rmsnorm(emb, NULL, w_norm, T, H, eps, normed);
  orc_rope_and_write_kv(qkv, positions, slots, T, Hq, Hkv, D, cos_t, sin_t, k_cache, v_cache,
                        k_scale, v_scale, bs, int8);
  orc_fused_add_rmsnorm(residual, delta, w_norm, T, H, eps, normed);
  orc_silu_and_mul(gate_up, T, I, act);
}
