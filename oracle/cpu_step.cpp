// Multi-threaded CPU port of one layer step of the fused per-layer kernels, in
// the reference's forward-pass order (src/cuda/model/llama.cpp:79-80,122,131,
// 139): embedding gather into `emb`, RMSNorm of that row (no delta), RoPE +
// paged-KV write, residual-add + RMSNorm, SwiGLU.  TEST INFRASTRUCTURE: it is the CPU baseline that
// bench.py times next to the GPU (and that tests/test_cpu_step.py checks
// against the oracle); nothing in the product path links or calls it.
//
// Per-op semantics are those of the reference's CPU path and kernels
// (Neil456/Redline): embedding = row copy (src/cpu/reference_model.cpp:167),
// RMSNorm with fp32 sum of squares and the kernels' fp16 rounding points
// (reference_model.cpp:145-155, src/cuda/kernels/elementwise.cu:45-61),
// rotation of pairs (i, i + D/2) in fp32 rounded to fp16 and the paged cell
// ((blk * Hkv + kvh) * block_size + off) * D (reference_model.cpp:174-182,
// src/cuda/kernels/rope_kv.cu:44-84), SwiGLU fp16(fp16(silu(g)) * u)
// (reference_model.cpp:224-230, elementwise.cu:77).
//
// Unlike oracle.c (which converts every fp16 through double-precision calls
// to stay obviously correct), this port converts 8 values per instruction with
// the x86 F16C unit (IEEE round-to-nearest-even, the same results), and splits
// every op over a persistent pool of std::threads by rows (tokens), or by
// ranges of 8-element groups for SwiGLU, whose exp is an AVX2 routine of its
// own (exp8: Cody-Waite reduction and a Taylor polynomial, about 1 ulp; the
// SwiGLU output stays within fp16 tolerance of the oracle's libm exp).
// Threads are pinned to the cores of the process's affinity mask
// (sched_getaffinity).
#include <immintrin.h>
#include <pthread.h>
#include <sched.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <condition_variable>
#include <cstdint>
#include <cstring>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

#pragma STDC FP_CONTRACT OFF

namespace {

inline __m256 load8h(const uint16_t* p) {
  return _mm256_cvtph_ps(_mm_loadu_si128(reinterpret_cast<const __m128i*>(p)));
}
inline void store8h(uint16_t* p, __m256 v) {
  _mm_storeu_si128(reinterpret_cast<__m128i*>(p), _mm256_cvtps_ph(v, _MM_FROUND_TO_NEAREST_INT));
}
inline __m256 round8h(__m256 v) {
  return _mm256_cvtph_ps(_mm256_cvtps_ph(v, _MM_FROUND_TO_NEAREST_INT));
}
inline float h2f(uint16_t h) { return _cvtsh_ss(h); }
inline uint16_t f2h(float f) { return _cvtss_sh(f, _MM_FROUND_TO_NEAREST_INT); }
inline float roundh(float f) { return h2f(f2h(f)); }

// Persistent pool: run(n, fn) calls fn(i) for i in [0, n) over the threads
// (the caller is thread 0) and returns when all are done.  An idle worker
// spins on the generation counter for a while (about a millisecond) before it
// sleeps on the condition variable, so back-to-back ops of a step are handed
// out in about a microsecond instead of a futex wake-up each.
class Pool {
 public:
  explicit Pool(int threads) : n_(std::max(1, threads)) {
    cpu_set_t set;
    std::vector<int> cores;
    if (sched_getaffinity(0, sizeof(set), &set) == 0) {
      for (int c = 0; c < CPU_SETSIZE; ++c)
        if (CPU_ISSET(c, &set)) cores.push_back(c);
    }
    for (int t = 1; t < n_; ++t) {
      workers_.emplace_back([this, t] { loop(t); });
      if (!cores.empty()) {
        cpu_set_t one;
        CPU_ZERO(&one);
        CPU_SET(cores[t % cores.size()], &one);
        pthread_setaffinity_np(workers_.back().native_handle(), sizeof(one), &one);
      }
    }
  }
  ~Pool() {
    {
      std::lock_guard<std::mutex> l(mu_);
      stop_ = true;
      gen_.fetch_add(1, std::memory_order_release);
    }
    cv_.notify_all();
    for (auto& w : workers_) w.join();
  }
  int size() const { return n_; }

  // Splits [0, total) into n_ contiguous ranges and runs fn(begin, end) on each.
  void run(int64_t total, const std::function<void(int64_t, int64_t)>& fn) {
    if (n_ == 1 || total <= 1) {
      fn(0, total);
      return;
    }
    {
      std::lock_guard<std::mutex> l(mu_);
      fn_ = &fn;
      total_ = total;
      pending_.store(n_ - 1, std::memory_order_relaxed);
      gen_.fetch_add(1, std::memory_order_release);
    }
    cv_.notify_all();
    range(0, fn);
    while (pending_.load(std::memory_order_acquire) != 0) _mm_pause();
  }

 private:
  void range(int t, const std::function<void(int64_t, int64_t)>& fn) {
    const int64_t b = total_ * t / n_, e = total_ * (t + 1) / n_;
    if (b < e) fn(b, e);
  }
  void loop(int t) {
    uint64_t seen = 0;
    for (;;) {
      const std::function<void(int64_t, int64_t)>* fn;
      bool fresh = false;
      for (int i = 0; i < kSpin && !fresh; ++i) {
        fresh = gen_.load(std::memory_order_acquire) != seen;
        if (!fresh) _mm_pause();
      }
      {
        std::unique_lock<std::mutex> l(mu_);
        if (!fresh) cv_.wait(l, [&] { return gen_.load(std::memory_order_acquire) != seen; });
        seen = gen_.load(std::memory_order_acquire);
        if (stop_) return;
        fn = fn_;
      }
      range(t, *fn);
      pending_.fetch_sub(1, std::memory_order_acq_rel);
    }
  }
  int n_;
  std::vector<std::thread> workers_;
  std::mutex mu_;
  std::condition_variable cv_;
  static constexpr int kSpin = 1 << 14;  // pause instructions before sleeping
  std::atomic<uint64_t> gen_{0};
  bool stop_ = false;
  const std::function<void(int64_t, int64_t)>* fn_ = nullptr;
  int64_t total_ = 0;
  std::atomic<int> pending_{0};
};

void embedding(Pool& pool, const int32_t* ids, const uint16_t* table, int T, int H, uint16_t* out) {
  pool.run(T, [&](int64_t b, int64_t e) {
    for (int64_t t = b; t < e; ++t)
      std::memcpy(out + t * H, table + static_cast<int64_t>(ids[t]) * H, 2 * static_cast<size_t>(H));
  });
}

void add_rmsnorm(Pool& pool, uint16_t* res, const uint16_t* delta, const uint16_t* w, int T, int H,
                 float eps, uint16_t* out) {
  pool.run(T, [&](int64_t b, int64_t e) {
    for (int64_t t = b; t < e; ++t) {
      uint16_t* r = res + t * H;
      __m256 acc = _mm256_setzero_ps();
      for (int i = 0; i < H; i += 8) {
        __m256 x = load8h(r + i);
        if (delta != nullptr) {
          x = round8h(_mm256_add_ps(x, load8h(delta + t * H + i)));
          store8h(r + i, x);
        }
        acc = _mm256_add_ps(acc, _mm256_mul_ps(x, x));
      }
      alignas(32) float lanes[8];
      _mm256_store_ps(lanes, acc);
      float ss = 0.f;
      for (float v : lanes) ss += v;
      const __m256 inv = _mm256_set1_ps(1.0f / std::sqrt(ss / static_cast<float>(H) + eps));
      for (int i = 0; i < H; i += 8)
        store8h(out + t * H + i, _mm256_mul_ps(round8h(_mm256_mul_ps(load8h(r + i), inv)), load8h(w + i)));
    }
  });
}

void rope_kv(Pool& pool, uint16_t* qkv, const int32_t* pos, const int32_t* slots, int T, int Hq,
             int Hkv, int D, const float* cos_t, const float* sin_t, void* kc, void* vc,
             float* ks, float* vs, int bs, int int8) {
  const int half = D / 2, heads = Hq + 2 * Hkv;
  pool.run(T, [&](int64_t b, int64_t e) {
    alignas(32) float x0[64], x1[64];
    for (int64_t t = b; t < e; ++t) {
      const float* c = cos_t + static_cast<int64_t>(pos[t]) * half;
      const float* s = sin_t + static_cast<int64_t>(pos[t]) * half;
      const int slot = slots[t];
      for (int h = 0; h < heads; ++h) {
        uint16_t* hp = qkv + (t * heads + h) * D;
        for (int i = 0; i < half; i += 8) {
          __m256 a = load8h(hp + i), bb = load8h(hp + half + i);
          if (h < Hq + Hkv) {
            const __m256 cv = _mm256_loadu_ps(c + i), sv = _mm256_loadu_ps(s + i);
            const __m256 y0 = _mm256_sub_ps(_mm256_mul_ps(a, cv), _mm256_mul_ps(bb, sv));
            const __m256 y1 = _mm256_add_ps(_mm256_mul_ps(bb, cv), _mm256_mul_ps(a, sv));
            a = round8h(y0);
            bb = round8h(y1);
          }
          _mm256_store_ps(x0 + i, a);
          _mm256_store_ps(x1 + i, bb);
        }
        if (h < Hq) {
          for (int i = 0; i < half; i += 8) {
            store8h(hp + i, _mm256_load_ps(x0 + i));
            store8h(hp + half + i, _mm256_load_ps(x1 + i));
          }
          continue;
        }
        if (slot < 0) continue;
        const bool is_v = h >= Hq + Hkv;
        const int kvh = is_v ? h - Hq - Hkv : h - Hq;
        const int blk = slot / bs, off = slot % bs;
        const int64_t cell = (static_cast<int64_t>(blk) * Hkv + kvh) * bs + off;
        if (!int8) {
          uint16_t* dst = static_cast<uint16_t*>(is_v ? vc : kc) + cell * D;
          for (int i = 0; i < half; i += 8) {
            store8h(dst + i, _mm256_load_ps(x0 + i));
            store8h(dst + half + i, _mm256_load_ps(x1 + i));
          }
        } else {
          float amax = 0.f;
          for (int i = 0; i < half; ++i)
            amax = std::max(amax, std::max(std::fabs(x0[i]), std::fabs(x1[i])));
          const float scale = amax > 0.f ? amax / 127.f : 1.f;
          const float inv = 1.f / scale;
          int8_t* dst = static_cast<int8_t*>(is_v ? vc : kc) + cell * D;
          for (int i = 0; i < half; ++i) {
            dst[i] = static_cast<int8_t>(std::nearbyint(std::min(std::max(x0[i] * inv, -127.f), 127.f)));
            dst[half + i] =
                static_cast<int8_t>(std::nearbyint(std::min(std::max(x1[i] * inv, -127.f), 127.f)));
          }
          (is_v ? vs : ks)[cell] = scale;
        }
      }
    }
  });
}

// e^x for 8 floats (AVX2, no FMA): Cody-Waite range reduction x = n ln2 + r
// with ln2 split in two parts (the first exact in 9 bits), e^r on
// [-ln2/2, ln2/2] by its Taylor polynomial to degree 6 (truncation error
// below 1.3e-7 relative), and 2^n built in the exponent field.  Inputs are
// clamped to [-87.3, 88.7], where e^x is a normal float.
inline __m256 exp8(__m256 x) {
  x = _mm256_min_ps(_mm256_max_ps(x, _mm256_set1_ps(-87.3f)), _mm256_set1_ps(88.7f));
  const __m256 n = _mm256_round_ps(_mm256_mul_ps(x, _mm256_set1_ps(1.44269504088896341f)),
                                   _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
  __m256 r = _mm256_sub_ps(x, _mm256_mul_ps(n, _mm256_set1_ps(0.693359375f)));
  r = _mm256_sub_ps(r, _mm256_mul_ps(n, _mm256_set1_ps(-2.12194440054690583e-4f)));
  __m256 p = _mm256_set1_ps(1.f / 720.f);
  const float c[6] = {1.f / 120.f, 1.f / 24.f, 1.f / 6.f, 0.5f, 1.f, 1.f};
  for (float k : c) p = _mm256_add_ps(_mm256_mul_ps(p, r), _mm256_set1_ps(k));
  const __m256i e = _mm256_slli_epi32(_mm256_add_epi32(_mm256_cvtps_epi32(n), _mm256_set1_epi32(127)), 23);
  return _mm256_mul_ps(p, _mm256_castsi256_ps(e));
}

// fp16(fp16(silu(g)) * u), 8 elements at a time (inter is a multiple of 8).
void silu_and_mul(Pool& pool, const uint16_t* gu, int T, int I, uint16_t* out) {
  const int gpr = I / 8;  // groups of 8 per row
  pool.run(static_cast<int64_t>(T) * gpr, [&](int64_t b, int64_t e) {
    int64_t r = b / gpr, j = b - r * gpr;
    const __m256 one = _mm256_set1_ps(1.f);
    for (int64_t q = b; q < e; ++q) {
      const uint16_t* row = gu + r * 2 * I + 8 * j;
      const __m256 x = _mm256_cvtph_ps(_mm_loadu_si128(reinterpret_cast<const __m128i*>(row)));
      const __m256 u = _mm256_cvtph_ps(_mm_loadu_si128(reinterpret_cast<const __m128i*>(row + I)));
      __m256 s = _mm256_div_ps(x, _mm256_add_ps(one, exp8(_mm256_sub_ps(_mm256_setzero_ps(), x))));
      s = _mm256_cvtph_ps(_mm256_cvtps_ph(s, _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC));
      _mm_storeu_si128(reinterpret_cast<__m128i*>(out + r * I + 8 * j),
                       _mm256_cvtps_ph(_mm256_mul_ps(s, u), _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC));
      if (++j == gpr) {
        j = 0;
        ++r;
      }
    }
  });
}

}  // namespace

extern "C" {

// Threads usable by this process: the size of its CPU affinity mask.
int cps_affinity_cores(void) {
  cpu_set_t set;
  if (sched_getaffinity(0, sizeof(set), &set) != 0) return 1;
  return CPU_COUNT(&set);
}

// A pool of `threads` threads (the caller counts as one), or null when the CPU
// lacks AVX2/F16C.
void* cps_create(int threads) {
  if (!__builtin_cpu_supports("avx2") || !__builtin_cpu_supports("f16c")) return nullptr;
  return new Pool(threads);
}

void cps_destroy(void* pool) { delete static_cast<Pool*>(pool); }

void cps_layer_step_timed(void* pool_, const int32_t* ids, const uint16_t* table, int T, int H,
                          uint16_t* emb, uint16_t* residual, const uint16_t* delta,
                          const uint16_t* w_norm, float eps, uint16_t* normed, uint16_t* qkv,
                          const int32_t* positions, const int32_t* slots, int Hq, int Hkv, int D,
                          const float* cos_t, const float* sin_t, void* k_cache, void* v_cache,
                          float* k_scale, float* v_scale, int bs, int int8,
                          const uint16_t* gate_up, int I, uint16_t* act, double* seconds);

// One layer step, the same arguments as the oracle's orc_layer_step.
// head_dim must be 64 or 128, hidden and inter multiples of 8.
void cps_layer_step(void* pool_, const int32_t* ids, const uint16_t* table, int T, int H,
                    uint16_t* emb, uint16_t* residual, const uint16_t* delta,
                    const uint16_t* w_norm, float eps, uint16_t* normed, uint16_t* qkv,
                    const int32_t* positions, const int32_t* slots, int Hq, int Hkv, int D,
                    const float* cos_t, const float* sin_t, void* k_cache, void* v_cache,
                    float* k_scale, float* v_scale, int bs, int int8, const uint16_t* gate_up,
                    int I, uint16_t* act) {
  cps_layer_step_timed(pool_, ids, table, T, H, emb, residual, delta, w_norm, eps, normed, qkv,
                       positions, slots, Hq, Hkv, D, cos_t, sin_t, k_cache, v_cache, k_scale,
                       v_scale, bs, int8, gate_up, I, act, nullptr);
}

// The same step; with seconds != null, adds each op's wall time (its rows
// split over the pool, dispatch and join included) to seconds[0..4]:
// embedding, RMSNorm without delta, RoPE + KV, add + RMSNorm, SwiGLU.
void cps_layer_step_timed(void* pool_, const int32_t* ids, const uint16_t* table, int T, int H,
                          uint16_t* emb, uint16_t* residual, const uint16_t* delta,
                          const uint16_t* w_norm, float eps, uint16_t* normed, uint16_t* qkv,
                          const int32_t* positions, const int32_t* slots, int Hq, int Hkv, int D,
                          const float* cos_t, const float* sin_t, void* k_cache, void* v_cache,
                          float* k_scale, float* v_scale, int bs, int int8,
                          const uint16_t* gate_up, int I, uint16_t* act, double* seconds) {
  Pool& pool = *static_cast<Pool*>(pool_);
  using clock = std::chrono::steady_clock;
  auto t = clock::now();
  auto lap = [&](int op) {
    if (seconds == nullptr) return;
    const auto now = clock::now();
    seconds[op] += std::chrono::duration<double>(now - t).count();
    t = now;
  };
  embedding(pool, ids, table, T, H, emb);
  lap(0);
  add_rmsnorm(pool, emb, nullptr, w_norm, T, H, eps, normed);
  lap(1);
  rope_kv(pool, qkv, positions, slots, T, Hq, Hkv, D, cos_t, sin_t, k_cache, v_cache, k_scale,
          v_scale, bs, int8);
  lap(2);
  add_rmsnorm(pool, residual, delta, w_norm, T, H, eps, normed);
  lap(3);
  silu_and_mul(pool, gate_up, T, I, act);
  lap(4);
}

}  // extern "C"
