// Host-only check of the C++ launch interface: argument errors throw
// redline::Error before anything is launched; empty batches are no-ops.
#include <cstdio>
#include <string>

#include "redline_amd/kernels.h"

using namespace redline;

static int failures = 0;

template <typename F>
static void expect_throw(const char* what, F f, const char* needle) {
  try {
    f();
    std::printf("FAIL %s: no exception\n", what);
    ++failures;
  } catch (const Error& e) {
    if (std::string(e.what()).find(needle) == std::string::npos) {
      std::printf("FAIL %s: message '%s'\n", what, e.what());
      ++failures;
    }
  }
}

int main() {
  expect_throw("embedding", [] { kernels::embedding_lookup(nullptr, nullptr, 2, 12, nullptr, nullptr); },
               "multiple of 8");
  expect_throw("norm", [] { kernels::fused_add_rmsnorm(nullptr, nullptr, nullptr, 2, 20, 1e-5f, nullptr, nullptr); },
               "multiple of 8");
  expect_throw("swiglu", [] { kernels::silu_and_mul(nullptr, 2, 20, nullptr, nullptr); }, "multiple of 8");
  KVLayerView kv;
  kv.num_kv_heads = 2;
  kv.head_dim = 80;
  expect_throw("rope", [&] { kernels::rope_and_write_kv(nullptr, nullptr, nullptr, 1, 4, nullptr, nullptr, kv, nullptr); },
               "unsupported head_dim 80");
  alignas(16) static unsigned char dummy[256];
  const half* hx = reinterpret_cast<const half*>(dummy);
  half* hy = reinterpret_cast<half*>(dummy);
  expect_throw("gemv_w4 null", [&] { kernels::gemv_w4a16(nullptr, 1, dummy, hx, hx, 128, nullptr, 8, 256, hy, false, nullptr); },
               "null pointer");
  expect_throw("gemv_w4 k", [&] { kernels::gemv_w4a16(hx, 1, dummy, hx, hx, 128, nullptr, 8, 200, hy, false, nullptr); },
               "multiples of 32");
  expect_throw("gemv_w4 m", [&] { kernels::gemv_w4a16(hx, kernels::kGemvW4MaxM + 1, dummy, hx, hx, 128, nullptr, 8, 256, hy, true, nullptr); },
               "unsupported m");
  expect_throw("gemv_w4 swiglu n", [&] { kernels::gemv_w4a16_swiglu(hx, 2, dummy, hx, hx, 128, 7, 256, hy, nullptr); },
               "even");
  kernels::gemv_w4a16_swiglu(hx, 0, dummy, hx, hx, 128, 8, 256, hy, nullptr);
  const int8_t* w8 = reinterpret_cast<const int8_t*>(dummy);
  expect_throw("gemv_w8 k", [&] { kernels::gemv_w8a16(hx, 1, w8, hx, nullptr, 8, 200, hy, false, nullptr); },
               "K % 16");
  expect_throw("gemv_w8 m", [&] { kernels::gemv_w8a16(hx, kernels::kGemvW8MaxM + 1, w8, hx, nullptr, 8, 256, hy, true, nullptr); },
               "unsupported m");
  kernels::gemv_w8a16(hx, 0, w8, hx, nullptr, 8, 256, hy, false, nullptr);
  kernels::AttentionParams ap;
  ap.num_heads = 4;
  ap.kv.num_kv_heads = 2;
  ap.kv.head_dim = 96;
  ap.kv.block_size = 16;
  kernels::PrefillAttentionWork pw;
  kernels::paged_attention_prefill(ap, pw, nullptr);  // no sequences: no-op
  pw.num_seqs = 1;
  pw.max_q_tiles = 1;
  expect_throw("prefill head_dim", [&] { kernels::paged_attention_prefill(ap, pw, nullptr); },
               "unsupported head_dim 96");
  ap.kv.head_dim = 64;
  expect_throw("prefill null", [&] { kernels::paged_attention_prefill(ap, pw, nullptr); }, "null pointer");
  // n <= 0 is a silent no-op, as in the reference.
  kernels::embedding_lookup(nullptr, nullptr, 0, 12, nullptr, nullptr);
  kernels::rope_and_write_kv(nullptr, nullptr, nullptr, 0, 4, nullptr, nullptr, kv, nullptr);
  std::printf(failures == 0 ? "PASS\n" : "FAILED\n");
  return failures == 0 ? 0 : 1;
}
