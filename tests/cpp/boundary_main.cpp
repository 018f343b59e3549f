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
  // n <= 0 is a silent no-op, as in the reference.
  kernels::embedding_lookup(nullptr, nullptr, 0, 12, nullptr, nullptr);
  kernels::rope_and_write_kv(nullptr, nullptr, nullptr, 0, 4, nullptr, nullptr, kv, nullptr);
  std::printf(failures == 0 ? "PASS\n" : "FAILED\n");
  return failures == 0 ? 0 : 1;
}
