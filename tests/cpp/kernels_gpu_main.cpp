// GPU test of the C++ drop-in header: a program written the way the
// reference's engine and tests call redline::kernels (include
// "redline_amd/kernels.h", a KVLayerView of the reference's layout, half*
// device buffers, a hipStream_t), checked against fixtures the CPU oracle
// wrote (tests/golden/kernels_cpp.bin, from tests/golden/make_cpp_fixtures.py).
// Mirrors tests/cuda/test_kernels.cu:18-69,90-148,289-322 of Neil456/Redline.
//
// Usage: kernels_gpu <fixture file>.  Prints one line per check and PASS or
// FAIL at the end; exit status 0 only on PASS.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <map>
#include <string>
#include <vector>

#include "redline_amd/kernels.h"

using namespace redline;

namespace {

int failures = 0;

#define HIP_OK(x)                                                                    \
  do {                                                                               \
    const hipError_t e_ = (x);                                                       \
    if (e_ != hipSuccess) {                                                          \
      std::printf("HIP error %s at %s:%d\n", hipGetErrorString(e_), __FILE__, __LINE__); \
      std::exit(2);                                                                  \
    }                                                                                \
  } while (0)

std::map<std::string, std::vector<char>> load(const char* path) {
  std::map<std::string, std::vector<char>> out;
  std::ifstream f(path, std::ios::binary);
  char magic[8];
  uint32_t count = 0;
  if (!f.read(magic, 8) || std::memcmp(magic, "RLKFIX01", 8) != 0 ||
      !f.read(reinterpret_cast<char*>(&count), 4)) {
    std::printf("cannot read fixture %s\n", path);
    std::exit(2);
  }
  for (uint32_t i = 0; i < count; ++i) {
    uint32_t nlen = 0;
    uint64_t nbytes = 0;
    f.read(reinterpret_cast<char*>(&nlen), 4);
    std::string name(nlen, '\0');
    f.read(&name[0], nlen);
    f.read(reinterpret_cast<char*>(&nbytes), 8);
    std::vector<char> data(nbytes);
    f.read(data.data(), static_cast<std::streamsize>(nbytes));
    if (!f) {
      std::printf("truncated fixture at %s\n", name.c_str());
      std::exit(2);
    }
    out.emplace(name, std::move(data));
  }
  return out;
}

std::map<std::string, std::vector<char>> fx;

const std::vector<char>& get(const std::string& name) {
  auto it = fx.find(name);
  if (it == fx.end()) {
    std::printf("fixture has no array %s\n", name.c_str());
    std::exit(2);
  }
  return it->second;
}

// Device copy of a fixture array (or zeros of its size).
template <typename T>
T* upload(const std::string& name, bool zero = false) {
  const auto& a = get(name);
  void* d = nullptr;
  HIP_OK(hipMalloc(&d, a.size()));
  if (zero) {
    HIP_OK(hipMemset(d, 0, a.size()));
  } else {
    HIP_OK(hipMemcpy(d, a.data(), a.size(), hipMemcpyHostToDevice));
  }
  return static_cast<T*>(d);
}

std::vector<char> download(const void* d, size_t bytes) {
  std::vector<char> h(bytes);
  HIP_OK(hipMemcpy(h.data(), d, bytes, hipMemcpyDeviceToHost));
  return h;
}

void check_exact(const char* what, const void* d, const std::string& want) {
  const auto& w = get(want);
  const auto got = download(d, w.size());
  const bool ok = std::memcmp(got.data(), w.data(), w.size()) == 0;
  std::printf("%s %s (bit-exact, %zu bytes)\n", ok ? "ok  " : "FAIL", what, w.size());
  failures += !ok;
}

float h2f(uint16_t h) {
  _Float16 v;
  std::memcpy(&v, &h, 2);
  return static_cast<float>(v);
}

// fp16 outputs: |got - want| <= 2e-3 + 1e-2 |want| elementwise (the tolerance
// the hot path is held to after fp32 accumulation).
void check_close(const char* what, const void* d, const std::string& want) {
  const auto& w = get(want);
  const auto got = download(d, w.size());
  const size_t n = w.size() / 2;
  const auto* g = reinterpret_cast<const uint16_t*>(got.data());
  const auto* e = reinterpret_cast<const uint16_t*>(w.data());
  double worst = 0;
  bool ok = true;
  for (size_t i = 0; i < n; ++i) {
    const double a = h2f(g[i]), b = h2f(e[i]);
    const double err = std::fabs(a - b);
    worst = std::max(worst, err);
    if (!(err <= 2e-3 + 1e-2 * std::fabs(b))) ok = false;
  }
  std::printf("%s %s (max abs err %.3g over %zu values)\n", ok ? "ok  " : "FAIL", what, worst, n);
  failures += !ok;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc != 2) {
    std::printf("usage: %s <kernels_cpp.bin>\n", argv[0]);
    return 2;
  }
  fx = load(argv[1]);
  hipStream_t stream;
  HIP_OK(hipStreamCreate(&stream));

  {  // embedding_lookup
    auto* table = upload<half>("emb_table");
    auto* ids = upload<int32_t>("emb_ids");
    auto* out = upload<half>("emb_out", true);
    kernels::embedding_lookup(ids, table, 7, 256, out, stream);
    HIP_OK(hipStreamSynchronize(stream));
    check_exact("embedding_lookup", out, "emb_out");
    // extension: the gather and RMSNorm (no delta) in one launch
    auto* w = upload<half>("embnorm_w");
    auto* res = upload<half>("emb_out", true);
    auto* normed = upload<half>("emb_out", true);
    kernels::embedding_rmsnorm(ids, table, 7, 256, w, 1e-5f, res, normed, stream);
    HIP_OK(hipStreamSynchronize(stream));
    check_exact("embedding_rmsnorm residual", res, "emb_out");
    check_close("embedding_rmsnorm out", normed, "embnorm_out");
  }
  {  // fused_add_rmsnorm with delta, then without (on the original residual)
    auto* res = upload<half>("norm_res");
    auto* delta = upload<half>("norm_delta");
    auto* w = upload<half>("norm_w");
    auto* out = upload<half>("norm_out", true);
    kernels::fused_add_rmsnorm(res, delta, w, 5, 512, 1e-5f, out, stream);
    HIP_OK(hipStreamSynchronize(stream));
    check_exact("fused_add_rmsnorm residual", res, "norm_res_out");
    check_close("fused_add_rmsnorm out", out, "norm_out");
    auto* res2 = upload<half>("norm_res");
    kernels::fused_add_rmsnorm(res2, nullptr, w, 5, 512, 1e-5f, out, stream);
    HIP_OK(hipStreamSynchronize(stream));
    check_exact("fused_add_rmsnorm(delta = nullptr) residual untouched", res2, "norm_res");
    check_close("fused_add_rmsnorm(delta = nullptr) out", out, "norm_nodelta_out");
  }
  {  // silu_and_mul, split and interleaved
    auto* gu = upload<half>("swiglu_gu");
    auto* out = upload<half>("swiglu_out", true);
    kernels::silu_and_mul(gu, 3, 256, out, stream);
    HIP_OK(hipStreamSynchronize(stream));
    check_close("silu_and_mul", out, "swiglu_out");
    kernels::silu_and_mul_interleaved(gu, 3, 256, out, stream);
    HIP_OK(hipStreamSynchronize(stream));
    check_close("silu_and_mul_interleaved", out, "swiglu_il_out");
  }
  {  // rope_and_write_kv FP16 into a shuffled paged pool, then decode attention
    const auto& dims_b = get("rope_dims");
    int dims[8];
    std::memcpy(dims, dims_b.data(), sizeof(dims));
    const int T = dims[0], hq = dims[1], hkv = dims[2], D = dims[3], bs = dims[4];
    const int max_blocks = dims[7];
    auto* qkv = upload<half>("rope_qkv");
    auto* pos = upload<int32_t>("rope_pos");
    auto* slots = upload<int32_t>("rope_slots");
    auto* cos = upload<float>("rope_cos");
    auto* sin = upload<float>("rope_sin");
    auto* tables = upload<int32_t>("rope_tables");
    KVLayerView kv;  // the reference's struct layout (kernels.h:18-27)
    kv.k = upload<half>("rope_k_out", true);
    kv.v = upload<half>("rope_v_out", true);
    kv.block_size = bs;
    kv.num_kv_heads = hkv;
    kv.head_dim = D;
    kv.dtype = KVDType::kFP16;
    kernels::rope_and_write_kv(qkv, pos, slots, T, hq, cos, sin, kv, stream);
    HIP_OK(hipStreamSynchronize(stream));
    check_exact("rope_and_write_kv q (in place)", qkv, "rope_qkv_out");
    check_exact("rope_and_write_kv K cells", kv.k, "rope_k_out");
    check_exact("rope_and_write_kv V cells", kv.v, "rope_v_out");

    auto* items = upload<int32_t>("att_items");
    auto* seqs = upload<int32_t>("att_seqs");
    half* out = nullptr;
    HIP_OK(hipMalloc(&out, static_cast<size_t>(T) * hq * D * 2));
    HIP_OK(hipMemset(out, 0, static_cast<size_t>(T) * hq * D * 2));
    kernels::AttentionParams p;
    p.q = qkv;
    p.q_stride = (hq + 2 * hkv) * D;
    p.out = out;
    p.num_heads = hq;
    p.scale = 1.0f / std::sqrt(static_cast<float>(D));
    p.kv = kv;
    p.block_tables = tables;
    p.max_blocks_per_seq = max_blocks;
    p.positions = pos;
    kernels::DecodeAttentionWork w;
    w.item_token = items;
    w.item_seq = seqs;
    w.num_items = 2;
    w.max_partitions = 1;
    kernels::paged_attention_decode(p, w, stream);
    HIP_OK(hipStreamSynchronize(stream));
    // the two decode rows (tokens 47 and 64), gathered on the host
    const auto& it = get("att_items");
    const auto* itv = reinterpret_cast<const int32_t*>(it.data());
    half* rows = nullptr;
    const size_t row_bytes = static_cast<size_t>(hq) * D * 2;
    HIP_OK(hipMalloc(&rows, 2 * row_bytes));
    for (int i = 0; i < 2; ++i)
      HIP_OK(hipMemcpy(reinterpret_cast<char*>(rows) + i * row_bytes,
                       reinterpret_cast<char*>(out) + static_cast<size_t>(itv[i]) * row_bytes,
                       row_bytes, hipMemcpyDeviceToDevice));
    check_close("paged_attention_decode", rows, "att_out");
  }
  {  // INT8 KV write with fp32 scales (test_kernels.cu:289-322 geometry)
    auto* qkv = upload<half>("int8_qkv");
    auto* cos = upload<float>("int8_cos");
    auto* sin = upload<float>("int8_sin");
    const int32_t h_pos = 5, h_slot = 16 + 3;
    int32_t *pos = nullptr, *slot = nullptr;
    HIP_OK(hipMalloc(&pos, 4));
    HIP_OK(hipMalloc(&slot, 4));
    HIP_OK(hipMemcpy(pos, &h_pos, 4, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(slot, &h_slot, 4, hipMemcpyHostToDevice));
    KVLayerView kv;
    kv.k = upload<int8_t>("int8_k_out", true);
    kv.v = upload<int8_t>("int8_v_out", true);
    kv.k_scale = upload<float>("int8_ks_out", true);
    kv.v_scale = upload<float>("int8_vs_out", true);
    kv.block_size = 16;
    kv.num_kv_heads = 1;
    kv.head_dim = 64;
    kv.dtype = KVDType::kINT8;
    kernels::rope_and_write_kv(qkv, pos, slot, 1, 2, cos, sin, kv, stream);
    HIP_OK(hipStreamSynchronize(stream));
    check_exact("rope_and_write_kv INT8 q", qkv, "int8_qkv_out");
    check_exact("rope_and_write_kv INT8 K codes", kv.k, "int8_k_out");
    check_exact("rope_and_write_kv INT8 V codes", kv.v, "int8_v_out");
    check_exact("rope_and_write_kv INT8 k_scale", kv.k_scale, "int8_ks_out");
    check_exact("rope_and_write_kv INT8 v_scale", kv.v_scale, "int8_vs_out");
  }
  {  // a launcher error still throws redline::Error on the GPU path
    bool threw = false;
    try {
      kernels::silu_and_mul(nullptr, 2, 20, nullptr, stream);
    } catch (const Error&) {
      threw = true;
    }
    std::printf("%s silu_and_mul(inter 20) throws redline::Error\n", threw ? "ok  " : "FAIL");
    failures += !threw;
  }
  HIP_OK(hipStreamDestroy(stream));
  std::printf("%s\n", failures == 0 ? "PASS" : "FAIL");
  return failures == 0 ? 0 : 1;
}
