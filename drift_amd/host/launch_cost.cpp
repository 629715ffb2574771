// Host cost of a C-ABI call: each entry point called 1000 times from a C++
// loop at its benchmark shape, in batches of 100 asynchronous calls with the
// stream drained between batches (so the queue never backs up into the
// call), timed on the host around each batch's calls. Prints one JSON line,
// microseconds per call by entry point. The caller's cost per launch is this
// plus the HIP runtime's dispatch, which the calls include.
#include <hip/hip_runtime.h>

#include <chrono>
#include <cstdint>
#include <cstdio>
#include <functional>
#include <string>
#include <vector>

#include "../../include/drift_kernels.h"

namespace {

constexpr int kBatches = 10;
constexpr int kPerBatch = 100;

void check(hipError_t e, const char* what) {
  if (e != hipSuccess) {
    std::fprintf(stderr, "%s: %s\n", what, hipGetErrorString(e));
    std::exit(1);
  }
}

void* device_zeros(size_t bytes) {
  void* p = nullptr;
  check(hipMalloc(&p, bytes), "hipMalloc");
  check(hipMemset(p, 0, bytes), "hipMemset");
  return p;
}

// Microseconds per call, after one untimed batch.
double per_call(const char* entry, hipStream_t stream, const std::function<int()>& call) {
  double total = 0.0;
  for (int batch = -1; batch < kBatches; ++batch) {
    const auto t0 = std::chrono::steady_clock::now();
    for (int i = 0; i < kPerBatch; ++i)
      if (const int code = call()) {
        std::fprintf(stderr, "%s: error %d: %s\n", entry, code, drift_last_error());
        std::exit(1);
      }
    const auto t1 = std::chrono::steady_clock::now();
    check(hipStreamSynchronize(stream), "hipStreamSynchronize");
    if (batch >= 0) total += std::chrono::duration<double, std::micro>(t1 - t0).count();
  }
  return total / (kBatches * kPerBatch);
}

}  // namespace

int main() {
  hipStream_t stream;
  check(hipStreamCreate(&stream), "hipStreamCreate");
  std::vector<std::pair<std::string, double>> results;

  // C3: per-head RMSNorm + NeoX RoPE, Q [4096, 32, 128], K [4096, 8, 128] bf16
  {
    const int tokens = 4096, heads = 32, kv = 8, dim = 128;
    auto* q = static_cast<uint16_t*>(device_zeros((size_t)tokens * heads * dim * 2));
    auto* k = static_cast<uint16_t*>(device_zeros((size_t)tokens * kv * dim * 2));
    auto* rq = static_cast<uint16_t*>(device_zeros((size_t)tokens * heads * dim * 2));
    auto* rk = static_cast<uint16_t*>(device_zeros((size_t)tokens * kv * dim * 2));
    auto* w = static_cast<float*>(device_zeros(dim * 4));
    auto* positions = static_cast<int32_t*>(device_zeros((size_t)tokens * 4));
    results.emplace_back("drift_qk_norm_rope_bf16", per_call("drift_qk_norm_rope_bf16", stream, [&] {
                           return drift_qk_norm_rope_bf16(q, k, rq, rk, w, w, positions, tokens, heads, kv, dim, 1e-6f,
                                                          0.0f, dim, 1e6f, DRIFT_ROPE_NEOX, DRIFT_SECTIONS_SINGLE, 0,
                                                          0, 0, 0, stream);
                         }));
    results.emplace_back("drift_rope_bf16", per_call("drift_rope_bf16", stream, [&] {
                           return drift_rope_bf16(q, positions, rq, 16, heads, dim, dim, 1e6f, DRIFT_ROPE_NEOX,
                                                  DRIFT_SECTIONS_SINGLE, 0, 0, 0, 0, stream);
                         }));
  }
  // C2 decode: RMSNorm bf16 [1, 4096], SwiGLU bf16 [1, 14336]
  {
    auto* x = static_cast<uint16_t*>(device_zeros(4096 * 2));
    auto* out = static_cast<uint16_t*>(device_zeros(4096 * 2));
    auto* w = static_cast<float*>(device_zeros(4096 * 4));
    results.emplace_back("drift_rms_norm_bf16", per_call("drift_rms_norm_bf16", stream, [&] {
                           return drift_rms_norm_bf16(x, nullptr, w, out, 1, 4096, 1e-5f, 0.0f, 1, nullptr, nullptr,
                                                      nullptr, stream);
                         }));
    auto* g = static_cast<uint16_t*>(device_zeros(14336 * 2));
    auto* u = static_cast<uint16_t*>(device_zeros(14336 * 2));
    auto* s = static_cast<uint16_t*>(device_zeros(14336 * 2));
    results.emplace_back("drift_gated_bf16", per_call("drift_gated_bf16", stream, [&] {
                           return drift_gated_bf16(g, u, s, 14336, DRIFT_SILU, nullptr, nullptr, nullptr, stream);
                         }));
  }
  // C4: Q8_0 gather of 64 ids from a [1024, 4096] table (the call's cost does
  // not depend on the sizes)
  {
    auto* table = static_cast<uint8_t*>(device_zeros((size_t)1024 * 128 * 34));
    auto* ids = static_cast<int32_t*>(device_zeros(64 * 4));
    auto* out = static_cast<uint16_t*>(device_zeros((size_t)64 * 4096 * 2));
    results.emplace_back("drift_embedding_q8_0_bf16", per_call("drift_embedding_q8_0_bf16", stream, [&] {
                           return drift_embedding_q8_0_bf16(table, ids, out, 64, 1024, 4096, nullptr, stream);
                         }));
  }
  check(hipStreamSynchronize(stream), "hipStreamSynchronize");

  std::string line = "{";
  for (size_t i = 0; i < results.size(); ++i) {
    char value[64];
    std::snprintf(value, sizeof value, "%.3f", results[i].second);
    line += (i ? ", \"" : "\"") + results[i].first + "\": " + value;
  }
  line += ", \"calls\": " + std::to_string(kBatches * kPerBatch) + "}";
  std::printf("%s\n", line.c_str());
  return 0;
}
