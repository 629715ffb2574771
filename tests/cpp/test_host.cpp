// Tests of the C++ host side (drift_amd/host): `--checks` runs on the CPU the
// shape and dtype refusals with the reference's messages (object Ops's
// `require`s, as the reference's CPU suite meets them) and a refusal of the
// library surfacing as a HipException, launching nothing; `--gpu` runs
// operations on the device through HipOps and holds them to the oracle
// (oracle/cpu_ops.h, the reference's CPU arithmetic restated in C) at the
// bars the Python parity tests use: F32 |a - e| <= 1e-6 + 1e-5 |e|, BF16
// within 1 ulp, gathers and decodes bit-exact.
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <optional>
#include <tuple>
#include <random>
#include <string>
#include <vector>

#include "../../drift_amd/host/drift_ops.hpp"
#include "../../drift_amd/host/gguf.hpp"
#include "../../oracle/cpu_ops.h"
#include "comparison.hpp"

using namespace drift;

namespace {

int failures = 0;
std::vector<std::pair<std::string, std::function<void()>>>& registry(bool gpu) {
  static std::vector<std::pair<std::string, std::function<void()>>> cpu, device;
  return gpu ? device : cpu;
}

struct Register {
  Register(bool gpu, const char* name, std::function<void()> body) { registry(gpu).emplace_back(name, body); }
};

#define CHECK_TEST(name) \
  static void name();    \
  static Register reg_##name(false, #name, name);\
  static void name()
#define GPU_TEST(name) \
  static void name();  \
  static Register reg_##name(true, #name, name);\
  static void name()

struct Failure : std::runtime_error {
  using std::runtime_error::runtime_error;
};

void expect(bool condition, const std::string& what) {
  if (!condition) throw Failure(what);
}

// `body` must throw `E` whose message contains `needle`.
template <typename E = std::invalid_argument>
void refused(const std::function<void()>& body, const std::string& needle) {
  try {
    body();
  } catch (const E& e) {
    expect(std::string(e.what()).find(needle) != std::string::npos,
           "message \"" + std::string(e.what()) + "\" lacks \"" + needle + "\"");
    return;
  }
  throw Failure("not refused: expected \"" + needle + "\"");
}

// A tensor at a made-up device address: the checks never dereference it.
Tensor fake(DType dtype, Shape shape, uintptr_t address = 4096) {
  return Tensor{dtype, std::move(shape), reinterpret_cast<void*>(address)};
}

// ---------------------------------------------------------------- checks (CPU)

CHECK_TEST(row_wise_checks_carry_the_reference_messages) {
  HipOps hip;
  const Tensor x = fake(DType::F32, {3, 7}), w = fake(DType::F32, {7});
  refused([&] { hip.rmsNorm(x, w, 1e-6f, 0.0f, fake(DType::F32, {3, 8})); },
          "requirement failed: rmsNorm needs equal shapes, got [3×7], [3×8]");
  refused([&] { hip.rmsNorm(x, fake(DType::F32, {6}), 1e-6f, 0.0f, x); }, "rmsNorm: [6] for rows of 7");
  refused([&] { hip.rmsNorm(fake(DType::I32, {3, 7}), w, 1e-6f, 0.0f, fake(DType::I32, {3, 7})); },
          "rmsNorm takes F32 or BF16, not I32");
  refused([&] { hip.rmsNorm(x, w, 1e-6f, 0.0f, fake(DType::BF16, {3, 7})); },
          "rmsNorm takes one type, not F32 and BF16");
  refused([&] { hip.rmsNorm(x, fake(DType::BF16, {7}), 1e-6f, 0.0f, x); }, "rmsNorm takes F32, not BF16");
  refused([&] { hip.groupRmsNorm(x, w, 2, 1e-6f, 0.0f, x); }, "requirement failed: [3×7] in 2 groups");
  refused([&] { hip.groupRmsNorm(x, fake(DType::F32, {6}), 7, 1e-6f, 0.0f, x); }, "groupRmsNorm: [6] for rows of 7");
  refused([&] { hip.layerNorm(fake(DType::BF16, {3, 7}), nullptr, nullptr, 1e-6f, fake(DType::BF16, {3, 7})); },
          "layerNorm takes F32, not BF16");
  refused([&] { hip.addRmsNorm(x, fake(DType::F32, {3, 6}), RowNorm{w, 1e-6f, 0.0f, x}); },
          "addRmsNorm needs equal shapes, got [3×7], [3×6]");
}

CHECK_TEST(modulation_and_gates_are_checked) {
  HipOps hip;
  const Tensor x = fake(DType::BF16, {4, 8}), table = fake(DType::F32, {4, 48});
  refused([&] { hip.modulateChunks(x, table, 3, 6, x); },
          "modulateChunks: table [4×48] for [4×8], chunks ArraySeq(3, 6)");
  refused([&] { hip.gatedAddChunk(x, x, fake(DType::F32, {5, 48}), 1); },
          "gatedAddChunk: table [5×48] for [4×8], chunks ArraySeq(1)");
  refused([&] { hip.rowGatedAdd(x, x, fake(DType::F32, {3})); }, "rowGatedAdd: gate [3] for [4×8]");
  refused([&] { hip.gatedAdd(x, x, fake(DType::F32, {2, 8}), 0); }, "gatedAdd: per-sample gates need rowsPerSample");
  refused([&] { hip.gatedAdd(x, x, fake(DType::F32, {3, 8}), 2); }, "gatedAdd: [3×8] for 2 samples of rows of 8");
  refused([&] { hip.layerNormModulate(x, fake(DType::F32, {2, 8}), fake(DType::F32, {2, 8}), 1e-6f, x, 1); },
          "layerNormModulate: 2 samples of 1 rows for 4 rows");
  refused([&] { hip.layerNormModulate(x, fake(DType::F32, {2, 7}), fake(DType::F32, {2, 7}), 1e-6f, x); },
          "layerNormModulate: scale [2×7], shift [2×7] for rows of 8");
}

CHECK_TEST(rope_rules) {
  HipOps hip;
  const Tensor x = fake(DType::F32, {5, 2, 128});
  const Rope neox{1e4f, 128, RopeLayout::Neox, RopeSections::Single()};
  refused([&] { hip.rope(x, fake(DType::F32, {5}), neox, x); }, "rope positions are I32, not F32");
  refused([&] { hip.rope(x, fake(DType::I32, {4}), neox, x); }, "rope positions [4], expected [5]");
  refused([&] { hip.rope(x, fake(DType::I32, {5}), Rope{1e4f, 130, RopeLayout::Neox, {}}, x); },
          "rope: 130 rotary dimensions in heads of 128");
  const Rope axes{1e4f, 128, RopeLayout::Interleaved, RopeSections::Axes({16, 24, 23})};
  refused([&] { hip.rope(x, fake(DType::I32, {3, 5}), axes, x); }, "rope: axes of [16, 24, 23] pairs for 128");
  const Rope mrope{1e6f, 128, RopeLayout::Neox, RopeSections::Contiguous(16, 24, 24)};
  refused([&] { hip.rope(x, fake(DType::I32, {5}), mrope, x); }, "rope positions [5], expected [3×5]");
  refused([&] { hip.rope(fake(DType::F32, {5, 256}), fake(DType::I32, {5}), neox, fake(DType::F32, {5, 256})); },
          "rope takes [tokens, heads, headDimension], got [5×256]");
  refused([&] { hip.ropeTable(x, fake(DType::F32, {5, 65}), fake(DType::F32, {5, 65}), x); },
          "ropeTable: tables [5×65], [5×65] for [5×2×128]");
  QueryKeyNorms norms{fake(DType::F32, {128}), fake(DType::F32, {64}), 1e-6f, 0.0f, neox};
  refused([&] {
    hip.queryKeyNormRope(x, fake(DType::F32, {5, 1, 128}), norms, fake(DType::I32, {5}), x,
                         fake(DType::F32, {5, 1, 128}));
  }, "queryKeyNormRope: keyNorm [64] for heads of 128");
}

CHECK_TEST(cache_and_attention_inputs_are_checked) {
  HipOps hip;
  refused([&] { KvCache::of(fake(DType::F16, {2, 8, 2, 64}), fake(DType::F16, {2, 2, 64, 8}), 8); },
          "pages of 8 tokens: not a multiple of 16");
  refused([&] { KvCache::of(fake(DType::F16, {2, 16, 2, 64}), fake(DType::F16, {2, 2, 16, 64}), 16); },
          "cache values [2×2×16×64] for keys [2×16×2×64]");
  const KvCache cache = KvCache::of(fake(DType::F16, {2, 16, 2, 64}), fake(DType::F16, {2, 2, 64, 16}), 16);
  const Tensor k = fake(DType::BF16, {20, 2, 64});
  refused([&] { hip.cacheWrite(k, k, cache, fake(DType::I32, {1}), 0); }, "a page table of 1 pages for 20 positions");
  refused([&] { hip.cacheWrite(fake(DType::BF16, {20, 3, 64}), fake(DType::BF16, {20, 3, 64}), cache,
                               fake(DType::I32, {2}), 0); },
          "cacheWrite: [20×3×64] into a cache of 2 heads of 64");
  refused([&] { hip.cacheWrite(k, k, cache, fake(DType::F32, {2}), 0); }, "a page table is I32 [pages], not F32 [2]");
  refused([&] { hip.splitHalves(fake(DType::F32, {4, 10}), fake(DType::F32, {4, 4}), fake(DType::F32, {4, 4})); },
          "splitHalves: [4×10] into [4×4]");
  const Rope rope{1e6f, 64, RopeLayout::Neox, {}};
  QueryKeyNorms norms{fake(DType::F32, {64}), fake(DType::F32, {64}), 1e-6f, 0.0f, rope};
  refused([&] {
    hip.queryKeyNormRopeCache(fake(DType::BF16, {20, 4, 1024}), k, k, norms, fake(DType::I32, {20}), cache,
                              fake(DType::I32, {2}), 0, fake(DType::BF16, {20, 4, 1024}));
  }, "queryKeyNormRopeCache: queries [20×4×1024]");
}

CHECK_TEST(tables_are_checked) {
  HipOps hip;
  const StorageType& q4k = StorageType::named("Q4_K");
  const StoredTable table{fake(DType::U8, {10, 144}), &q4k, 256};
  refused([&] { hip.embedding(table, fake(DType::I8, {3}), fake(DType::F32, {3, 256})); },
          "embedding ids are I32 [tokens], not I8 [3]");
  refused([&] { hip.embedding(table, fake(DType::I32, {3}), fake(DType::F32, {4, 256})); },
          "embedding: out [4×256] for 3 rows of 256");
  refused([&] { hip.embedding(StoredTable{fake(DType::U8, {10, 140}), &q4k, 256}, fake(DType::I32, {3}),
                              fake(DType::F32, {3, 256})); },
          "embedding: Q4_K bytes [10×140] for rows of 256");
  refused([&] { hip.dequantize(table, fake(DType::F32, {10, 256})); }, "dequantize writes BF16 or F16, not F32");
  refused([&] { hip.rotated(fake(DType::U8, {4, 256}), ConvRotParts{fake(DType::F32, {4}), {}}); },
          "rotated: U8 codes [4×256]");
  refused([&] { hip.rotated(fake(DType::I8, {4, 200}), ConvRotParts{fake(DType::F32, {4}), {}}); },
          "rotated: rows of 200 columns");
  refused([&] { hip.rotated(fake(DType::I8, {4, 256}), ConvRotParts{fake(DType::F32, {3}), {}}); },
          "rotated: 3 F32 scales for 4 rows");
  const ConvRotLevels levels{fake(DType::F32, {16}), fake(DType::U8, {4, 16}), 24};
  refused([&] { hip.rotated(fake(DType::I8, {4, 256}), ConvRotParts{fake(DType::F32, {4}), levels}); },
          "rotated: 512 columns in groups of 24");
  const RotatedTable rotated = hip.rotated(fake(DType::I8, {4, 256}), ConvRotParts{fake(DType::F32, {1}), {}});
  expect(rotated.shape() == Shape({4, 256}) && std::string(rotated.dtype()) == "CONVROT_I8", "rotated shape");
  refused([&] { hip.convert(rotated, fake(DType::F32, {4, 256})); }, "convert: no conversion from CONVROT_I8 to F32");
  refused([&] { hip.convert(fake(DType::BF16, {4}), fake(DType::F16, {4})); },
          "convert: no conversion from BF16 to F16");
}

CHECK_TEST(library_refusals_are_hip_exceptions) {
  // shapes the checks accept, a table 4 bytes off the 8-byte alignment Q4_K's
  // fields need: the library refuses before launching anything
  HipOps hip;
  const StorageType& q4k = StorageType::named("Q4_K");
  const StoredTable shifted{fake(DType::U8, {3, 144}, 4100), &q4k, 256};
  refused<HipException>([&] { hip.embedding(shifted, fake(DType::I32, {1}), fake(DType::F32, {1, 256})); },
                        "8-byte aligned");
  try {
    hip.embedding(shifted, fake(DType::I32, {1}), fake(DType::F32, {1, 256}));
  } catch (const HipException& e) {
    expect(e.entry == "drift_embedding_f32" && e.code == 1, "the exception names the entry point and code");
  }
}

CHECK_TEST(comparison_rule_as_the_reference_states_it) {
  using testing::Comparison;
  using testing::Tolerance;
  const float nan = std::nanf(""), inf = INFINITY;
  expect(Comparison::of({1.0f, nan, inf, -inf}, {1.0f, nan, inf, -inf}, Tolerance{}).passed(),
         "equal values, NaN with NaN, infinities with themselves");
  const Comparison c = Comparison::of({1.0f, nan, inf, 0.0f, 2.0f}, {1.5f, 0.0f, -inf, nan, 2.0f}, Tolerance{0.25, 0.0});
  expect(c.mismatches == 4 && c.firstMismatch == 0 && c.maxAbsolute == 0.5 && c.maxRelative == 0.5,
         "mismatches " + c.summary());
  expect(Comparison::of({100.0f}, {100.9f}, Tolerance{0.0, 1e-2}).passed() &&
             !Comparison::of({100.0f}, {101.1f}, Tolerance{0.0, 1e-2}).passed(),
         "relative part scales with |expected|");
  refused([] { Comparison::of({1.0f}, {1.0f, 2.0f}, Tolerance{}); }, "comparing 2 values with 1");
}

// ---------------------------------------------------------------- GPU parity

void hip_check(hipError_t status, const char* what) {
  if (status != hipSuccess) throw Failure(std::string(what) + ": " + hipGetErrorString(status));
}

// Device memory for a test, freed at scope end.
struct Device {
  std::vector<void*> owned;
  ~Device() {
    for (void* p : owned) (void)hipFree(p);
  }
  template <typename T>
  Tensor upload(DType dtype, Shape shape, const std::vector<T>& host) {
    void* p = nullptr;
    const size_t bytes = host.size() * sizeof(T);
    hip_check(hipMalloc(&p, bytes ? bytes : 16), "hipMalloc");
    owned.push_back(p);
    if (bytes) hip_check(hipMemcpy(p, host.data(), bytes, hipMemcpyHostToDevice), "hipMemcpy");
    return Tensor{dtype, std::move(shape), p};
  }
  Tensor empty(DType dtype, Shape shape) {
    void* p = nullptr;
    const int64_t bytes = Tensor{dtype, shape, nullptr}.byteSize();
    hip_check(hipMalloc(&p, (size_t)(bytes ? bytes : 16)), "hipMalloc");
    owned.push_back(p);
    return Tensor{dtype, std::move(shape), p};
  }
  template <typename T>
  std::vector<T> download(const Tensor& t) {
    std::vector<T> host((size_t)(t.byteSize() / (int64_t)sizeof(T)));
    hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
    hip_check(hipMemcpy(host.data(), t.data, host.size() * sizeof(T), hipMemcpyDeviceToHost), "hipMemcpy");
    return host;
  }
};

std::vector<float> gaussian(uint64_t seed, size_t n, float scale = 1.0f) {
  std::mt19937_64 rng(seed);
  std::normal_distribution<float> normal(0.0f, scale);
  std::vector<float> v(n);
  for (float& x : v) x = normal(rng);
  return v;
}

std::vector<uint16_t> to_bf16(const std::vector<float>& x) {
  std::vector<uint16_t> b(x.size());
  oracle_f32_to_bf16_n(x.data(), b.data(), (int64_t)x.size());
  return b;
}

std::vector<float> from_bf16(const std::vector<uint16_t>& b) {
  std::vector<float> x(b.size());
  oracle_bf16_to_f32_n(b.data(), x.data(), (int64_t)b.size());
  return x;
}

// F32 results: the reference's rule at the F32 bar.
void close_f32(const std::vector<float>& want, const std::vector<float>& got, const char* what) {
  const testing::Comparison c = testing::Comparison::of(want, got, testing::Tolerance{1e-6, 1e-5});
  if (!c.passed()) throw Failure(std::string(what) + ": " + c.summary());
}

int64_t ordered(uint16_t b) { return (b & 0x8000) ? -(int64_t)(b & 0x7fff) : (int64_t)b; }

void within_ulp(const std::vector<uint16_t>& want, const std::vector<uint16_t>& got, const char* what) {
  expect(want.size() == got.size(), std::string(what) + ": sizes");
  for (size_t i = 0; i < want.size(); ++i)
    if (std::llabs(ordered(want[i]) - ordered(got[i])) > 1)
      throw Failure(std::string(what) + ": index " + std::to_string(i) + " beyond 1 ulp");
}

template <typename T>
void exact(const std::vector<T>& want, const std::vector<T>& got, const char* what) {
  expect(want.size() == got.size() && std::memcmp(want.data(), got.data(), want.size() * sizeof(T)) == 0,
         std::string(what) + ": not bit-exact");
}

GPU_TEST(rms_norm_f32_and_bf16) {
  HipOps hip;
  Device dev;
  const int64_t rows = 5, cols = 4097;
  std::vector<float> x = gaussian(1, rows * cols, 3.0f), w = gaussian(2, cols);
  const Tensor xd = dev.upload(DType::F32, {rows, cols}, x), wd = dev.upload(DType::F32, {cols}, w);
  const Tensor out = dev.empty(DType::F32, {rows, cols});
  hip.rmsNorm(xd, wd, 1e-6f, 1.0f, out);
  std::vector<float> want(x.size());
  oracle_rms_norm(x.data(), nullptr, w.data(), want.data(), rows, cols, 1e-6f, 1.0f, 1);
  close_f32(want, dev.download<float>(out), "rmsNorm f32");

  const int64_t r2 = 8, c2 = 4096;
  std::vector<uint16_t> xb = to_bf16(gaussian(3, r2 * c2));
  std::vector<float> w2 = gaussian(4, c2);
  const Tensor xbd = dev.upload(DType::BF16, {r2, c2}, xb), w2d = dev.upload(DType::F32, {c2}, w2);
  const Tensor outb = dev.empty(DType::BF16, {r2, c2});
  hip.rmsNorm(xbd, w2d, 1e-5f, 0.0f, outb);
  std::vector<float> xf = from_bf16(xb), wantf(xf.size());
  oracle_rms_norm(xf.data(), nullptr, w2.data(), wantf.data(), r2, c2, 1e-5f, 0.0f, 1);
  within_ulp(to_bf16(wantf), dev.download<uint16_t>(outb), "rmsNorm bf16");
}

// groupRmsNorm: each of a row's groups normed on its own with its slice of
// the weights (ops/HipNormalisation.scala:133-158)
GPU_TEST(group_rms_norm) {
  HipOps hip;
  Device dev;
  const int64_t rows = 6, groups = 3, width = 1024, cols = groups * width;
  std::vector<float> x = gaussian(21, rows * cols, 2.0f), w = gaussian(22, cols);
  const Tensor xd = dev.upload(DType::F32, {rows, cols}, x), wd = dev.upload(DType::F32, {cols}, w);
  const Tensor out = dev.empty(DType::F32, {rows, cols});
  hip.groupRmsNorm(xd, wd, (int)groups, 1e-6f, 0.5f, out);
  std::vector<float> want(x.size());
  oracle_rms_norm(x.data(), nullptr, w.data(), want.data(), rows * groups, width, 1e-6f, 0.5f, (int)groups);
  close_f32(want, dev.download<float>(out), "groupRmsNorm f32");
}

GPU_TEST(adaln_bf16_two_samples) {
  HipOps hip;
  Device dev;
  const int64_t rows = 64, cols = 3072, per = 32;
  std::vector<uint16_t> xb = to_bf16(gaussian(5, rows * cols));
  std::vector<float> scale = gaussian(6, 2 * cols, 0.1f), shift = gaussian(7, 2 * cols, 0.1f);
  const Tensor x = dev.upload(DType::BF16, {rows, cols}, xb);
  const Tensor sc = dev.upload(DType::F32, {2, cols}, scale), sh = dev.upload(DType::F32, {2, cols}, shift);
  const Tensor out = dev.empty(DType::BF16, {rows, cols});
  hip.layerNormModulate(x, sc, sh, 1e-6f, out, per);
  std::vector<float> xf = from_bf16(xb), normed(xf.size()), want(xf.size());
  oracle_layer_norm(xf.data(), nullptr, nullptr, normed.data(), rows, cols, 1e-6f);
  for (int s = 0; s < 2; ++s)
    oracle_modulate(normed.data() + s * per * cols, scale.data() + s * cols, shift.data() + s * cols,
                    want.data() + s * per * cols, per, cols);
  within_ulp(to_bf16(want), dev.download<uint16_t>(out), "layerNormModulate bf16");
}

GPU_TEST(activations_and_gated) {
  HipOps hip;
  Device dev;
  const int64_t n = 100003;
  std::vector<float> g = gaussian(8, n, 3.0f), u = gaussian(9, n);
  std::vector<uint16_t> gb = to_bf16(g);
  const Tensor gbd = dev.upload(DType::BF16, {n}, gb), outb = dev.empty(DType::BF16, {n});
  hip.activation(Activation::GeluTanh, gbd, outb);
  std::vector<float> gf = from_bf16(gb), want(n);
  oracle_activation(1, 1.0f, gf.data(), want.data(), n);
  within_ulp(to_bf16(want), dev.download<uint16_t>(outb), "GELU-tanh bf16");
  const Tensor gd = dev.upload(DType::F32, {n}, g), ud = dev.upload(DType::F32, {n}, u);
  const Tensor out = dev.empty(DType::F32, {n});
  hip.gated(Activation::Silu, gd, ud, out);
  std::vector<float> want2(n);
  oracle_gated(0, g.data(), u.data(), want2.data(), n);
  close_f32(want2, dev.download<float>(out), "SwiGLU f32");
}

GPU_TEST(gated_residuals_per_sample) {
  HipOps hip;
  Device dev;
  const int64_t rows = 48, cols = 3072, per = 24;
  std::vector<float> x = gaussian(10, rows * cols), y = gaussian(11, rows * cols), gate = gaussian(12, 2 * cols);
  const Tensor xd = dev.upload(DType::F32, {rows, cols}, x), yd = dev.upload(DType::F32, {rows, cols}, y);
  hip.gatedAdd(xd, yd, dev.upload(DType::F32, {2, cols}, gate), per);
  oracle_gated_add(x.data(), y.data(), gate.data(), rows, cols, per);
  close_f32(x, dev.download<float>(xd), "gatedAdd per sample");
}

GPU_TEST(rope_neox_f32) {
  HipOps hip;
  Device dev;
  const int tokens = 37, heads = 3, dim = 128;
  std::vector<float> x = gaussian(13, (size_t)tokens * heads * dim);
  std::vector<int32_t> positions(tokens);
  for (int t = 0; t < tokens; ++t) positions[t] = (t * 131) % 4096;
  const Tensor xd = dev.upload(DType::F32, {tokens, heads, dim}, x);
  const Tensor pd = dev.upload(DType::I32, {tokens}, positions), out = dev.empty(DType::F32, {tokens, heads, dim});
  hip.rope(xd, pd, Rope{1e6f, dim, RopeLayout::Neox, {}}, out);
  std::vector<float> want(x.size());
  const int32_t s[4] = {0, 0, 0, 0};
  oracle_rope(x.data(), positions.data(), want.data(), tokens, heads, dim, dim, 1e6f, 0, 0, s);
  close_f32(want, dev.download<float>(out), "rope NeoX f32");
}

GPU_TEST(q8_0_embedding_bit_exact) {
  HipOps hip;
  Device dev;
  const int64_t vocab = 300, cols = 512, count = 77, row_bytes = cols / 32 * 34;
  std::mt19937_64 rng(14);
  std::vector<uint8_t> table((size_t)(vocab * row_bytes));
  for (size_t i = 0; i < table.size(); ++i) table[i] = (uint8_t)rng();
  for (int64_t b = 0; b < vocab * cols / 32; ++b) {  // finite fp16 scales
    const uint16_t d = oracle_f32_to_f16(std::ldexp(1.0f + (float)(rng() % 1000) / 1000.0f, -8));
    std::memcpy(&table[(size_t)(b * 34)], &d, 2);
  }
  std::vector<int32_t> ids(count);
  for (auto& id : ids) id = (int32_t)(rng() % vocab);
  const StoredTable t{dev.upload(DType::U8, {vocab, row_bytes}, table), &StorageType::named("Q8_0"), cols};
  const Tensor out = dev.empty(DType::BF16, {count, cols});
  hip.embedding(t, dev.upload(DType::I32, {count}, ids), out);
  std::vector<float> want((size_t)(count * cols));
  expect(oracle_embedding_q8_0(table.data(), vocab, cols, ids.data(), count, want.data()) == -1, "ids in range");
  exact(to_bf16(want), dev.download<uint16_t>(out), "Q8_0 embedding bf16");
}

GPU_TEST(convrot_four_bit_decode_bit_exact) {
  HipOps hip;
  Device dev;
  const int64_t rows = 9, cols = 768, group = 32;
  std::mt19937_64 rng(15);
  std::vector<uint8_t> codes((size_t)(rows * cols / 2)), relative((size_t)(rows * cols / group));
  for (auto& c : codes) c = (uint8_t)rng();
  for (auto& r : relative) r = (uint8_t)(0x58 + rng() % 0x1f);
  std::vector<float> codebook = gaussian(16, 16, 0.5f), scales(rows);
  for (auto& s : scales) s = 1e-4f + 1e-3f * (float)(rng() % 1000) / 1000.0f;
  const ConvRotLevels levels{dev.upload(DType::F32, {16}, codebook),
                             dev.upload(DType::U8, {rows, cols / group}, relative), (int)group};
  const RotatedTable w = hip.rotated(dev.upload(DType::I8, {rows, cols / 2}, codes),
                                     ConvRotParts{dev.upload(DType::F32, {rows}, scales), levels});
  const Tensor out = dev.empty(DType::BF16, {rows, cols});
  hip.convert(w, out);
  std::vector<float> want((size_t)(rows * cols));
  oracle_convrot_rows(codes.data(), scales.data(), rows, codebook.data(), relative.data(), group, cols, 0, rows,
                      want.data());
  exact(to_bf16(want), dev.download<uint16_t>(out), "ConvRot 4-bit decode");
}

GPU_TEST(fp8_convert_bit_exact) {
  HipOps hip;
  Device dev;
  std::vector<uint8_t> codes(256);
  for (int i = 0; i < 256; ++i) codes[i] = (uint8_t)i;
  const Tensor out = dev.empty(DType::F32, {256});
  hip.convert(dev.upload(DType::F8E4M3, {256}, codes), out);
  std::vector<float> got = dev.download<float>(out);
  for (int i = 0; i < 256; ++i) {
    const float want = oracle_f8e4m3(i);
    expect((std::isnan(want) && std::isnan(got[i])) || std::memcmp(&want, &got[i], 4) == 0,
           "fp8 code " + std::to_string(i));
  }
}

// Callers write over an input (out aliases x): per-head rmsNorm in place
// (models/DenseDecoder.scala:834-851), modulate(normed, ..., normed)
// (models/Wan.scala:432), activation(up, up) (:474) and gated(gate, up,
// gate) (models/DenseDecoder.scala:927).
GPU_TEST(outputs_may_alias_their_inputs) {
  HipOps hip;
  Device dev;
  const int64_t rows = 4096 * 8 / 64, cols = 128;
  std::vector<float> x = gaussian(17, rows * cols), w = gaussian(18, cols);
  const Tensor xd = dev.upload(DType::F32, {rows, cols}, x), wd = dev.upload(DType::F32, {cols}, w);
  hip.rmsNorm(xd, wd, 1e-6f, 0.0f, xd);
  std::vector<float> want(x.size());
  oracle_rms_norm(x.data(), nullptr, w.data(), want.data(), rows, cols, 1e-6f, 0.0f, 1);
  close_f32(want, dev.download<float>(xd), "rmsNorm in place");

  const int64_t r2 = 6, c2 = 3072;
  std::vector<float> n = gaussian(19, r2 * c2), scale = gaussian(20, c2, 0.1f), shift = gaussian(21, c2, 0.1f);
  const Tensor nd = dev.upload(DType::F32, {r2, c2}, n);
  hip.modulate(nd, dev.upload(DType::F32, {c2}, scale), dev.upload(DType::F32, {c2}, shift), nd);
  std::vector<float> want2(n.size());
  oracle_modulate(n.data(), scale.data(), shift.data(), want2.data(), r2, c2);
  close_f32(want2, dev.download<float>(nd), "modulate in place");

  const int64_t count = 3 * 14336;
  std::vector<uint16_t> up = to_bf16(gaussian(22, count, 2.0f));
  const Tensor upd = dev.upload(DType::BF16, {count}, up);
  hip.activation(Activation::GeluTanh, upd, upd);
  std::vector<float> upf = from_bf16(up), want3(count);
  oracle_activation(1, 1.0f, upf.data(), want3.data(), count);
  within_ulp(to_bf16(want3), dev.download<uint16_t>(upd), "activation in place");

  std::vector<float> g = gaussian(23, count), u = gaussian(24, count);
  const Tensor gd = dev.upload(DType::F32, {count}, g);
  hip.gated(Activation::Silu, gd, dev.upload(DType::F32, {count}, u), gd);
  std::vector<float> want4(count);
  oracle_gated(0, g.data(), u.data(), want4.data(), count);
  close_f32(want4, dev.download<float>(gd), "gated into its gate");
}

GPU_TEST(norms_modulation_and_residual_gates) {
  HipOps hip;
  Device dev;
  const int64_t rows = 6, cols = 3072;
  std::vector<float> x = gaussian(30, rows * cols), y = gaussian(31, rows * cols), w = gaussian(32, cols),
                     b = gaussian(33, cols);
  // addRmsNorm: x += y written back, then the norm of the sum
  const Tensor xd = dev.upload(DType::F32, {rows, cols}, x), out = dev.empty(DType::F32, {rows, cols});
  hip.addRmsNorm(xd, dev.upload(DType::F32, {rows, cols}, y), RowNorm{dev.upload(DType::F32, {cols}, w), 1e-6f, 0.0f, out});
  std::vector<float> summed = x, want(x.size());
  oracle_rms_norm(summed.data(), y.data(), w.data(), want.data(), rows, cols, 1e-6f, 0.0f, 1);
  exact(summed, dev.download<float>(xd), "addRmsNorm x += y");
  close_f32(want, dev.download<float>(out), "addRmsNorm");
  // layerNorm with weight and bias, then modulate
  const Tensor wd = dev.upload(DType::F32, {cols}, w), bd = dev.upload(DType::F32, {cols}, b);
  const Tensor x2 = dev.upload(DType::F32, {rows, cols}, x), ln = dev.empty(DType::F32, {rows, cols});
  hip.layerNorm(x2, &wd, &bd, 1e-5f, ln);
  std::vector<float> want_ln(x.size());
  oracle_layer_norm(x.data(), w.data(), b.data(), want_ln.data(), rows, cols, 1e-5f);
  close_f32(want_ln, dev.download<float>(ln), "layerNorm");
  const Tensor mod = dev.empty(DType::F32, {rows, cols});
  hip.modulate(x2, wd, bd, mod);
  std::vector<float> want_mod(x.size());
  oracle_modulate(x.data(), w.data(), b.data(), want_mod.data(), rows, cols);
  close_f32(want_mod, dev.download<float>(mod), "modulate");
  // per-row chunk tables: modulateChunks, gatedAddChunk, rowGatedAdd
  const int chunks = 6;
  std::vector<float> table = gaussian(34, rows * chunks * cols, 0.1f), g = gaussian(35, rows);
  const Tensor td = dev.upload(DType::F32, {rows, chunks * cols}, table);
  const Tensor mc = dev.empty(DType::F32, {rows, cols});
  hip.modulateChunks(x2, td, 3, 4, mc);
  std::vector<float> want_mc(x.size());
  oracle_modulate_chunks(x.data(), table.data(), want_mc.data(), rows, cols, chunks, 3, 4);
  close_f32(want_mc, dev.download<float>(mc), "modulateChunks");
  const Tensor x3 = dev.upload(DType::F32, {rows, cols}, x), yd = dev.upload(DType::F32, {rows, cols}, y);
  hip.gatedAddChunk(x3, yd, td, 5);
  std::vector<float> want_gc = x;
  oracle_gated_add_chunk(want_gc.data(), y.data(), table.data(), rows, cols, chunks, 5);
  close_f32(want_gc, dev.download<float>(x3), "gatedAddChunk");
  const Tensor x4 = dev.upload(DType::F32, {rows, cols}, x);
  hip.rowGatedAdd(x4, yd, dev.upload(DType::F32, {rows}, g));
  std::vector<float> want_rg = x;
  oracle_row_gated_add(want_rg.data(), y.data(), g.data(), rows, cols);
  close_f32(want_rg, dev.download<float>(x4), "rowGatedAdd");
}

GPU_TEST(quantize_and_scaled_activation) {
  HipOps hip;
  Device dev;
  const int64_t blocks = 515;
  std::vector<float> x = gaussian(36, blocks * 32, 2.0f);
  std::vector<int8_t> codes0(blocks * 32);
  const Tensor xd = dev.upload(DType::F32, {blocks * 32}, x);
  const Tensor codes = dev.upload(DType::I8, {blocks * 32}, codes0);
  const Tensor scales = dev.empty(DType::F32, {blocks}), sums = dev.empty(DType::F32, {blocks});
  hip.quantizeTo(xd, blocks, QuantizedOutput{codes.data, static_cast<float*>(scales.data), static_cast<float*>(sums.data)});
  std::vector<int8_t> want_codes(blocks * 32);
  std::vector<float> want_scales(blocks), want_sums(blocks);
  oracle_quantize_x(x.data(), want_codes.data(), want_scales.data(), want_sums.data(), blocks);
  exact(want_codes, dev.download<int8_t>(codes), "quantize codes");
  exact(want_scales, dev.download<float>(scales), "quantize scales");
  exact(want_sums, dev.download<float>(sums), "quantize sums");
  const Tensor out = dev.empty(DType::F32, {blocks * 32});
  hip.scaledActivation(Activation::GeluErf, 0.5f, xd, out);
  std::vector<float> want(x.size());
  oracle_activation(2, 0.5f, x.data(), want.data(), (int64_t)x.size());
  close_f32(want, dev.download<float>(out), "scaledActivation GELU-erf");
}

GPU_TEST(rope_tables_and_wan_3d) {
  HipOps hip;
  Device dev;
  const int tokens = 9, heads = 3, dim = 128, pairs = 48;
  std::vector<float> x = gaussian(37, (size_t)tokens * heads * dim), c(tokens * pairs), sn(tokens * pairs);
  for (int i = 0; i < tokens * pairs; ++i) {
    c[i] = std::cos(0.01f * (float)i);
    sn[i] = std::sin(0.01f * (float)i);
  }
  const Tensor xd = dev.upload(DType::F32, {tokens, heads, dim}, x), out = dev.empty(DType::F32, {tokens, heads, dim});
  hip.ropeTable(xd, dev.upload(DType::F32, {tokens, pairs}, c), dev.upload(DType::F32, {tokens, pairs}, sn), out, true);
  std::vector<float> want(x.size());
  oracle_rope_table(x.data(), c.data(), sn.data(), want.data(), tokens, heads, dim, pairs, 0, 1);
  close_f32(want, dev.download<float>(out), "ropeTable halves");
  // Wan's 3-D grid 2 x 3 x 5, in place on bf16
  const int frames = 2, grid_rows = 3, grid_cols = 5, wan_tokens = frames * grid_rows * grid_cols;
  std::vector<uint16_t> xb = to_bf16(gaussian(38, (size_t)wan_tokens * 2 * dim));
  const Tensor wd = dev.upload(DType::BF16, {wan_tokens, 2, dim}, xb);
  hip.rope3d(wd, frames, grid_rows, grid_cols, wd);
  std::vector<float> wc((size_t)wan_tokens * dim / 2), ws(wc.size()), xf = from_bf16(xb), wwant(xf.size());
  oracle_wan_angles(frames, grid_rows, grid_cols, dim, 10000.0, wc.data(), ws.data());
  oracle_rope_table(xf.data(), wc.data(), ws.data(), wwant.data(), wan_tokens, 2, dim, dim / 2, 0, 0);
  within_ulp(to_bf16(wwant), dev.download<uint16_t>(wd), "rope3d bf16 in place");
}

GPU_TEST(query_key_norm_rope_f32) {
  HipOps hip;
  Device dev;
  const int tokens = 11, qh = 4, kh = 2, dim = 128;
  std::vector<float> q = gaussian(39, (size_t)tokens * qh * dim, 2.0f), k = gaussian(40, (size_t)tokens * kh * dim, 2.0f);
  std::vector<float> qw = gaussian(41, dim, 0.1f), kw = gaussian(42, dim, 0.1f);
  for (float& v : qw) v += 1.0f;
  for (float& v : kw) v += 1.0f;
  std::vector<int32_t> positions(tokens);
  for (int t = 0; t < tokens; ++t) positions[t] = 100 + 7 * t;
  const Rope rope{1e6f, dim, RopeLayout::Neox, {}};
  const QueryKeyNorms norms{dev.upload(DType::F32, {dim}, qw), dev.upload(DType::F32, {dim}, kw), 1e-6f, 0.0f, rope};
  const Tensor rq = dev.empty(DType::F32, {tokens, qh, dim}), rk = dev.empty(DType::F32, {tokens, kh, dim});
  hip.queryKeyNormRope(dev.upload(DType::F32, {tokens, qh, dim}, q), dev.upload(DType::F32, {tokens, kh, dim}, k),
                       norms, dev.upload(DType::I32, {tokens}, positions), rq, rk);
  // the reference's composition: rmsNorm per head (F32 written), then rope
  const int32_t s[4] = {0, 0, 0, 0};
  auto composed = [&](std::vector<float> v, const std::vector<float>& w, int heads) {
    std::vector<float> normed(v.size()), rotated(v.size());
    oracle_rms_norm(v.data(), nullptr, w.data(), normed.data(), (int64_t)tokens * heads, dim, 1e-6f, 0.0f, 1);
    oracle_rope(normed.data(), positions.data(), rotated.data(), tokens, heads, dim, dim, 1e6f, 0, 0, s);
    return rotated;
  };
  close_f32(composed(q, qw, qh), dev.download<float>(rq), "queryKeyNormRope queries");
  close_f32(composed(k, kw, kh), dev.download<float>(rk), "queryKeyNormRope keys");
}

GPU_TEST(attention_inputs_equal_their_steps) {
  // the fused gated step against split, norms + rope and the cache write
  // launched one by one (FusedOpsTests.scala:406-499 asks the same), in F32:
  // with BF16 the steps would round the turned keys to BF16 before F16
  HipOps hip;
  Device dev;
  const int tokens = 21, qh = 8, kh = 2, dim = 128, page = 16, pages = 4;
  const int64_t start = 5;
  std::vector<float> qg = gaussian(43, (size_t)tokens * qh * 2 * dim, 2.0f);
  std::vector<float> k = gaussian(44, (size_t)tokens * kh * dim, 2.0f);
  std::vector<float> v = gaussian(45, (size_t)tokens * kh * dim);
  std::vector<float> w = gaussian(46, dim, 0.1f);
  for (float& x : w) x += 1.0f;
  std::vector<int32_t> positions(tokens), table = {2, 0, 3, 1};
  for (int t = 0; t < tokens; ++t) positions[t] = (int32_t)start + t;
  std::vector<uint16_t> blank((size_t)pages * page * kh * dim, 0);
  const Tensor wd = dev.upload(DType::F32, {dim}, w);
  const QueryKeyNorms norms{wd, wd, 1e-6f, 0.0f, Rope{1e6f, dim, RopeLayout::Neox, {}}};
  const Tensor qgd = dev.upload(DType::F32, {tokens, qh, 2 * dim}, qg), kd = dev.upload(DType::F32, {tokens, kh, dim}, k);
  const Tensor vd = dev.upload(DType::F32, {tokens, kh, dim}, v), pos = dev.upload(DType::I32, {tokens}, positions);
  const Tensor pt = dev.upload(DType::I32, {pages}, table);
  auto make_cache = [&] {
    return KvCache::of(dev.upload(DType::F16, {pages, page, kh, dim}, blank),
                       dev.upload(DType::F16, {pages, kh, dim, page}, blank), page);
  };
  // fused
  const KvCache fused_cache = make_cache();
  const Tensor queries = dev.empty(DType::F32, {tokens, qh, dim}), gate = dev.empty(DType::F32, {tokens, qh, dim});
  const Tensor rkeys = dev.empty(DType::F32, {tokens, kh, dim}), rq = dev.empty(DType::F32, {tokens, qh, dim});
  hip.attentionInputs(qgd, kd, vd, norms, pos, fused_cache, pt, start, queries, gate, rkeys, rq);
  // step by step
  const KvCache steps_cache = make_cache();
  const Tensor q2 = dev.empty(DType::F32, {tokens, qh, dim}), g2 = dev.empty(DType::F32, {tokens, qh, dim});
  const Tensor rq2 = dev.empty(DType::F32, {tokens, qh, dim}), rk2 = dev.empty(DType::F32, {tokens, kh, dim});
  hip.splitHalves(qgd, q2, g2);
  hip.queryKeyNormRope(q2, kd, norms, pos, rq2, rk2);
  hip.cacheWrite(rk2, vd, steps_cache, pt, start);
  exact(dev.download<float>(g2), dev.download<float>(gate), "the gate half");
  exact(dev.download<float>(rq2), dev.download<float>(rq), "rotated queries");
  exact(dev.download<uint16_t>(steps_cache.keys), dev.download<uint16_t>(fused_cache.keys), "cached keys");
  exact(dev.download<uint16_t>(steps_cache.values), dev.download<uint16_t>(fused_cache.values), "cached values");
  // queryKeyNormRopeCache: the same without the gate
  const KvCache nogate_cache = make_cache();
  const Tensor rq3 = dev.empty(DType::F32, {tokens, qh, dim});
  hip.queryKeyNormRopeCache(q2, kd, vd, norms, pos, nogate_cache, pt, start, rq3);
  exact(dev.download<float>(rq2), dev.download<float>(rq3), "queryKeyNormRopeCache queries");
  exact(dev.download<uint16_t>(steps_cache.keys), dev.download<uint16_t>(nogate_cache.keys), "queryKeyNormRopeCache keys");
}

GPU_TEST(stored_and_rotated_tables) {
  HipOps hip;
  Device dev;
  // Q4_K: the whole table decoded to BF16, bit-exact
  const StorageType& q4k = StorageType::named("Q4_K");
  const int64_t rows = 12, cols = 512, row_bytes = q4k.rowBytes(cols);
  std::mt19937_64 rng(47);
  std::vector<uint8_t> bytes((size_t)(rows * row_bytes));
  for (auto& b : bytes) b = (uint8_t)rng();
  for (int64_t blk = 0; blk < rows * cols / 256; ++blk) {  // finite d and dmin
    const uint16_t d = oracle_f32_to_f16(1e-3f * (float)(1 + rng() % 100)),
                   dm = oracle_f32_to_f16(1e-3f * (float)(1 + rng() % 100));
    std::memcpy(&bytes[(size_t)(blk * 144)], &d, 2);
    std::memcpy(&bytes[(size_t)(blk * 144 + 2)], &dm, 2);
  }
  const StoredTable t{dev.upload(DType::U8, {rows, row_bytes}, bytes), &q4k, cols};
  const Tensor out = dev.empty(DType::BF16, {rows, cols});
  hip.dequantize(t, out);
  std::vector<float> want((size_t)(rows * cols));
  for (int64_t r = 0; r < rows; ++r)
    expect(oracle_decode_row(q4k.ggmlId, bytes.data() + r * row_bytes, cols, want.data() + r * cols) == 0, "decode");
  exact(to_bf16(want), dev.download<uint16_t>(out), "Q4_K dequantize");
  // an int8 rotated weight gathered to F32 (the BF16 value widened)
  const int64_t rr = 7, rc = 512;
  std::vector<int8_t> codes((size_t)(rr * rc));
  for (auto& c : codes) c = (int8_t)(rng() % 255 - 127);
  std::vector<float> scales(rr);
  for (auto& s : scales) s = 1e-3f * (float)(1 + rng() % 10);
  const RotatedTable w = hip.rotated(dev.upload(DType::I8, {rr, rc}, codes), ConvRotParts{dev.upload(DType::F32, {rr}, scales), {}});
  std::vector<int32_t> ids = {6, 0, 3, 3};
  const Tensor got = dev.empty(DType::F32, {4, rc});
  hip.embedding(w, dev.upload(DType::I32, {4}, ids), got);
  std::vector<float> want_rows((size_t)(4 * rc));
  expect(oracle_convrot_embedding(reinterpret_cast<const uint8_t*>(codes.data()), scales.data(), rr, nullptr, nullptr,
                                  0, rr, rc, ids.data(), 4, want_rows.data()) == -1, "ids in range");
  exact(want_rows, dev.download<float>(got), "rotated embedding");
  // F32 -> BF16
  std::vector<float> x = gaussian(48, 1000, 5.0f);
  const Tensor xb = dev.empty(DType::BF16, {1000});
  hip.convert(dev.upload(DType::F32, {1000}, x), xb);
  exact(to_bf16(x), dev.download<uint16_t>(xb), "convert F32 to BF16");
}

// ops/HipBase.scala:117-214 and FusedOpsTests.scala:96-176: once int8
// products run, the F32 norm and `gated` write their output quantized too,
// the same as quantizing it afterwards; any launch after makes it stale.
GPU_TEST(the_int8_side_output_bookkeeping) {
  HipOps hip;
  Device dev;
  const int64_t rows = 4, cols = 4096;
  std::vector<float> x = gaussian(50, rows * cols, 2.0f), w = gaussian(51, cols, 0.1f);
  for (float& v : w) v += 1.0f;
  const Tensor xd = dev.upload(DType::F32, {rows, cols}, x), wd = dev.upload(DType::F32, {cols}, w);
  const Tensor out = dev.empty(DType::F32, {rows, cols});
  hip.rmsNorm(xd, wd, 1e-6f, 0.0f, out);
  expect(!hip.quantizesX() && !hip.quantizedInput(out, rows, cols), "no side output before int8 products run");
  hip.quantize(xd, rows, cols);  // the first int8 product
  expect(hip.quantizesX(), "quantize marks that int8 products run");
  hip.rmsNorm(xd, wd, 1e-6f, 0.0f, out);
  const std::optional<QuantizedOutput> side = hip.quantizedInput(out, rows, cols);
  expect(side.has_value(), "the norm wrote its output quantized");
  auto grab = [&](const QuantizedOutput& q, int64_t values) {
    std::vector<int8_t> codes((size_t)values);
    std::vector<float> scales((size_t)(values / 32)), sums((size_t)(values / 32));
    hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
    hip_check(hipMemcpy(codes.data(), q.codes, codes.size(), hipMemcpyDeviceToHost), "hipMemcpy");
    hip_check(hipMemcpy(scales.data(), q.scales, scales.size() * 4, hipMemcpyDeviceToHost), "hipMemcpy");
    hip_check(hipMemcpy(sums.data(), q.sums, sums.size() * 4, hipMemcpyDeviceToHost), "hipMemcpy");
    return std::make_tuple(codes, scales, sums);
  };
  const auto written = grab(*side, rows * cols);
  // rows 2-3 alone: the same blocks, from where they start
  const Tensor tail{DType::F32, {2, cols}, static_cast<float*>(out.data) + 2 * cols};
  const auto tail_side = grab(*hip.quantizedInput(tail, 2, cols), 2 * cols);
  expect(std::equal(std::get<0>(tail_side).begin(), std::get<0>(tail_side).end(),
                    std::get<0>(written).begin() + 2 * cols), "rows 2-3 of the side output");
  const auto fresh = grab(hip.quantize(out, rows, cols), rows * cols);
  exact(std::get<0>(fresh), std::get<0>(written), "side output codes");
  exact(std::get<1>(fresh), std::get<1>(written), "side output scales");
  exact(std::get<2>(fresh), std::get<2>(written), "side output sums");
  expect(!hip.quantizedInput(out, rows, cols), "a launch after the norm makes its side output stale");
  // gated writes its output quantized too; productInput finds it
  std::vector<float> g = gaussian(52, rows * cols), u = gaussian(53, rows * cols);
  const Tensor gout = dev.empty(DType::F32, {rows, cols});
  hip.gated(Activation::Silu, dev.upload(DType::F32, {rows, cols}, g), dev.upload(DType::F32, {rows, cols}, u), gout);
  const int64_t before = hip.deviceWrites();
  const auto product = grab(hip.productInput(gout, rows, cols), rows * cols);
  expect(hip.deviceWrites() == before, "productInput read the side output without a launch");
  const auto requantized = grab(hip.quantize(gout, rows, cols), rows * cols);
  exact(std::get<0>(requantized), std::get<0>(product), "gated side output codes");
  exact(std::get<1>(requantized), std::get<1>(product), "gated side output scales");
}

}  // namespace

// --gguf FILE...: each file as the C++ reader sees it, one line a fact
// (version and alignment, then each tensor by name, then each unsupported
// one), or the refusal; tests/test_cpp_host.py holds it to the Python reader.
int summarize_gguf(int count, char** paths) {
  for (int i = 0; i < count; ++i) {
    std::printf("file %s\n", paths[i]);
    try {
      const gguf::File f = gguf::File::open(paths[i]);
      std::printf("version %d alignment %lld\n", f.version(), (long long)f.alignment());
      for (const auto& [name, t] : f.tensors()) {
        std::string shape;
        for (int64_t d : t.shape) shape += (shape.empty() ? "" : ",") + std::to_string(d);
        std::printf("tensor %s %s [%s] %lld %lld\n", name.c_str(), t.type->name, shape.c_str(),
                    (long long)t.fileOffset, (long long)t.byteSize());
      }
      for (const auto& [name, reason] : f.unsupported()) std::printf("unsupported %s: %s\n", name.c_str(), reason.c_str());
    } catch (const gguf::FormatError& e) {
      std::printf("refused %s\n", e.what());
    }
  }
  return 0;
}

// --gguf-embed FILE NAME ID...: the table NAME gathered to F32 on the GPU at
// the ids, printed as one FNV-1a hash of the output's bytes.
int embed_gguf(int argc, char** argv) {
  const gguf::File f = gguf::File::open(argv[0]);
  const gguf::DeviceTable t = f.table(argv[1]);
  std::vector<int32_t> ids;
  for (int i = 2; i < argc; ++i) ids.push_back(std::atoi(argv[i]));
  HipOps hip;
  Device dev;
  const int64_t cols = t.table().cols, count = (int64_t)ids.size();
  const Tensor out = dev.empty(DType::F32, {count, cols});
  hip.embedding(t.table(), dev.upload(DType::I32, {count}, ids), out);
  const std::vector<uint8_t> bytes = dev.download<uint8_t>(out);
  uint64_t h = 1469598103934665603ull;
  for (uint8_t b : bytes) h = (h ^ b) * 1099511628211ull;
  std::printf("embedding %llu\n", (unsigned long long)h);
  return 0;
}

int main(int argc, char** argv) {
  if (argc > 1 && std::string(argv[1]) == "--gguf") return summarize_gguf(argc - 2, argv + 2);
  if (argc > 3 && std::string(argv[1]) == "--gguf-embed") return embed_gguf(argc - 2, argv + 2);
  const bool gpu = argc > 1 && std::string(argv[1]) == "--gpu";
  if (argc < 2 || (!gpu && std::string(argv[1]) != "--checks")) {
    std::printf("usage: test_host --checks | --gpu\n");
    return 2;
  }
  int count = 0;
  for (auto& [name, body] : registry(gpu)) {
    ++count;
    std::printf("[%s] %s ... ", gpu ? "gpu" : "cpu", name.c_str());
    std::fflush(stdout);
    try {
      body();
      std::printf("ok\n");
    } catch (const std::exception& e) {
      ++failures;
      std::printf("FAILED: %s\n", e.what());
    }
    std::fflush(stdout);
  }
  std::printf("%d tests, %d failed\n", count, failures);
  return failures ? 1 : 0;
}
