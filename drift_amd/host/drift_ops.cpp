// The C++ host side of the fused layer kernels: object Ops's checks and the
// HipOps methods of this path, over libdrift_kernels' C ABI.
#include "drift_ops.hpp"

#include <algorithm>
#include <numeric>
#include <sstream>

#include <hip/hip_runtime_api.h>

#include "../../include/drift_kernels.h"

namespace drift {

// ---------------------------------------------------------------- basics

const char* name(DType dtype) {
  switch (dtype) {
    case DType::F32: return "F32";
    case DType::F16: return "F16";
    case DType::BF16: return "BF16";
    case DType::I32: return "I32";
    case DType::I8: return "I8";
    case DType::U8: return "U8";
    case DType::F8E4M3: return "F8_E4M3";
  }
  return "?";
}

int64_t elementBytes(DType dtype) {
  switch (dtype) {
    case DType::F32:
    case DType::I32: return 4;
    case DType::F16:
    case DType::BF16: return 2;
    default: return 1;
  }
}

int64_t Shape::elementCount() const {
  return std::accumulate(dimensions.begin(), dimensions.end(), (int64_t)1, std::multiplies<int64_t>());
}

std::string Shape::str() const {
  std::string s = "[";
  for (size_t i = 0; i < dimensions.size(); ++i) {
    if (i) s += "×";
    s += std::to_string(dimensions[i]);
  }
  return s + "]";
}

HipException::HipException(const std::string& entry_, int code_, const std::string& reason)
    : std::runtime_error(entry_ + " failed (" + std::to_string(code_) + "): " + reason), entry(entry_), code(code_) {}

namespace {

// Scala's require: IllegalArgumentException("requirement failed: " + message).
[[noreturn]] void refuse(const std::string& message) { throw std::invalid_argument("requirement failed: " + message); }

void require(bool condition, const std::string& message) {
  if (!condition) refuse(message);
}

template <typename... Parts>
std::string text(const Parts&... parts) {
  std::ostringstream s;
  (s << ... << parts);
  return s.str();
}

bool isBf16(const Tensor& t) { return t.dtype == DType::BF16; }
template <typename T>
T* at(const Tensor& t) {
  return static_cast<T*>(t.data);
}
template <typename T>
T* at(const Tensor* t) {
  return t ? static_cast<T*>(t->data) : nullptr;
}

}  // namespace

KvCache KvCache::of(const Tensor& keys, const Tensor& values, int pageSize) {
  require(pageSize > 0 && pageSize % 16 == 0, text("pages of ", pageSize, " tokens: not a multiple of 16"));
  require(keys.dtype == DType::F16 && values.dtype == DType::F16, "the cache is F16");
  require(keys.shape.rank() == 4 && values.shape.rank() == 4, "the cache's keys and values are 4-dimensional");
  require(keys.shape[1] == pageSize &&
              values.shape == Shape{keys.shape[0], keys.shape[2], keys.shape[3], (int64_t)pageSize},
          text("cache values ", values.shape.str(), " for keys ", keys.shape.str()));
  return KvCache{keys, values, pageSize};
}

// tensor/DType.scala, GgmlQuants.scala:12-118, KQuants.scala:100-134,
// IQuants.scala:40-80, RocmFp4.scala:75-84, with the GGUF type ids
const std::vector<StorageType>& StorageType::all() {
  static const std::vector<StorageType> types = {
      {"F32", 0, 1, 4, 4},         {"F16", 1, 1, 2, 2},          {"BF16", 30, 1, 2, 2},
      {"Q4_0", 2, 32, 18, 2},      {"Q4_1", 3, 32, 20, 4},       {"Q5_0", 6, 32, 22, 2},
      {"Q5_1", 7, 32, 24, 4},      {"Q8_0", 8, 32, 34, 2},       {"Q4_K", 12, 256, 144, 8},
      {"Q5_K", 13, 256, 176, 8},   {"Q6_K", 14, 256, 210, 2},    {"IQ4_NL", 20, 32, 18, 2},
      {"IQ4_XS", 23, 256, 136, 8}, {"Q4_0_ROCMFP4", 100, 32, 18, 2}, {"Q4_0_ROCMFP4_FAST", 101, 32, 17, 1}};
  return types;
}

const StorageType& StorageType::named(const std::string& wanted) {
  for (const StorageType& t : all())
    if (wanted == t.name) return t;
  refuse(text("no storage type ", wanted));
}

int64_t StorageType::rowBytes(int64_t cols) const {
  require(cols % values == 0, text(cols, " elements are not whole ", name, " blocks of ", values));
  return cols / values * bytes;
}

// ---------------------------------------------------------------- checks

namespace checks {

void requireF32(const char* operation, std::initializer_list<const Tensor*> tensors) {
  for (const Tensor* t : tensors) require(t->dtype == DType::F32, text(operation, " takes F32, not ", name(t->dtype)));
}

void requireSameShape(const char* operation, std::initializer_list<const Tensor*> tensors) {
  bool same = true;
  for (const Tensor* t : tensors) same = same && t->shape == (*tensors.begin())->shape;
  if (same) return;
  std::string shapes;
  for (const Tensor* t : tensors) shapes += (shapes.empty() ? "" : ", ") + t->shape.str();
  refuse(text(operation, " needs equal shapes, got ", shapes));
}

// Same-shape operands of one float type: F32 as the reference's, or BF16.
void checkElementwise(const char* operation, std::initializer_list<const Tensor*> tensors) {
  const Tensor* first = *tensors.begin();
  require(first->dtype == DType::F32 || first->dtype == DType::BF16,
          text(operation, " takes F32 or BF16, not ", name(first->dtype)));
  for (const Tensor* t : tensors)
    require(t->dtype == first->dtype,
            text(operation, " takes one type, not ", name(first->dtype), " and ", name(t->dtype)));
  requireSameShape(operation, tensors);
}

// ops/Ops.scala:76-92: the row count.
int64_t checkRowWise(const char* operation, const Tensor& x, const Tensor& out,
                     std::initializer_list<const Tensor*> rowVectors) {
  checkElementwise(operation, {&x, &out});
  require(x.shape.rank() >= 1, text(operation, " needs at least one dimension"));
  for (const Tensor* vector : rowVectors) {
    requireF32(operation, {vector});
    require(vector->shape == Shape{x.shape.last()},
            text(operation, ": ", vector->shape.str(), " for rows of ", x.shape.last()));
  }
  return x.shape.last() ? x.elementCount() / x.shape.last() : 0;
}

// ops/ElementwiseOps.scala:55-76: x, out [rows, C], table F32 [rows, chunks
// C], every index a chunk.
Chunks checkChunks(const char* operation, const Tensor& x, const Tensor& table, const Tensor& out,
                   std::initializer_list<int> indices) {
  checkElementwise(operation, {&x, &out});
  requireF32(operation, {&table});
  require(x.shape.rank() == 2, text(operation, " takes [rows, C], not ", x.shape.str()));
  const int64_t rows = x.shape[0], channels = x.shape[1];
  const int64_t width = table.shape.rank() > 0 ? table.shape.last() : 0;
  bool ok = table.shape.rank() == 2 && table.shape[0] == rows && channels > 0 && width % channels == 0;
  std::string list;
  for (int i : indices) {
    ok = ok && i >= 0 && i < (channels > 0 ? width / channels : 0);
    list += (list.empty() ? "" : ", ") + std::to_string(i);
  }
  require(ok, text(operation, ": table ", table.shape.str(), " for ", x.shape.str(), ", chunks ArraySeq(", list,
                   ")"));
  return {rows, channels, width / channels};
}

// ops/AttentionOps.scala:185-223
Heads checkRope(const Tensor& x, const Tensor& positions, const Rope& rope, const Tensor& out) {
  checkElementwise("rope", {&x, &out});
  require(x.shape.rank() == 3, text("rope takes [tokens, heads, headDimension], got ", x.shape.str()));
  const int64_t tokens = x.shape[0], heads = x.shape[1], dimension = x.shape[2];
  require(positions.dtype == DType::I32, text("rope positions are I32, not ", name(positions.dtype)));
  if (rope.sections.code == 3) {
    const std::vector<int>& pairs = rope.sections.sizes;
    const int total = std::accumulate(pairs.begin(), pairs.end(), 0);
    std::string list;
    for (int p : pairs) list += (list.empty() ? "" : ", ") + std::to_string(p);
    require(pairs.size() <= 4 && std::all_of(pairs.begin(), pairs.end(), [](int p) { return p > 0; }) &&
                total * 2 == rope.rotaryDimensions,
            text("rope: axes of [", list, "] pairs for ", rope.rotaryDimensions, " rotary values"));
  }
  const int count = rope.sections.positionsPerToken();
  const Shape expected = count == 1 ? Shape{tokens} : Shape{(int64_t)count, tokens};
  require(positions.shape == expected, text("rope positions ", positions.shape.str(), ", expected ", expected.str()));
  require(rope.rotaryDimensions % 2 == 0 && rope.rotaryDimensions <= dimension && rope.rotaryDimensions >= 0,
          text("rope: ", rope.rotaryDimensions, " rotary dimensions in heads of ", dimension));
  return {tokens, heads, dimension};
}

// ops/AttentionOps.scala:129-151
TableRope checkRopeTable(const Tensor& x, const Tensor& cosines, const Tensor& sines, const Tensor& out) {
  checkElementwise("ropeTable", {&x, &out});
  requireF32("ropeTable", {&cosines, &sines});
  require(x.shape.rank() == 3, text("ropeTable takes [tokens, heads, D], not ", x.shape.str()));
  const int64_t tokens = x.shape[0], heads = x.shape[1], d = x.shape[2];
  const int64_t pairs = cosines.shape.rank() ? cosines.shape.last() : 0;
  const bool perHead = cosines.shape.rank() == 3;
  require((cosines.shape == Shape{tokens, pairs} || cosines.shape == Shape{tokens, heads, pairs}) &&
              sines.shape == cosines.shape && 2 * pairs <= d,
          text("ropeTable: tables ", cosines.shape.str(), ", ", sines.shape.str(), " for ", x.shape.str()));
  return {tokens, heads, d, pairs, perHead};
}

// ops/LinearOps.scala:92-106
void checkEmbedding(const Shape& table, const Tensor& ids, const Tensor& out) {
  require(table.rank() == 2, text("an embedding table is [vocabulary, D], not ", table.str()));
  require(ids.dtype == DType::I32 && ids.shape.rank() == 1,
          text("embedding ids are I32 [tokens], not ", name(ids.dtype), " ", ids.shape.str()));
  require(out.dtype == DType::F32 || out.dtype == DType::BF16,
          text("embedding takes F32 or BF16, not ", name(out.dtype)));
  require(out.shape == Shape{ids.shape[0], table.last()},
          text("embedding: out ", out.shape.str(), " for ", ids.shape[0], " rows of ", table.last()));
}

// ops/LinearOps.scala:121-157: the weight `codes` make with `parts`.
RotatedTable checkRotated(const Tensor& codes, const ConvRotParts& parts) {
  require(codes.dtype == DType::I8 && codes.shape.rank() == 2,
          text("rotated: ", name(codes.dtype), " codes ", codes.shape.str()));
  const int64_t n = codes.shape[0];
  const int64_t k = codes.shape[1] * (parts.levels ? 2 : 1);
  require(k % 256 == 0, text("rotated: rows of ", k, " columns"));  // ConvRot.Group
  const int64_t scaleCount = parts.scales.elementCount();
  require(parts.scales.dtype == DType::F32 && (scaleCount == n || (scaleCount == 1 && !parts.levels)),
          text("rotated: ", scaleCount, " ", name(parts.scales.dtype), " scales for ", n, " rows"));
  if (parts.levels) {
    const ConvRotLevels& l = *parts.levels;
    require(l.groupSize > 0 && l.groupSize % 16 == 0 && k % l.groupSize == 0,
            text("rotated: ", k, " columns in groups of ", l.groupSize));
    require(l.codebook.dtype == DType::F32 && l.codebook.elementCount() == 16,
            text("rotated: a codebook ", name(l.codebook.dtype), " ", l.codebook.shape.str()));
    require((l.relative.dtype == DType::F8E4M3 || l.relative.dtype == DType::U8) &&
                l.relative.shape == Shape{n, k / l.groupSize},
            text("rotated: relative scales ", name(l.relative.dtype), " ", l.relative.shape.str()));
  }
  return RotatedTable{codes, parts, k};
}

// ops/AttentionOps.scala:243-256
void checkPageTable(const Tensor& pageTable, const KvCache& cache, int64_t positions) {
  require(pageTable.dtype == DType::I32 && pageTable.shape.rank() == 1,
          text("a page table is I32 [pages], not ", name(pageTable.dtype), " ", pageTable.shape.str()));
  require(pageTable.elementCount() * cache.pageSize >= positions,
          text("a page table of ", pageTable.elementCount(), " pages for ", positions, " positions"));
}

// ops/AttentionOps.scala:225-241: the token count.
int64_t checkCacheWrite(const Tensor& k, const Tensor& v, const KvCache& cache, const Tensor& pageTable,
                        int64_t start) {
  checkElementwise("cacheWrite", {&k, &v});
  require(k.shape.rank() == 3 && k.shape[1] == cache.kvHeads() && k.shape[2] == cache.headDimension(),
          text("cacheWrite: ", k.shape.str(), " into a cache of ", cache.kvHeads(), " heads of ",
               cache.headDimension()));
  const int64_t tokens = k.shape[0];
  checkPageTable(pageTable, cache, start + tokens);
  return tokens;
}

// ops/LayoutOps.scala:73-80
void checkSplitHalves(const Tensor& x, const Tensor& first, const Tensor& second) {
  checkElementwise("splitHalves", {&x});
  checkElementwise("splitHalves", {&first, &second});
  require(x.dtype == first.dtype,
          text("splitHalves takes one type, not ", name(x.dtype), " and ", name(first.dtype)));
  require(x.elementCount() == 2 * first.elementCount() && first.shape.rank() >= 1 &&
              x.shape.last() == 2 * first.shape.last(),
          text("splitHalves: ", x.shape.str(), " into ", first.shape.str()));
}

// ops/MemoryOps.scala:68-84 with ops/HipBase.scala:268-274's codes.
int checkConvert(const Tensor& x, const Tensor& out) {
  requireSameShape("convert", {&x, &out});
  const DType from = x.dtype, to = out.dtype;
  if (from == DType::F32 && to == DType::F16) return DRIFT_F32_TO_F16;
  if (from == DType::F32 && to == DType::BF16) return DRIFT_F32_TO_BF16;
  if (from == DType::F16 && to == DType::F32) return DRIFT_F16_TO_F32;
  if (from == DType::BF16 && to == DType::F32) return DRIFT_BF16_TO_F32;
  if ((from == DType::F8E4M3 || from == DType::U8) && to == DType::F32) return DRIFT_F8E4M3_TO_F32;
  refuse(text("convert: no conversion from ", name(from), " to ", name(to)));
}

}  // namespace checks

using namespace checks;

// ---------------------------------------------------------------- HipOps

HipOps::HipOps(void* stream) : stream_(stream) {
  if (drift_abi_version() != DRIFT_ABI_VERSION)
    throw std::runtime_error(text("libdrift_kernels implements ABI ", drift_abi_version(), ", this host expects ",
                                  DRIFT_ABI_VERSION));
}

HipOps::~HipOps() {
  if (quantizedBuffer_) (void)hipFree(quantizedBuffer_);
  if (scratch_) (void)hipFree(scratch_);
}

void HipOps::launched(const char* entry, int code) {
  ++writes_;
  if (code != 0) throw HipException(entry, code, drift_last_error());
}

// ---- the int8 side output's bookkeeping

namespace {
// Device memory of at least `bytes` in *buffer (grown, never shrunk).
void ensure(void*& buffer, size_t& size, size_t bytes) {
  if (size >= bytes) return;
  if (buffer) (void)hipFree(buffer);
  buffer = nullptr;
  size = 0;
  const size_t want = std::max<size_t>(bytes, 65536);
  const hipError_t status = hipMalloc(&buffer, want);
  if (status != hipSuccess) throw HipException("hipMalloc", (int)status, hipGetErrorString(status));
  size = want;
}
}  // namespace

QuantizedOutput HipOps::QuantizedValues::at(int64_t first) const {
  float* scales = reinterpret_cast<float*>(codes + values);
  float* sums = scales + values / 32;
  return QuantizedOutput{codes + first, scales + first / 32, sums + first / 32};
}

const QuantizedOutput* HipOps::quantizedTarget(const Tensor& out, int64_t cols, const QuantizedOutput* given,
                                               QuantizedOutput& owned, std::optional<QuantizedValues>& target) {
  target.reset();
  if (given) return given;
  const int64_t values = out.elementCount();
  if (!(quantizesX_ && out.dtype == DType::F32 && values <= QuantizedMaximumValues && cols % 32 == 0)) return nullptr;
  ensure(quantizedBuffer_, quantizedBytes_, (size_t)(values + 8 * (values / 32)));
  target = QuantizedValues{reinterpret_cast<uintptr_t>(out.data), values, static_cast<int8_t*>(quantizedBuffer_), 0};
  owned = target->at(0);
  return &owned;
}

void HipOps::wroteQuantized(const std::optional<QuantizedValues>& target) {
  if (!target) return;
  quantized_ = *target;
  quantized_->written = writes_;
}

std::optional<QuantizedOutput> HipOps::quantizedInput(const Tensor& x, int64_t m, int64_t k) const {
  if (!quantized_ || quantized_->written != writes_ || x.dtype != DType::F32) return std::nullopt;
  const auto address = reinterpret_cast<uintptr_t>(x.data);
  if (address < quantized_->address) return std::nullopt;
  const uintptr_t bytes = address - quantized_->address;
  const int64_t first = (int64_t)(bytes / 4);
  if (bytes % (4 * 32) != 0 || k % 32 != 0 || first + m * k > quantized_->values) return std::nullopt;
  return quantized_->at(first);
}

QuantizedOutput HipOps::quantize(const Tensor& x, int64_t m, int64_t k) {
  quantizesX_ = true;
  require((x.dtype == DType::F32 || x.dtype == DType::BF16) && (m * k) % 32 == 0 && x.elementCount() >= m * k,
          text("quantize: ", m, " rows of ", k, " from ", x.shape.str()));
  const int64_t values = m * k, blocks = values / 32;
  ensure(scratch_, scratchBytes_, (size_t)(values + 8 * blocks));
  const QuantizedOutput into = QuantizedValues{0, values, static_cast<int8_t*>(scratch_), 0}.at(0);
  quantizeTo(x, blocks, into);
  return into;
}

QuantizedOutput HipOps::productInput(const Tensor& x, int64_t m, int64_t k) {
  if (const std::optional<QuantizedOutput> found = quantizedInput(x, m, k)) return *found;
  return quantize(x, m, k);
}

// ---- norms

void HipOps::normRows(const Tensor& x, const Tensor* y, const Tensor& weight, float epsilon, float weightOffset,
                      const Tensor& out, int64_t rows, const QuantizedOutput* q) {
  const int32_t cols = (int32_t)x.shape.last();
  int8_t* xq = q ? static_cast<int8_t*>(q->codes) : nullptr;
  float* xd = q ? q->scales : nullptr;
  float* xs = q ? q->sums : nullptr;
  if (isBf16(x))
    launched("drift_rms_norm_bf16", drift_rms_norm_bf16(at<uint16_t>(x), at<const uint16_t>(y), at<float>(weight),
                                                         at<uint16_t>(out), rows, cols, epsilon, weightOffset, 1, xq,
                                                         xd, xs, stream_));
  else
    launched("drift_rms_norm_f32", drift_rms_norm_f32(at<float>(x), at<const float>(y), at<float>(weight),
                                                       at<float>(out), rows, cols, epsilon, weightOffset, 1, xq, xd,
                                                       xs, stream_));
}

void HipOps::rmsNorm(const Tensor& x, const Tensor& weight, float epsilon, float weightOffset, const Tensor& out,
                     const QuantizedOutput* quantized) {
  const int64_t rows = checkRowWise("rmsNorm", x, out, {&weight});
  QuantizedOutput owned;
  std::optional<QuantizedValues> target;
  const QuantizedOutput* q = quantizedTarget(out, out.shape.last(), quantized, owned, target);
  normRows(x, nullptr, weight, epsilon, weightOffset, out, rows, q);
  wroteQuantized(target);
}

void HipOps::addRmsNorm(const Tensor& x, const Tensor& y, const RowNorm& norm, const QuantizedOutput* quantized) {
  checkElementwise("addRmsNorm", {&x, &y});
  const int64_t rows = checkRowWise("addRmsNorm", x, norm.out, {&norm.weight});
  QuantizedOutput owned;
  std::optional<QuantizedValues> target;
  const QuantizedOutput* q = quantizedTarget(norm.out, norm.out.shape.last(), quantized, owned, target);
  normRows(x, &y, norm.weight, norm.epsilon, norm.weightOffset, norm.out, rows, q);
  wroteQuantized(target);
}

void HipOps::groupRmsNorm(const Tensor& x, const Tensor& weight, int groups, float epsilon, float weightOffset,
                          const Tensor& out) {
  const int64_t rows = checkRowWise("groupRmsNorm", x, out, {&weight});
  require(groups > 0 && x.shape.last() % groups == 0, text(x.shape.str(), " in ", groups, " groups"));
  const int32_t width = (int32_t)(x.shape.last() / groups);
  if (isBf16(x))
    launched("drift_rms_norm_bf16", drift_rms_norm_bf16(at<uint16_t>(x), nullptr, at<float>(weight), at<uint16_t>(out),
                                                         rows * groups, width, epsilon, weightOffset, groups, nullptr,
                                                         nullptr, nullptr, stream_));
  else
    launched("drift_rms_norm_f32", drift_rms_norm_f32(at<float>(x), nullptr, at<float>(weight), at<float>(out),
                                                       rows * groups, width, epsilon, weightOffset, groups, nullptr,
                                                       nullptr, nullptr, stream_));
}

void HipOps::layerNorm(const Tensor& x, const Tensor* weight, const Tensor* bias, float epsilon, const Tensor& out) {
  int64_t rows;
  if (weight && bias)
    rows = checkRowWise("layerNorm", x, out, {weight, bias});
  else if (weight || bias)
    rows = checkRowWise("layerNorm", x, out, {weight ? weight : bias});
  else
    rows = checkRowWise("layerNorm", x, out);
  requireF32("layerNorm", {&x});
  launched("drift_layer_norm_f32", drift_layer_norm_f32(at<float>(x), at<float>(weight), at<float>(bias),
                                                         at<float>(out), rows, (int32_t)x.shape.last(), epsilon,
                                                         stream_));
}

void HipOps::modulate(const Tensor& x, const Tensor& scale, const Tensor& shift, const Tensor& out) {
  const int64_t rows = checkRowWise("modulate", x, out, {&scale, &shift});
  requireF32("modulate", {&x});
  launched("drift_modulate_f32", drift_modulate_f32(at<float>(x), at<float>(scale), at<float>(shift), at<float>(out),
                                                     rows, (int32_t)x.shape.last(), stream_));
}

void HipOps::layerNormModulate(const Tensor& x, const Tensor& scale, const Tensor& shift, float epsilon,
                               const Tensor& out, int64_t rowsPerSample) {
  checkElementwise("layerNormModulate", {&x, &out});
  requireF32("layerNormModulate", {&scale, &shift});
  require(x.shape.rank() == 2, text("layerNormModulate takes [rows, C], not ", x.shape.str()));
  const int64_t rows = x.shape[0], cols = x.shape[1];
  const bool fits = scale.shape.rank() >= 1 && scale.shape.last() == cols && scale.shape.rank() <= 2 &&
                    shift.shape == scale.shape;
  require(fits, text("layerNormModulate: scale ", scale.shape.str(), ", shift ", shift.shape.str(), " for rows of ",
                     cols));
  const int64_t samples = scale.elementCount() / cols;
  const int64_t per = rowsPerSample > 0 ? rowsPerSample : (rows + samples - 1) / samples;
  require(per > 0 && samples * per >= rows,
          text("layerNormModulate: ", samples, " samples of ", per, " rows for ", rows, " rows"));
  if (isBf16(x))
    launched("drift_layer_norm_modulate_bf16",
             drift_layer_norm_modulate_bf16(at<uint16_t>(x), at<float>(scale), at<float>(shift), at<uint16_t>(out),
                                            rows, (int32_t)cols, per, epsilon, stream_));
  else
    launched("drift_layer_norm_modulate_f32",
             drift_layer_norm_modulate_f32(at<float>(x), at<float>(scale), at<float>(shift), at<float>(out), rows,
                                           (int32_t)cols, per, epsilon, stream_));
}

void HipOps::quantizeTo(const Tensor& x, int64_t blocks, const QuantizedOutput& into) {
  require((x.dtype == DType::F32 || x.dtype == DType::BF16) && blocks * 32 <= x.elementCount(),
          text("quantize: ", blocks, " blocks of 32 from ", x.shape.str()));
  int8_t* xq = static_cast<int8_t*>(into.codes);
  if (isBf16(x))
    launched("drift_quantize_x_bf16",
             drift_quantize_x_bf16(at<uint16_t>(x), xq, into.scales, into.sums, blocks, stream_));
  else
    launched("drift_quantize_x_f32", drift_quantize_x_f32(at<float>(x), xq, into.scales, into.sums, blocks, stream_));
}

// ---- gated residuals

void HipOps::gatedAdd(const Tensor& x, const Tensor& y, const Tensor& gate, int64_t rowsPerSample) {
  int64_t rows, per;
  const int64_t cols = x.shape.last();
  if (gate.shape.rank() <= 1) {
    rows = checkRowWise("gatedAdd", x, y, {&gate});
    per = std::max<int64_t>(rows, 1);
  } else {
    checkElementwise("gatedAdd", {&x, &y});
    requireF32("gatedAdd", {&gate});
    rows = cols ? x.elementCount() / cols : 0;
    require(rowsPerSample > 0, "gatedAdd: per-sample gates need rowsPerSample");
    const int64_t samples = (rows + rowsPerSample - 1) / rowsPerSample;
    require(gate.shape == Shape{samples, cols},
            text("gatedAdd: ", gate.shape.str(), " for ", samples, " samples of rows of ", cols));
    per = rowsPerSample;
  }
  if (isBf16(x))
    launched("drift_gated_add_bf16", drift_gated_add_bf16(at<uint16_t>(x), at<uint16_t>(y), at<float>(gate), rows,
                                                           (int32_t)cols, per, stream_));
  else
    launched("drift_gated_add_f32",
             drift_gated_add_f32(at<float>(x), at<float>(y), at<float>(gate), rows, (int32_t)cols, per, stream_));
}

void HipOps::modulateChunks(const Tensor& x, const Tensor& table, int shift, int scale, const Tensor& out) {
  const Chunks c = checkChunks("modulateChunks", x, table, out, {shift, scale});
  if (isBf16(x))
    launched("drift_modulate_chunks_bf16",
             drift_modulate_chunks_bf16(at<uint16_t>(x), at<float>(table), at<uint16_t>(out), c.rows,
                                        (int32_t)c.channels, (int32_t)c.chunks, shift, scale, stream_));
  else
    launched("drift_modulate_chunks_f32",
             drift_modulate_chunks_f32(at<float>(x), at<float>(table), at<float>(out), c.rows, (int32_t)c.channels,
                                       (int32_t)c.chunks, shift, scale, stream_));
}

void HipOps::gatedAddChunk(const Tensor& x, const Tensor& y, const Tensor& table, int gate) {
  const Chunks c = checkChunks("gatedAddChunk", x, table, y, {gate});
  if (isBf16(x))
    launched("drift_gated_add_chunk_bf16",
             drift_gated_add_chunk_bf16(at<uint16_t>(x), at<uint16_t>(y), at<float>(table), c.rows,
                                        (int32_t)c.channels, (int32_t)c.chunks, gate, stream_));
  else
    launched("drift_gated_add_chunk_f32",
             drift_gated_add_chunk_f32(at<float>(x), at<float>(y), at<float>(table), c.rows, (int32_t)c.channels,
                                       (int32_t)c.chunks, gate, stream_));
}

void HipOps::rowGatedAdd(const Tensor& x, const Tensor& y, const Tensor& gate) {
  // ops/ElementwiseOps.scala:79-92
  checkElementwise("rowGatedAdd", {&x, &y});
  requireF32("rowGatedAdd", {&gate});
  require(x.shape.rank() == 2, text("rowGatedAdd takes [rows, cols], not ", x.shape.str()));
  const int64_t rows = x.shape[0], cols = x.shape[1];
  require(gate.elementCount() == rows, text("rowGatedAdd: gate ", gate.shape.str(), " for ", x.shape.str()));
  if (isBf16(x))
    launched("drift_row_gated_add_bf16",
             drift_row_gated_add_bf16(at<uint16_t>(x), at<uint16_t>(y), at<float>(gate), rows, (int32_t)cols, stream_));
  else
    launched("drift_row_gated_add_f32",
             drift_row_gated_add_f32(at<float>(x), at<float>(y), at<float>(gate), rows, (int32_t)cols, stream_));
}

// ---- activations

void HipOps::activation(Activation kind, const Tensor& x, const Tensor& out) { scaledActivation(kind, 1.0f, x, out); }

void HipOps::scaledActivation(Activation kind, float inputScale, const Tensor& x, const Tensor& out) {
  checkElementwise("activation", {&x, &out});
  if (isBf16(x))
    launched("drift_activation_bf16", drift_activation_bf16(at<uint16_t>(x), at<uint16_t>(out), x.elementCount(),
                                                             (int32_t)kind, inputScale, stream_));
  else
    launched("drift_activation_f32", drift_activation_f32(at<float>(x), at<float>(out), x.elementCount(),
                                                           (int32_t)kind, inputScale, stream_));
}

void HipOps::gated(Activation kind, const Tensor& gate, const Tensor& up, const Tensor& out,
                   const QuantizedOutput* quantized) {
  checkElementwise("gated", {&gate, &up, &out});
  QuantizedOutput owned;
  std::optional<QuantizedValues> target;
  const QuantizedOutput* q = quantizedTarget(out, out.shape.last(), quantized, owned, target);
  int8_t* xq = q ? static_cast<int8_t*>(q->codes) : nullptr;
  float* xd = q ? q->scales : nullptr;
  float* xs = q ? q->sums : nullptr;
  if (isBf16(gate))
    launched("drift_gated_bf16", drift_gated_bf16(at<uint16_t>(gate), at<uint16_t>(up), at<uint16_t>(out),
                                                   gate.elementCount(), (int32_t)kind, xq, xd, xs, stream_));
  else
    launched("drift_gated_f32", drift_gated_f32(at<float>(gate), at<float>(up), at<float>(out), gate.elementCount(),
                                                 (int32_t)kind, xq, xd, xs, stream_));
  wroteQuantized(target);
}

// ---- rotary

namespace {
// rope_f32's four section sizes (ops/HipAttention.scala:73-79)
std::vector<int> sectionSizes(const Rope& rope) {
  std::vector<int> s = rope.sections.sizes;
  s.resize(4, 0);
  return s;
}
}  // namespace

void HipOps::rope(const Tensor& x, const Tensor& positions, const Rope& r, const Tensor& out) {
  const Heads h = checkRope(x, positions, r, out);
  const std::vector<int> s = sectionSizes(r);
  if (isBf16(x))
    launched("drift_rope_bf16", drift_rope_bf16(at<uint16_t>(x), at<int32_t>(positions), at<uint16_t>(out),
                                                 (int32_t)h.tokens, (int32_t)h.heads, (int32_t)h.dimension,
                                                 r.rotaryDimensions, r.theta, (int32_t)r.layout, r.sections.code, s[0],
                                                 s[1], s[2], s[3], stream_));
  else
    launched("drift_rope_f32", drift_rope_f32(at<float>(x), at<int32_t>(positions), at<float>(out), (int32_t)h.tokens,
                                               (int32_t)h.heads, (int32_t)h.dimension, r.rotaryDimensions, r.theta,
                                               (int32_t)r.layout, r.sections.code, s[0], s[1], s[2], s[3], stream_));
}

void HipOps::ropeTable(const Tensor& x, const Tensor& cosines, const Tensor& sines, const Tensor& out, bool halves) {
  const TableRope t = checkRopeTable(x, cosines, sines, out);
  if (isBf16(x))
    launched("drift_rope_table_bf16",
             drift_rope_table_bf16(at<uint16_t>(x), at<float>(cosines), at<float>(sines), at<uint16_t>(out),
                                   (int32_t)t.tokens, (int32_t)t.heads, (int32_t)t.dimension, (int32_t)t.pairs,
                                   t.perHead ? 1 : 0, halves ? 1 : 0, stream_));
  else
    launched("drift_rope_table_f32",
             drift_rope_table_f32(at<float>(x), at<float>(cosines), at<float>(sines), at<float>(out),
                                  (int32_t)t.tokens, (int32_t)t.heads, (int32_t)t.dimension, (int32_t)t.pairs,
                                  t.perHead ? 1 : 0, halves ? 1 : 0, stream_));
}

void HipOps::rope3d(const Tensor& x, int frames, int rows, int columns, const Tensor& out, int64_t tokenOffset,
                    double theta) {
  checkElementwise("rope3d", {&x, &out});
  require(x.shape.rank() == 3, text("rope3d takes [tokens, heads, D], not ", x.shape.str()));
  if (isBf16(x))
    launched("drift_rope_3d_bf16",
             drift_rope_3d_bf16(at<uint16_t>(x), at<uint16_t>(out), x.shape[0], (int32_t)x.shape[1],
                                (int32_t)x.shape[2], frames, rows, columns, tokenOffset, theta, stream_));
  else
    launched("drift_rope_3d_f32", drift_rope_3d_f32(at<float>(x), at<float>(out), x.shape[0], (int32_t)x.shape[1],
                                                     (int32_t)x.shape[2], frames, rows, columns, tokenOffset, theta,
                                                     stream_));
}

void HipOps::queryKeyNormRope(const Tensor& q, const Tensor& k, const QueryKeyNorms& norms, const Tensor& positions,
                              const Tensor& rotatedQueries, const Tensor& rotatedKeys) {
  checkElementwise("queryKeyNormRope", {&q, &rotatedQueries});
  checkElementwise("queryKeyNormRope", {&k, &rotatedKeys});
  require(q.dtype == k.dtype, "queryKeyNormRope takes one type for queries and keys");
  require(q.shape.rank() == 3 && k.shape.rank() == 3 && q.shape[0] == k.shape[0] && q.shape[2] == k.shape[2],
          text("queryKeyNormRope: queries ", q.shape.str(), ", keys ", k.shape.str()));
  const Heads h = checkRope(q, positions, norms.rope, rotatedQueries);
  for (const Tensor* w : {&norms.queryNorm, &norms.keyNorm}) {
    requireF32("queryKeyNormRope", {w});
    require(w->shape == Shape{h.dimension},
            text("queryKeyNormRope: ", w == &norms.queryNorm ? "queryNorm " : "keyNorm ", w->shape.str(),
                 " for heads of ", h.dimension));
  }
  const Rope& r = norms.rope;
  const std::vector<int> s = sectionSizes(r);
  const int32_t kv = (int32_t)k.shape[1];
  if (isBf16(q))
    launched("drift_qk_norm_rope_bf16",
             drift_qk_norm_rope_bf16(at<uint16_t>(q), at<uint16_t>(k), at<uint16_t>(rotatedQueries),
                                     at<uint16_t>(rotatedKeys), at<float>(norms.queryNorm), at<float>(norms.keyNorm),
                                     at<int32_t>(positions), (int32_t)h.tokens, (int32_t)h.heads, kv,
                                     (int32_t)h.dimension, norms.epsilon, norms.weightOffset, r.rotaryDimensions,
                                     r.theta, (int32_t)r.layout, r.sections.code, s[0], s[1], s[2], s[3], stream_));
  else
    launched("drift_qk_norm_rope_f32",
             drift_qk_norm_rope_f32(at<float>(q), at<float>(k), at<float>(rotatedQueries), at<float>(rotatedKeys),
                                    at<float>(norms.queryNorm), at<float>(norms.keyNorm), at<int32_t>(positions),
                                    (int32_t)h.tokens, (int32_t)h.heads, kv, (int32_t)h.dimension, norms.epsilon,
                                    norms.weightOffset, r.rotaryDimensions, r.theta, (int32_t)r.layout,
                                    r.sections.code, s[0], s[1], s[2], s[3], stream_));
}

// ---- attention inputs

void HipOps::cacheWrite(const Tensor& k, const Tensor& v, const KvCache& cache, const Tensor& pageTable,
                        int64_t start, int32_t* badPage) {
  const int64_t tokens = checkCacheWrite(k, v, cache, pageTable, start);
  uint16_t* keys = at<uint16_t>(cache.keys);
  uint16_t* values = at<uint16_t>(cache.values);
  const auto table = (int32_t)pageTable.elementCount();
  if (isBf16(k))
    launched("drift_cache_write_bf16",
             drift_cache_write_bf16(at<uint16_t>(k), at<uint16_t>(v), keys, values, at<int32_t>(pageTable), table,
                                    (int32_t)cache.pages(), (int32_t)tokens, (int32_t)cache.kvHeads(),
                                    (int32_t)cache.headDimension(), cache.pageSize, (int32_t)start, badPage, stream_));
  else
    launched("drift_cache_write_f32",
             drift_cache_write_f32(at<float>(k), at<float>(v), keys, values, at<int32_t>(pageTable), table,
                                   (int32_t)cache.pages(), (int32_t)tokens, (int32_t)cache.kvHeads(),
                                   (int32_t)cache.headDimension(), cache.pageSize, (int32_t)start, badPage, stream_));
}

void HipOps::splitHalves(const Tensor& x, const Tensor& first, const Tensor& second) {
  checkSplitHalves(x, first, second);
  const int64_t d = first.shape.last();
  if (isBf16(x))
    launched("drift_split_halves_bf16", drift_split_halves_bf16(at<uint16_t>(x), at<uint16_t>(first),
                                                                 at<uint16_t>(second), first.elementCount() / d,
                                                                 (int32_t)d, stream_));
  else
    launched("drift_split_halves_f32", drift_split_halves_f32(at<float>(x), at<float>(first), at<float>(second),
                                                               first.elementCount() / d, (int32_t)d, stream_));
}

void HipOps::attentionInputs(const Tensor& queryAndGate, const Tensor& keys, const Tensor& values,
                             const QueryKeyNorms& norms, const Tensor& positions, const KvCache& cache,
                             const Tensor& pageTable, int64_t start, const Tensor& queries, const Tensor& gate,
                             const Tensor& rotatedKeys, const Tensor& rotatedQueries, int32_t* badPage) {
  // the reference's fused launch checks the unfused steps' tensors
  // (ops/HipAttention.scala:144-215); `queries` and `rotatedKeys` are not
  // written
  const int64_t d = queries.shape.rank() == 3 ? queries.shape[2] : 0;
  require(d <= AttentionInputDimension,
          text("attentionInputs: heads of ", d, " values (at most ", AttentionInputDimension, " fused)"));
  checkSplitHalves(queryAndGate, queries, gate);
  checkRope(queries, positions, norms.rope, rotatedQueries);
  checkRope(keys, positions, norms.rope, rotatedKeys);
  checkCacheWrite(rotatedKeys, values, cache, pageTable, start);
  fusedAttentionInputs(queryAndGate, keys, values, norms, positions, cache, pageTable, start, &gate, rotatedQueries,
                       badPage);
}

void HipOps::queryKeyNormRopeCache(const Tensor& q, const Tensor& k, const Tensor& v, const QueryKeyNorms& norms,
                                   const Tensor& positions, const KvCache& cache, const Tensor& pageTable,
                                   int64_t start, const Tensor& rotatedQueries, int32_t* badPage) {
  require(q.shape.rank() == 3 && q.shape[2] <= AttentionInputDimension,
          text("queryKeyNormRopeCache: queries ", q.shape.str()));
  checkRope(q, positions, norms.rope, rotatedQueries);
  checkRope(k, positions, norms.rope, k);
  checkCacheWrite(k, v, cache, pageTable, start);
  fusedAttentionInputs(q, k, v, norms, positions, cache, pageTable, start, nullptr, rotatedQueries, badPage);
}

void HipOps::fusedAttentionInputs(const Tensor& queryAndGate, const Tensor& keys, const Tensor& values,
                                  const QueryKeyNorms& norms, const Tensor& positions, const KvCache& cache,
                                  const Tensor& pageTable, int64_t start, const Tensor* gate,
                                  const Tensor& rotatedQueries, int32_t* badPage) {
  const int64_t tokens = rotatedQueries.shape[0], heads = rotatedQueries.shape[1], d = rotatedQueries.shape[2];
  require(keys.shape == Shape{tokens, cache.kvHeads(), d},
          text("attentionInputs: keys ", keys.shape.str(), " for ", tokens, " tokens of heads of ", d));
  require(queryAndGate.dtype == keys.dtype && values.dtype == keys.dtype && rotatedQueries.dtype == keys.dtype &&
              (!gate || gate->dtype == keys.dtype),
          "attentionInputs takes one type for queries, gate, keys and values");
  for (const Tensor* w : {&norms.queryNorm, &norms.keyNorm}) {
    requireF32("attentionInputs", {w});
    require(w->shape == Shape{d}, text("attentionInputs: ", w == &norms.queryNorm ? "queryNorm " : "keyNorm ",
                                       w->shape.str(), " for heads of ", d));
  }
  const Rope& r = norms.rope;
  const std::vector<int> s = sectionSizes(r);
  const auto table = (int32_t)pageTable.elementCount();
  if (isBf16(keys))
    launched("drift_attention_inputs_bf16",
             drift_attention_inputs_bf16(
                 at<uint16_t>(queryAndGate), at<uint16_t>(keys), at<uint16_t>(values), at<float>(norms.queryNorm),
                 at<float>(norms.keyNorm), norms.epsilon, norms.weightOffset, at<int32_t>(positions), (int32_t)tokens,
                 (int32_t)heads, (int32_t)cache.kvHeads(), (int32_t)d, r.rotaryDimensions, r.theta,
                 (int32_t)r.layout, r.sections.code, s[0], s[1], s[2], s[3], at<uint16_t>(rotatedQueries),
                 at<uint16_t>(gate), at<uint16_t>(cache.keys), at<uint16_t>(cache.values), at<int32_t>(pageTable),
                 table, (int32_t)cache.pages(), cache.pageSize, (int32_t)start, badPage, stream_));
  else
    launched("drift_attention_inputs_f32",
             drift_attention_inputs_f32(
                 at<float>(queryAndGate), at<float>(keys), at<float>(values), at<float>(norms.queryNorm),
                 at<float>(norms.keyNorm), norms.epsilon, norms.weightOffset, at<int32_t>(positions), (int32_t)tokens,
                 (int32_t)heads, (int32_t)cache.kvHeads(), (int32_t)d, r.rotaryDimensions, r.theta,
                 (int32_t)r.layout, r.sections.code, s[0], s[1], s[2], s[3], at<float>(rotatedQueries),
                 at<float>(gate), at<uint16_t>(cache.keys), at<uint16_t>(cache.values), at<int32_t>(pageTable), table,
                 (int32_t)cache.pages(), cache.pageSize, (int32_t)start, badPage, stream_));
}

// ---- tables

namespace {
const StorageType& checkStored(const char* operation, const StoredTable& table) {
  require(table.type != nullptr, text(operation, ": a table of stored bytes"));
  const StorageType& t = *table.type;
  const int64_t vocab = table.shape()[0];
  require(table.cols % t.values == 0, text(table.cols, " elements are not whole ", t.name, " blocks of ", t.values));
  require(table.data.dtype == DType::U8 && table.data.shape == Shape{vocab, t.rowBytes(table.cols)},
          text(operation, ": ", t.name, " bytes ", table.data.shape.str(), " for rows of ", table.cols));
  require(table.cols % 8 == 0 || t.values == 1,
          text(operation, ": rows of ", table.cols, " values (quant kernels take multiples of 8)"));
  return t;
}
}  // namespace

void HipOps::embedding(const StoredTable& table, const Tensor& ids, const Tensor& out, int32_t* badId) {
  checkEmbedding(table.shape(), ids, out);
  const StorageType& t = checkStored("embedding", table);
  const int64_t vocab = table.shape()[0], count = ids.shape[0];
  const auto cols = (int32_t)table.cols;
  const auto* bytes = static_cast<const uint8_t*>(table.data.data);
  if (t.ggmlId == DRIFT_Q8_0) {
    if (isBf16(out))
      launched("drift_embedding_q8_0_bf16", drift_embedding_q8_0_bf16(bytes, at<int32_t>(ids), at<uint16_t>(out),
                                                                       count, vocab, cols, badId, stream_));
    else
      launched("drift_embedding_q8_0_f32", drift_embedding_q8_0_f32(bytes, at<int32_t>(ids), at<float>(out), count,
                                                                     vocab, cols, badId, stream_));
  } else if (isBf16(out)) {
    launched("drift_embedding_bf16", drift_embedding_bf16(bytes, t.ggmlId, at<int32_t>(ids), at<uint16_t>(out), count,
                                                           vocab, cols, badId, stream_));
  } else {
    launched("drift_embedding_f32", drift_embedding_f32(bytes, t.ggmlId, at<int32_t>(ids), at<float>(out), count,
                                                         vocab, cols, badId, stream_));
  }
}

RotatedTable HipOps::rotated(const Tensor& codes, const ConvRotParts& parts) { return checkRotated(codes, parts); }

void HipOps::decodeRotated(const RotatedTable& table, const Tensor& out, const Tensor* ids, int32_t* badId) {
  const RotatedTable t = checkRotated(table.codes, table.parts);
  const ConvRotParts& p = t.parts;
  const float* codebook = p.levels ? at<float>(p.levels->codebook) : nullptr;
  const auto* relative = p.levels ? at<const uint8_t>(p.levels->relative) : nullptr;
  const int32_t group = p.levels ? p.levels->groupSize : 0;
  const int64_t rows = t.shape()[0];
  const auto cols = (int32_t)t.cols;
  if (!ids) {
    launched("drift_rotated_dequantize_bf16",
             drift_rotated_dequantize_bf16(t.codes.data, at<float>(p.scales), p.scales.elementCount(), codebook,
                                           relative, group, at<uint16_t>(out), rows, cols, stream_));
  } else if (isBf16(out)) {
    launched("drift_rotated_embedding_bf16",
             drift_rotated_embedding_bf16(t.codes.data, at<float>(p.scales), p.scales.elementCount(), codebook,
                                          relative, group, at<int32_t>(*ids), at<uint16_t>(out), ids->shape[0], rows,
                                          cols, badId, stream_));
  } else {
    launched("drift_rotated_embedding_f32",
             drift_rotated_embedding_f32(t.codes.data, at<float>(p.scales), p.scales.elementCount(), codebook,
                                         relative, group, at<int32_t>(*ids), at<float>(out), ids->shape[0], rows, cols,
                                         badId, stream_));
  }
}

void HipOps::embedding(const RotatedTable& table, const Tensor& ids, const Tensor& out, int32_t* badId) {
  checkEmbedding(table.shape(), ids, out);
  decodeRotated(table, out, &ids, badId);
}

void HipOps::dequantize(const StoredTable& table, const Tensor& out) {
  const StorageType& t = checkStored("dequantize", table);
  require(out.dtype == DType::BF16 || out.dtype == DType::F16,
          text("dequantize writes BF16 or F16, not ", name(out.dtype)));
  require(out.shape == table.shape(),
          text("dequantize: out ", out.shape.str(), " for a table ", table.shape().str()));
  const auto* bytes = table.data.data;
  if (out.dtype == DType::BF16)
    launched("drift_dequantize_bf16", drift_dequantize_bf16(bytes, t.ggmlId, at<uint16_t>(out), table.shape()[0],
                                                             (int32_t)table.cols, stream_));
  else
    launched("drift_dequantize_f16", drift_dequantize_f16(bytes, t.ggmlId, at<uint16_t>(out), table.shape()[0],
                                                           (int32_t)table.cols, stream_));
}

void HipOps::convert(const Tensor& x, const Tensor& out) {
  const int kind = checkConvert(x, out);
  launched("drift_convert", drift_convert(x.data, out.data, x.elementCount(), kind, stream_));
}

void HipOps::convert(const RotatedTable& x, const Tensor& out) {
  // ops/MemoryOps.scala:74-75, ops/HipMemory.scala:127-130: to BF16
  require(out.dtype == DType::BF16, text("convert: no conversion from ", x.dtype(), " to ", name(out.dtype)));
  require(out.shape == x.shape(), text("convert needs equal shapes, got ", x.shape().str(), ", ", out.shape.str()));
  decodeRotated(x, out, nullptr, nullptr);
}

}  // namespace drift
