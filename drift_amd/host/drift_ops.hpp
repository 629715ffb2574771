// The drift runner's operation interface for the fused layer kernels, in C++
// over libdrift_kernels: the host side a compiled caller links.
//
// It mirrors the runner's Scala `Ops` trait for this path
// (runner/src/drift/runner/ops/Ops.scala:15-34): the same method names,
// argument meaning and shape/dtype rules, checked before any launch and
// refused with std::invalid_argument whose message is the reference's
// ("requirement failed: " + the `require` text of ops/Ops.scala:36-93 and the
// groups' checks; Scala's IllegalArgumentException). A refusal by the
// library itself, or a HIP failure, is a HipException carrying the entry
// point and the library's reason (native/HipRuntime.scala:123-130).
//
// Tensors are dense, row-major device memory the caller owns (the reference's
// Storage.Device); `out` is written, never read, and may be an input of the
// elementwise and row-wise operations. Beyond the reference's F32 kernels the
// operations take BF16 tensors with F32 norm, modulation and rope vectors.
// Everything launches asynchronously on the stream given to the constructor
// and nothing synchronizes. Nothing is allocated either, except the buffers
// of the int8 side output's bookkeeping (below), which this object owns, as
// the reference's backend owns its own (ops/HipBase.scala:148-183).
#pragma once

#include <cstdint>
#include <initializer_list>
#include <optional>
#include <stdexcept>
#include <string>
#include <vector>

namespace drift {

// tensor/DType.scala's element types on this path (F8E4M3: fp8 E4M3 "fn").
enum class DType { F32, F16, BF16, I32, I8, U8, F8E4M3 };

const char* name(DType dtype);
int64_t elementBytes(DType dtype);

// tensor/Tensor.scala:5-16: printed as the reference prints it, [2×3].
struct Shape {
  std::vector<int64_t> dimensions;

  Shape() = default;
  Shape(std::initializer_list<int64_t> dims) : dimensions(dims) {}
  explicit Shape(std::vector<int64_t> dims) : dimensions(std::move(dims)) {}

  int rank() const { return (int)dimensions.size(); }
  int64_t operator[](int i) const { return dimensions[(size_t)i]; }
  int64_t last() const { return dimensions.empty() ? 1 : dimensions.back(); }
  int64_t elementCount() const;
  bool operator==(const Shape& other) const { return dimensions == other.dimensions; }
  bool operator!=(const Shape& other) const { return !(*this == other); }
  std::string str() const;
};

// A tensor in device memory: type, shape and the address of its first
// element. Not owned.
struct Tensor {
  DType dtype = DType::F32;
  Shape shape;
  void* data = nullptr;

  int64_t elementCount() const { return shape.elementCount(); }
  int64_t byteSize() const { return shape.elementCount() * elementBytes(dtype); }
};

class HipException : public std::runtime_error {
 public:
  HipException(const std::string& entry, int code, const std::string& reason);
  std::string entry;
  int code;
};

// ops/Activation.scala:6-20; the value is the kernels' `kind`.
enum class Activation : int { Silu = 0, GeluTanh = 1, GeluErf = 2, Sigmoid = 3, Situ = 4 };

// ops/Rope.scala:7-37.
enum class RopeLayout : int { Neox = 0, Interleaved = 1 };

struct RopeSections {
  int code = 0;
  std::vector<int> sizes;

  static RopeSections Single() { return {}; }
  static RopeSections Contiguous(int temporal, int height, int width) { return {1, {temporal, height, width}}; }
  static RopeSections Interleaved(int temporal, int height, int width) { return {2, {temporal, height, width}}; }
  static RopeSections Axes(std::vector<int> pairs) { return {3, std::move(pairs)}; }
  int positionsPerToken() const { return code == 0 ? 1 : (code == 3 ? (int)sizes.size() : 3); }
};

struct Rope {
  float theta = 10000.0f;
  int rotaryDimensions = 0;
  RopeLayout layout = RopeLayout::Neox;
  RopeSections sections;
};

// ops/RowNorm.scala:17-23: an RMS norm taken of a result as it is written.
struct RowNorm {
  Tensor weight;
  float epsilon = 1e-6f;
  float weightOffset = 0.0f;
  Tensor out;
};

// ops/RowNorm.scala:5-15: query and key RMS norms, then `rope`.
struct QueryKeyNorms {
  Tensor queryNorm, keyNorm;
  float epsilon = 1e-6f;
  float weightOffset = 0.0f;
  Rope rope;
};

// ops/KvCache.scala:5-22: keys F16 [pages, pageSize, kvHeads, D], values F16
// [pages, kvHeads, D, pageSize] (transposed within a page). `of` checks the
// two tensors agree.
struct KvCache {
  Tensor keys, values;
  int pageSize = 16;

  static KvCache of(const Tensor& keys, const Tensor& values, int pageSize);
  int64_t pages() const { return keys.shape[0]; }
  int64_t kvHeads() const { return keys.shape[2]; }
  int64_t headDimension() const { return keys.shape[3]; }
};

// A table's storage type (tensor/DType.scala:14-66): values per block of
// bytes, its GGUF type id (the kernels' `format`) and the alignment its
// blocks' fields need.
struct StorageType {
  const char* name;
  int ggmlId, values, bytes, align;

  int64_t rowBytes(int64_t cols) const;
  static const StorageType& named(const std::string& name);
  static const std::vector<StorageType>& all();
};

// A table ([vocabulary, cols] values) as its stored bytes: U8 [vocabulary,
// row bytes] (a GGUF tensor's data as it lies in the file).
struct StoredTable {
  Tensor data;
  const StorageType* type = nullptr;
  int64_t cols = 0;

  Shape shape() const { return Shape{data.shape.rank() > 0 ? data.shape[0] : 0, cols}; }
};

// ops/ConvRotParts.scala: what a rotated linear's codes are decoded with.
struct ConvRotLevels {
  Tensor codebook;  // F32 [16]
  Tensor relative;  // fp8 E4M3 (U8 or F8E4M3) [rows, cols / groupSize]
  int groupSize = 0;
};

struct ConvRotParts {
  Tensor scales;  // F32 [rows], or [1] without levels
  std::optional<ConvRotLevels> levels;
};

// A rotated linear [rows, cols] left where the file holds it
// (ops/LinearOps.scala:21-33): CONVROT_I8 codes I8 [rows, cols], or
// CONVROT_W4A8 4-bit codes [rows, cols / 2].
struct RotatedTable {
  Tensor codes;
  ConvRotParts parts;
  int64_t cols = 0;

  Shape shape() const { return Shape{codes.shape[0], cols}; }
  const char* dtype() const { return parts.levels ? "CONVROT_W4A8" : "CONVROT_I8"; }
};

// The int8 side output of a norm or `gated` (ops/HipBase.scala:117-214):
// codes (one int8 a value) and, per block of 32 values, the scale and the
// codes' sum, all device memory.
struct QuantizedOutput {
  void* codes = nullptr;
  float* scales = nullptr;
  float* sums = nullptr;
};

// object Ops's checks for this path (ops/Ops.scala:36-93,
// ops/ElementwiseOps.scala, ops/AttentionOps.scala, ops/LinearOps.scala,
// ops/LayoutOps.scala, ops/MemoryOps.scala), shared by every backend.
namespace checks {
void requireF32(const char* operation, std::initializer_list<const Tensor*> tensors);
void requireSameShape(const char* operation, std::initializer_list<const Tensor*> tensors);
void checkElementwise(const char* operation, std::initializer_list<const Tensor*> tensors);
int64_t checkRowWise(const char* operation, const Tensor& x, const Tensor& out,
                     std::initializer_list<const Tensor*> rowVectors = {});
// (rows, channels, chunks)
struct Chunks {
  int64_t rows, channels, chunks;
};
Chunks checkChunks(const char* operation, const Tensor& x, const Tensor& table, const Tensor& out,
                   std::initializer_list<int> indices);
// (tokens, heads, head dimension)
struct Heads {
  int64_t tokens, heads, dimension;
};
Heads checkRope(const Tensor& x, const Tensor& positions, const Rope& rope, const Tensor& out);
struct TableRope {
  int64_t tokens, heads, dimension, pairs;
  bool perHead;
};
TableRope checkRopeTable(const Tensor& x, const Tensor& cosines, const Tensor& sines, const Tensor& out);
void checkEmbedding(const Shape& table, const Tensor& ids, const Tensor& out);
RotatedTable checkRotated(const Tensor& codes, const ConvRotParts& parts);
void checkPageTable(const Tensor& pageTable, const KvCache& cache, int64_t positions);
int64_t checkCacheWrite(const Tensor& k, const Tensor& v, const KvCache& cache, const Tensor& pageTable,
                        int64_t start);
void checkSplitHalves(const Tensor& x, const Tensor& first, const Tensor& second);
int checkConvert(const Tensor& x, const Tensor& out);  // the reference's conversion code
}  // namespace checks

// The GPU backend of this path (the reference's HipOps, ops/HipOps.scala).
class HipOps {
 public:
  // attention.hip's ATTENTION_INPUT_DIMENSION (ops/HipAttention.scala:217-218)
  static constexpr int64_t AttentionInputDimension = 512;

  // `stream`: a hipStream_t, null for the default stream.
  explicit HipOps(void* stream = nullptr);
  ~HipOps();
  HipOps(const HipOps&) = delete;
  HipOps& operator=(const HipOps&) = delete;

  // Launches so far (ops/HipBase.scala:128-147 counts them for the int8 side
  // output's freshness).
  int64_t deviceWrites() const { return writes_; }

  // ---- norms (ops/NormalisationOps.scala:30-80)
  void rmsNorm(const Tensor& x, const Tensor& weight, float epsilon, float weightOffset, const Tensor& out,
               const QuantizedOutput* quantized = nullptr);
  void addRmsNorm(const Tensor& x, const Tensor& y, const RowNorm& norm, const QuantizedOutput* quantized = nullptr);
  // RMS norm of each of a row's `groups` equal parts on its own, `weight`
  // spanning the whole row ([groups × width]); no int8 side output
  // (ops/NormalisationOps.scala:46-58, ops/HipNormalisation.scala:133-158)
  void groupRmsNorm(const Tensor& x, const Tensor& weight, int groups, float epsilon, float weightOffset,
                    const Tensor& out);
  void layerNorm(const Tensor& x, const Tensor* weight, const Tensor* bias, float epsilon, const Tensor& out);
  void modulate(const Tensor& x, const Tensor& scale, const Tensor& shift, const Tensor& out);
  // AdaLN in one launch: layerNorm without affine, then sample s's row of
  // scale and shift ([samples, C]) over rows [s * rowsPerSample, ...).
  void layerNormModulate(const Tensor& x, const Tensor& scale, const Tensor& shift, float epsilon, const Tensor& out,
                         int64_t rowsPerSample = 0);
  // quantize_x: `blocks` blocks of 32 values of x into the caller's buffers
  void quantizeTo(const Tensor& x, int64_t blocks, const QuantizedOutput& into);

  // ---- the int8 side output's bookkeeping (ops/HipBase.scala:117-214,
  // ops/HipLinear.scala:142-143,366-386). Once int8 products run (the first
  // `quantize`), rmsNorm, addRmsNorm and gated quantize an F32 output of at
  // most QuantizedMaximumValues values (rows of a multiple of 32) as they
  // write it, into a buffer this object owns, unless the caller passes its
  // own QuantizedOutput. The buffers stay valid until the next call that
  // writes them.
  static constexpr int64_t QuantizedMaximumValues = 8 * 16384;
  bool quantizesX() const { return quantizesX_; }
  // `m` rows of x (`k` wide) as the last launch wrote them quantized, if it did
  std::optional<QuantizedOutput> quantizedInput(const Tensor& x, int64_t m, int64_t k) const;
  // `m` rows of x quantized now, into this object's scratch
  QuantizedOutput quantize(const Tensor& x, int64_t m, int64_t k);
  // what an int8 product over `m` rows of x reads: quantizedInput, else quantize
  QuantizedOutput productInput(const Tensor& x, int64_t m, int64_t k);

  // ---- gated residuals (ops/ElementwiseOps.scala:28-92)
  void gatedAdd(const Tensor& x, const Tensor& y, const Tensor& gate, int64_t rowsPerSample = 0);
  void modulateChunks(const Tensor& x, const Tensor& table, int shift, int scale, const Tensor& out);
  void gatedAddChunk(const Tensor& x, const Tensor& y, const Tensor& table, int gate);
  void rowGatedAdd(const Tensor& x, const Tensor& y, const Tensor& gate);

  // ---- activations (ops/NormalisationOps.scala:10-24)
  void activation(Activation kind, const Tensor& x, const Tensor& out);
  void scaledActivation(Activation kind, float inputScale, const Tensor& x, const Tensor& out);
  void gated(Activation kind, const Tensor& gate, const Tensor& up, const Tensor& out,
             const QuantizedOutput* quantized = nullptr);

  // ---- rotary (ops/AttentionOps.scala:25-45, models/Wan.scala:324-361)
  void rope(const Tensor& x, const Tensor& positions, const Rope& rope, const Tensor& out);
  void ropeTable(const Tensor& x, const Tensor& cosines, const Tensor& sines, const Tensor& out, bool halves = false);
  void rope3d(const Tensor& x, int frames, int rows, int columns, const Tensor& out, int64_t tokenOffset = 0,
              double theta = 10000.0);
  void queryKeyNormRope(const Tensor& q, const Tensor& k, const QueryKeyNorms& norms, const Tensor& positions,
                        const Tensor& rotatedQueries, const Tensor& rotatedKeys);

  // ---- attention inputs (ops/AttentionOps.scala:52-107, ops/LayoutOps.scala:31)
  void cacheWrite(const Tensor& k, const Tensor& v, const KvCache& cache, const Tensor& pageTable, int64_t start,
                  int32_t* badPage = nullptr);
  void splitHalves(const Tensor& x, const Tensor& first, const Tensor& second);
  void attentionInputs(const Tensor& queryAndGate, const Tensor& keys, const Tensor& values, const QueryKeyNorms& norms,
                       const Tensor& positions, const KvCache& cache, const Tensor& pageTable, int64_t start,
                       const Tensor& queries, const Tensor& gate, const Tensor& rotatedKeys,
                       const Tensor& rotatedQueries, int32_t* badPage = nullptr);
  void queryKeyNormRopeCache(const Tensor& q, const Tensor& k, const Tensor& v, const QueryKeyNorms& norms,
                             const Tensor& positions, const KvCache& cache, const Tensor& pageTable, int64_t start,
                             const Tensor& rotatedQueries, int32_t* badPage = nullptr);

  // ---- tables (ops/LinearOps.scala:16-33, ops/MemoryOps.scala:46)
  // An id outside the table (which the reference refuses) gets a zero row
  // and sets *badId (device int32) when given.
  void embedding(const StoredTable& table, const Tensor& ids, const Tensor& out, int32_t* badId = nullptr);
  void embedding(const RotatedTable& table, const Tensor& ids, const Tensor& out, int32_t* badId = nullptr);
  RotatedTable rotated(const Tensor& codes, const ConvRotParts& parts);
  // the whole table for the GEMM path: BF16 or F16 (a rotated table: BF16)
  void dequantize(const StoredTable& table, const Tensor& out);
  void convert(const Tensor& x, const Tensor& out);
  void convert(const RotatedTable& x, const Tensor& out);

 private:
  void* stream_;
  int64_t writes_ = 0;

  // values at `address` a launch also wrote quantized at `codes` (codes, then
  // scales, then sums), as of launch `written`
  struct QuantizedValues {
    uintptr_t address = 0;
    int64_t values = 0;
    int8_t* codes = nullptr;
    int64_t written = 0;
    QuantizedOutput at(int64_t first) const;
  };
  bool quantizesX_ = false;
  std::optional<QuantizedValues> quantized_;
  void* quantizedBuffer_ = nullptr;
  size_t quantizedBytes_ = 0;
  void* scratch_ = nullptr;
  size_t scratchBytes_ = 0;

  const QuantizedOutput* quantizedTarget(const Tensor& out, int64_t cols, const QuantizedOutput* given,
                                         QuantizedOutput& owned, std::optional<QuantizedValues>& target);
  void wroteQuantized(const std::optional<QuantizedValues>& target);

  void launched(const char* entry, int code);
  void normRows(const Tensor& x, const Tensor* y, const Tensor& weight, float epsilon, float weightOffset,
                const Tensor& out, int64_t rows, const QuantizedOutput* quantized);
  void fusedAttentionInputs(const Tensor& queryAndGate, const Tensor& keys, const Tensor& values,
                            const QueryKeyNorms& norms, const Tensor& positions, const KvCache& cache,
                            const Tensor& pageTable, int64_t start, const Tensor* gate, const Tensor& rotatedQueries,
                            int32_t* badPage);
  void decodeRotated(const RotatedTable& table, const Tensor& out, const Tensor* ids, int32_t* badId);
};

}  // namespace drift
