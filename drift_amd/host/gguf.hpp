// GGUF files (versions 2 and 3, little-endian) for the C++ host, read as the
// runner reads them (runner/src/drift/runner/formats/Gguf.scala): metadata,
// tensor infos, then the data section, each tensor at a multiple of
// `general.alignment`. The file is memory-mapped; a tensor's bytes are a view
// of the mapping until `table` copies them to the device for
// HipOps::embedding or HipOps::dequantize.
//
// GGUF lists dimensions innermost first; shapes here are outermost first, as
// the reference's Shape. The reference's checks are kept, with its messages
// (a FormatError for its FormatException): the magic and version, plausible
// counts, metadata value types, a power-of-two alignment, at most 8
// dimensions, rows of whole blocks, aligned offsets within the data, each
// tensor's byte size against the room the file gives it (Gguf.scala:262-285),
// and ROCmFP4's finite scale bytes (tensor/RocmFp4.scala:64-73).
#pragma once

#include <cstdint>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

#include "drift_ops.hpp"

namespace drift::gguf {

// formats/StoredTensor.scala:57 FormatException
struct FormatError : std::runtime_error {
  using std::runtime_error::runtime_error;
};

// A GGUF tensor type the runner decodes (tensor/DType.scala:168-193).
struct GgmlType {
  const char* name;
  int id, values, bytes;
  int64_t byteSize(int64_t elements) const;
};

// DType.fromGgmlId: the type, or null with the reason it is unsupported.
const GgmlType* typeOf(int id, std::string& reason);

// A metadata value: an integer (`fits` when it fits a signed 64-bit long), a
// real, a boolean, a string, or an array of values.
struct Value {
  enum Kind { Integer, Real, Boolean, Text, Array } kind = Integer;
  int64_t integer = 0;
  bool fits = true;
  double real = 0.0;
  bool flag = false;
  std::string text;
  std::vector<Value> items;
};

// formats/StoredTensor.scala:9-38: type, shape (outermost first) and where its
// bytes start in the file.
struct StoredTensor {
  std::string name;
  const GgmlType* type = nullptr;
  std::vector<int64_t> shape;
  int64_t fileOffset = 0;
  int64_t byteSize() const;
};

// A table copied to the device: the StoredTable HipOps takes, and the device
// memory it owns.
class DeviceTable {
 public:
  DeviceTable(StoredTable table, void* memory) : table_(std::move(table)), memory_(memory) {}
  ~DeviceTable();
  DeviceTable(DeviceTable&& other) noexcept;
  DeviceTable(const DeviceTable&) = delete;
  DeviceTable& operator=(const DeviceTable&) = delete;
  const StoredTable& table() const { return table_; }

 private:
  StoredTable table_;
  void* memory_;
};

class File {
 public:
  // Gguf.open: maps the file and reads it.
  static File open(const std::string& path);
  ~File();
  File(File&& other) noexcept;
  File(const File&) = delete;
  File& operator=(const File&) = delete;

  const std::string& source() const { return source_; }
  int version() const { return version_; }
  int64_t alignment() const { return alignment_; }
  const std::map<std::string, Value>& metadata() const { return metadata_; }
  const std::map<std::string, StoredTensor>& tensors() const { return tensors_; }
  const std::map<std::string, std::string>& unsupported() const { return unsupported_; }

  // GgufFile's typed getters (Gguf.scala:37-82)
  int64_t longValue(const std::string& key) const;
  double doubleValue(const std::string& key) const;
  std::string stringValue(const std::string& key) const;
  bool booleanValue(const std::string& key) const;
  std::vector<std::string> strings(const std::string& key) const;
  std::string architecture() const { return stringValue("general.architecture"); }

  // TensorSource.apply (StoredTensor.scala:46-54): std::out_of_range when absent
  const StoredTensor& operator[](const std::string& name) const;
  // a tensor's bytes, a view of the mapping
  const uint8_t* bytes(const std::string& name) const;
  // a 2-D tensor ([rows, cols]) as a table in device memory, its bytes copied
  // as they lie in the file
  DeviceTable table(const std::string& name) const;

 private:
  File() = default;
  friend class Reader;
  std::string source_;
  int version_ = 0;
  int64_t alignment_ = 32;
  std::map<std::string, Value> metadata_;
  std::map<std::string, StoredTensor> tensors_;
  std::map<std::string, std::string> unsupported_;
  const uint8_t* data_ = nullptr;
  size_t size_ = 0;
};

}  // namespace drift::gguf
